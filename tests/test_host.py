"""Host-side logic, no GPU: layout bytes, C-ABI symbol table and argument
rejection, Python validation, and that nothing silently falls back to CPU."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from wkvm_amd import _lib, ops, synthetic
from wkvm_amd.layout import ModelStateSpec, RWKV7StateLayout, StateFamilySpec
from wkvm_amd.runner import WKV7Runner


# -- layout (wkvm/models/rwkv7.py:41-99) ---------------------------------------------------

@pytest.mark.parametrize("name,wkv_bytes,shift_bytes", [
    ("0.1B", 12 * 12 * 64 * 64 * 4, 12 * 2 * 768 * 2),
    ("1.5B", 12_582_912, 196_608),          # 12.19 MiB per slot (m2_engine_bench.md:9)
    ("7B", 33_554_432, 524_288),
])
def test_layout_bytes(name, wkv_bytes, shift_bytes):
    lay = RWKV7StateLayout.for_shape(name)
    spec = lay.state_spec()
    fam = {f.name: f for f in spec.families}
    assert fam["wkv"].bytes_per_slot == wkv_bytes
    assert fam["shift"].bytes_per_slot == shift_bytes
    assert spec.bytes_per_request == wkv_bytes + shift_bytes
    assert fam["wkv"].layer_ids == tuple(range(lay.n_layer))
    assert lay.wkv_shape == (lay.num_heads, 64, 64)
    assert lay.shift_shape == (lay.hidden_size,)


def test_layout_from_config_mirrors_reference():
    class Cfg:
        num_hidden_layers = 12
        hidden_size = 768
        num_heads = 12
        head_dim = 64
        value_dim = [768] * 12
        attn = None

    lay = RWKV7StateLayout.from_config(Cfg, dtype=torch.bfloat16)
    assert lay == RWKV7StateLayout.for_shape("0.1B")
    Cfg.value_dim = [768, 512]
    with pytest.raises(NotImplementedError):
        RWKV7StateLayout.from_config(Cfg, dtype=torch.bfloat16)


def test_spec_validation():
    with pytest.raises(ValueError):
        StateFamilySpec(name="wkv", bytes_per_slot=0)
    f = StateFamilySpec(name="wkv", bytes_per_slot=4)
    with pytest.raises(ValueError):
        ModelStateSpec(families=(f, f))


# -- C ABI ---------------------------------------------------------------------------------

def test_header_declares_exactly_the_bound_symbols():
    declared = set(_lib.header_symbols())
    assert declared == set(_lib.SIGNATURES), declared ^ set(_lib.SIGNATURES)


def test_library_loads_and_exports_every_header_symbol():
    lib = _lib.load()
    for name in _lib.header_symbols():
        assert hasattr(lib, name), name
    assert lib.wkv7_abi_version() == _lib.WKV7_ABI_VERSION == 10


def test_a_library_of_another_abi_version_is_refused(monkeypatch):
    """A stale libwkv7.so (built from other sources) would be called with the
    wrong argument lists; load() compares its version with the binding's and
    raises with a rebuild hint instead."""
    _lib.load()
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "WKV7_ABI_VERSION", _lib.WKV7_ABI_VERSION - 1)
    with pytest.raises(RuntimeError, match="rebuild"):
        _lib.load()


def test_abi_rejects_bad_arguments_before_any_launch():
    """Every rejection returns before touching the GPU, so it runs on CPU."""
    lib = _lib.load()
    dummy = ctypes.c_void_p(16)
    six = [dummy] * 6
    # decode: negative B, bad y dtype, null pool
    assert lib.wkv7_decode_slots(dummy, 5, 2, dummy, None, -1, *six, dummy, 0, 1.0, None) == _lib.WKV7_ERR_ARG
    assert lib.wkv7_decode_slots(dummy, 5, 2, dummy, None, 1, *six, dummy, 7, 1.0, None) == _lib.WKV7_ERR_ARG
    assert lib.wkv7_decode_slots(None, 5, 2, dummy, None, 1, *six, dummy, 0, 1.0, None) == _lib.WKV7_ERR_ARG
    assert lib.wkv7_decode_slots(dummy, 5, 0, dummy, None, 1, *six, dummy, 0, 1.0, None) == _lib.WKV7_ERR_ARG
    assert lib.wkv7_decode_slots(dummy, 5, 2, dummy, None, 0, *six, dummy, 0, 1.0, None) == _lib.WKV7_OK
    # out-of-place decode: ids without their tensor, too few rows without ids,
    # bad y dtype; zero state in and no state out is a valid launch shape
    assert lib.wkv7_decode_into(None, 0, dummy, dummy, 4, None, 2, None, 1, *six, dummy, 0, 1.0,
                                None) == _lib.WKV7_ERR_ARG
    assert lib.wkv7_decode_into(dummy, 4, None, None, 0, dummy, 2, None, 1, *six, dummy, 0, 1.0,
                                None) == _lib.WKV7_ERR_ARG
    assert lib.wkv7_decode_into(dummy, 2, None, dummy, 4, None, 2, None, 3, *six, dummy, 0, 1.0,
                                None) == _lib.WKV7_ERR_SHAPE
    assert lib.wkv7_decode_into(None, 0, None, dummy, 2, None, 2, None, 3, *six, dummy, 0, 1.0,
                                None) == _lib.WKV7_ERR_SHAPE
    assert lib.wkv7_decode_into(None, 0, None, None, 0, None, 2, None, 3, *six, dummy, 9, 1.0,
                                None) == _lib.WKV7_ERR_ARG
    assert lib.wkv7_decode_into(None, 0, None, None, 0, None, 2, None, 0, *six, dummy, 0, 1.0,
                                None) == _lib.WKV7_OK
    # prefill: negative sizes, missing cu_seqlens
    assert lib.wkv7_prefill_varlen(dummy, 5, 2, dummy, dummy, None, -1, 0, *six, dummy, 0, 0,
                                   1.0, None) == _lib.WKV7_ERR_ARG
    assert lib.wkv7_prefill_varlen(dummy, 5, 2, dummy, None, None, 1, 4, *six, dummy, 0, 0,
                                   1.0, None) == _lib.WKV7_ERR_ARG
    # slot copy: negative count, null src, row wider than the slot stride
    assert lib.wkv7_slot_copy(dummy, 0, 64, 4, None, dummy, 0, 64, 4, None, 1, 64, -1,
                              None) == _lib.WKV7_ERR_ARG
    assert lib.wkv7_slot_copy(dummy, 0, 64, 4, None, None, 0, 64, 4, None, 1, 64, 1,
                              None) == _lib.WKV7_ERR_ARG
    assert lib.wkv7_slot_copy(dummy, 0, 64, 4, None, dummy, 0, 32, 4, None, 1, 64, 1,
                              None) == _lib.WKV7_ERR_SHAPE
    assert lib.wkv7_slot_zero(None, 0, 64, 4, dummy, 1, 64, 1, None) == _lib.WKV7_ERR_ARG
    # slot transfer: bad direction, slot out of range, null host, row wider than a stride
    assert lib.wkv7_slot_transfer(2, dummy, dummy, 256, 64, 4, 1, 2, 64, None, 0, None) == _lib.WKV7_ERR_ARG
    assert lib.wkv7_slot_transfer(0, dummy, dummy, 256, 64, 4, 4, 2, 64, None, 0, None) == _lib.WKV7_ERR_ARG
    assert lib.wkv7_slot_transfer(0, dummy, dummy, 256, 64, 4, -1, 2, 64, None, 0, None) == _lib.WKV7_ERR_ARG
    assert lib.wkv7_slot_transfer(1, None, dummy, 256, 64, 4, 1, 2, 64, None, 0, None) == _lib.WKV7_ERR_ARG
    assert lib.wkv7_slot_transfer(0, dummy, dummy, 256, 32, 4, 1, 2, 64, None, 0, None) == _lib.WKV7_ERR_SHAPE
    assert lib.wkv7_slot_transfer(0, dummy, dummy, 32, 64, 4, 1, 2, 64, None, 0, None) == _lib.WKV7_ERR_SHAPE
    assert lib.wkv7_slot_transfer(0, dummy, dummy, 256, 64, 4, 1, 0, 64, None, 0, None) == _lib.WKV7_OK
    # a staging buffer smaller than the slot's rows (2 x 64 B)
    assert lib.wkv7_slot_transfer(0, dummy, dummy, 256, 64, 4, 1, 2, 64, dummy, 127,
                                  None) == _lib.WKV7_ERR_WORKSPACE
    for code in (_lib.WKV7_ERR_ARG, _lib.WKV7_ERR_SHAPE, _lib.WKV7_ERR_WORKSPACE):
        assert _lib.strerror(code)


def test_abi_rejects_bad_projection_and_decode_block_arguments():
    """wkv7_proj_grouped and wkv7_decode_block validate everything before any
    device call (CPU-runnable), and zero rows is a successful no-op."""
    lib = _lib.load()
    G = _lib.ProjGroup

    def groups(**kw):
        base = dict(x=4096, w=8192, bias=None, y=12288, ldx=64, ldw=64, ldy=32, n=32, k=64,
                    act=_lib.WKV7_ACT_NONE, reserved=0)
        base.update(kw)
        arr = (G * 1)()
        arr[0] = G(**base)
        return arr

    ok = groups()
    assert lib.wkv7_proj_grouped(0, ok, 1, None, 0, None) == _lib.WKV7_OK
    assert lib.wkv7_proj_workspace_bytes(0, ok, 1) == 0  # no rows: nothing to split
    assert lib.wkv7_proj_workspace_bytes(4, groups(k=48), 1) == 0  # rejected: no workspace
    assert lib.wkv7_proj_grouped(-1, ok, 1, None, 0, None) == _lib.WKV7_ERR_ARG
    assert lib.wkv7_proj_grouped(4, ok, 0, None, 0, None) == _lib.WKV7_ERR_ARG
    assert lib.wkv7_proj_grouped(4, ok, _lib.WKV7_PROJ_MAX_GROUPS + 1, None, 0, None) == _lib.WKV7_ERR_ARG
    assert lib.wkv7_proj_grouped(4, None, 1, None, 0, None) == _lib.WKV7_ERR_ARG
    for bad in (dict(k=48), dict(k=0), dict(n=0), dict(act=3), dict(x=None), dict(w=None),
                dict(y=None)):
        assert lib.wkv7_proj_grouped(4, groups(**bad), 1, None, 0, None) == _lib.WKV7_ERR_ARG, bad
    for bad in (dict(ldx=32), dict(ldw=68), dict(ldy=16), dict(x=4100), dict(w=8200)):
        assert lib.wkv7_proj_grouped(4, groups(**bad), 1, None, 0, None) == _lib.WKV7_ERR_SHAPE, bad

    d = ctypes.c_void_p(4096)

    def block(B=1, H=2, eps=64e-5, r=d, v_lora=None, v_first=None, out=d, v_out=None):
        return lib.wkv7_decode_block(d, 5, H, d, None, B, r, d, d, d, d, v_lora, v_first, d, d,
                                     d, d, d, d, eps, 1.0, out, v_out, None)

    assert block(B=0) == _lib.WKV7_OK
    assert block(B=-1) == _lib.WKV7_ERR_ARG
    assert block(H=0) == _lib.WKV7_ERR_ARG
    assert block(eps=-1.0) == _lib.WKV7_ERR_ARG
    assert block(eps=float("nan")) == _lib.WKV7_ERR_ARG
    assert block(r=None) == _lib.WKV7_ERR_ARG
    assert block(out=None) == _lib.WKV7_ERR_ARG
    assert block(v_lora=d) == _lib.WKV7_ERR_ARG  # v_lora without v_first
    assert block(r=ctypes.c_void_p(4100)) == _lib.WKV7_ERR_SHAPE
    assert block(v_lora=d, v_first=ctypes.c_void_p(4098)) == _lib.WKV7_ERR_SHAPE
    assert block(v_out=ctypes.c_void_p(4097)) == _lib.WKV7_ERR_SHAPE


def test_check_maps_codes_to_exceptions():
    with pytest.raises(ValueError):
        _lib.check(_lib.WKV7_ERR_ARG, "x")
    _lib.check(_lib.WKV7_OK, "x")


# -- Python validation / no CPU fallback ------------------------------------------------------

def _vecs(B, H):
    g = synthetic.make_generator(0)
    return synthetic.order(synthetic.wkv7_vectors((B, H, 64), g))


def test_ops_refuse_cpu_tensors():
    pool = torch.zeros((4, 2, 64, 64))
    with pytest.raises(ValueError, match="GPU"):
        ops.wkv7_decode_slots(pool, [1, 2], *_vecs(2, 2))
    with pytest.raises(ValueError, match="GPU"):
        ops.wkv7_prefill_varlen(pool, [1], [0, 2], *_vecs(2, 2))
    with pytest.raises(ValueError, match="GPU"):
        ops.slot_copy(pool, [1], pool, [2], slot_dim=0)
    with pytest.raises(ValueError, match="GPU"):
        ops.chunk_rwkv7(*(x[None] for x in _vecs(3, 2)))


def test_host_id_validation():
    assert ops.host_ids([3, 1], 4, "ids", distinct=True) == [3, 1]
    with pytest.raises(ValueError, match="out of range"):
        ops.host_ids([4], 4, "ids", distinct=True)
    with pytest.raises(ValueError, match="out of range"):
        ops.host_ids([-1], 4, "ids", distinct=True)
    with pytest.raises(ValueError, match="duplicate"):
        ops.host_ids([2, 2], 4, "ids", distinct=True)
    assert ops.host_ids(np.array([2, 2]), 4, "ids", distinct=False) == [2, 2]
    assert ops.host_ids(torch.tensor([0, 3]), 4, "ids", distinct=True) == [0, 3]


def test_host_cu_validation():
    assert ops._host_cu([0, 3, 3, 7], 7) == [0, 3, 3, 7]
    for bad in ([1, 7], [0, 5], [0, 4, 3, 7], []):
        with pytest.raises(ValueError):
            ops._host_cu(bad, 7)


def test_longest_first_order():
    # lengths 3, 0, 9, 3, 5: longest first, equal lengths in index order
    assert ops.longest_first([0, 3, 3, 12, 15, 20]) == [2, 4, 0, 3, 1]
    assert ops.longest_first([0]) == []


def test_slot_view_describes_bank_tensors():
    L, S, H, D = 3, 5, 2, 6
    wkv = torch.zeros((L, S + 1, H, 64, 64))
    assert ops.slot_view(wkv, 1) == (L, (S + 1) * H * 4096 * 4, H * 4096 * 4, S + 1, H * 4096 * 4)
    shift = torch.zeros((L, 2, S + 1, D), dtype=torch.bfloat16)
    assert ops.slot_view(shift, 2) == (2 * L, (S + 1) * D * 2, D * 2, S + 1, D * 2)
    assert ops.slot_view(wkv[1], 0) == (1, 0, H * 4096 * 4, S + 1, H * 4096 * 4)
    with pytest.raises(ValueError):
        ops.slot_view(wkv.transpose(3, 4), 1)
    with pytest.raises(ValueError):
        ops.slot_view(shift.transpose(0, 1), 2)


def test_runner_argument_errors():
    class FakeBank:
        class layout:
            n_layer = 2
        device = torch.device("cpu")
        num_slots = 4

    with pytest.raises(ValueError):
        WKV7Runner(FakeBank(), prefill_chunk=0)
    for bad in (0, "four", 2.0):
        with pytest.raises(ValueError, match="prefill_segments"):
            WKV7Runner(FakeBank(), prefill_segments=bad)
    WKV7Runner(FakeBank(), prefill_segments="auto")
    run = WKV7Runner(FakeBank(), prefill_chunk=64)
    empty = tuple(torch.zeros((0, 2, 64), dtype=torch.bfloat16) for _ in range(6))
    with pytest.raises(ValueError, match="empty prompt"):
        run.prefill([empty, empty], {"wkv": 1, "shift": 1})
    with pytest.raises(ValueError, match="layers"):
        run.prefill([empty], {"wkv": 1, "shift": 1})
    one = _vecs(1, 2)
    with pytest.raises(ValueError, match="mismatch"):
        run.decode_step([{"wkv": 1, "shift": 1}, {"wkv": 2, "shift": 2}], [one, one])


# -- synthetic inputs ---------------------------------------------------------------------------

def test_synthetic_distributions_and_determinism():
    g1, g2 = synthetic.make_generator(7), synthetic.make_generator(7)
    a1 = synthetic.wkv7_vectors((32, 4, 64), g1)
    a2 = synthetic.wkv7_vectors((32, 4, 64), g2)
    for n in "rwkvab":
        assert a1[n].dtype == torch.bfloat16
        assert torch.equal(a1[n], a2[n])
    decay = torch.exp(a1["w"].float())
    assert decay.min() > 0.544 and decay.max() < 1.0
    kn = -a1["a"].float()
    assert torch.allclose(kn.norm(dim=-1), torch.ones(32, 4), atol=1e-2)
    ratio = a1["b"].float() / kn
    assert ratio.min() > -1e-3 and ratio.max() < 1.0 + 1e-2
    ids = synthetic.active_slots(16, 4, synthetic.make_generator(3))
    assert len(set(ids)) == 4 and min(ids) >= 1 and max(ids) <= 16
    lens = synthetic.ragged_lengths(64, 1, 2048, synthetic.make_generator(4))
    assert min(lens) >= 1 and max(lens) <= 2048


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    """No CPU or eager fallback: without the built library every op raises."""
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "libwkv7.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="not built"):
        _lib.load()


def test_segment_entry_points_reject_bad_arguments():
    lib = _lib.load()
    buf = (ctypes.c_uint8 * 4096)()
    p = ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 16
    E_ARG, E_SHAPE = _lib.WKV7_ERR_ARG, _lib.WKV7_ERR_SHAPE
    # runs: n_primary beyond nseq, secondary runs without ranges, misaligned inputs
    assert lib.wkv7_prefill_runs(p, 4, 2, p, p, None, 2, 8, *[p] * 6, p, 0, 0, 1.0, None, None,
                                 3, None, 0, None, None, 0, None, None) == E_ARG
    assert lib.wkv7_prefill_runs(p, 4, 2, p, p, None, 2, 8, *[p] * 6, p, 0, 0, 1.0, p, None,
                                 1, p, 2, None, None, 0, None, None) == E_ARG
    assert lib.wkv7_prefill_runs(p, 4, 2, p, p, None, 2, 8, p + 2, *[p] * 5, p, 0, 0, 1.0,
                                 None, None, 2, None, 0, None, None, 0, None, None) == E_SHAPE
    assert lib.wkv7_prefill_runs(p, 4, 2, p, p, None, 0, 8, *[p] * 6, p, 0, 0, 1.0, None, None,
                                 0, None, 0, None, None, 0, None, None) == 0
    # y and y_alt are stored as whole-row vectors: 8-byte (bf16) / 16-byte (fp32) aligned
    assert lib.wkv7_prefill_runs(p, 4, 2, p, p, None, 2, 8, *[p] * 6, p + 4, 0, 0, 1.0, None,
                                 None, 2, None, 0, None, None, 0, None, None) == E_SHAPE
    assert lib.wkv7_prefill_runs(p, 4, 2, p, p, None, 2, 8, *[p] * 6, p + 8, 1, 0, 1.0, None,
                                 None, 2, None, 0, None, None, 0, None, None) == E_SHAPE
    assert lib.wkv7_prefill_runs(p, 4, 2, p, p, None, 2, 8, *[p] * 6, p, 0, 0, 1.0, None,
                                 None, 2, None, 0, p + 2, None, 0, None, None) == E_SHAPE
    # runs reading initial states from state_in: ids without the tensor, too few rows
    assert lib.wkv7_prefill_runs(p, 4, 2, p, p, None, 2, 8, *[p] * 6, p, 0, 0, 1.0, None, None,
                                 2, None, 0, None, None, 0, p, None) == E_ARG
    assert lib.wkv7_prefill_runs(p, 4, 2, p, p, None, 2, 8, *[p] * 6, p, 0, 0, 1.0, None, None,
                                 2, None, 0, None, p, 1, None, None) == E_SHAPE
    # out-of-place prefill: ids without their tensor, too few rows without ids,
    # bad y dtype, misaligned y; zero state in and no state out is a valid shape
    assert lib.wkv7_prefill_into(None, 0, p, p, 4, None, 2, p, None, 2, 8, *[p] * 6, p, 0, 1.0,
                                 None) == E_ARG
    assert lib.wkv7_prefill_into(p, 4, None, None, 0, p, 2, p, None, 2, 8, *[p] * 6, p, 0, 1.0,
                                 None) == E_ARG
    assert lib.wkv7_prefill_into(p, 1, None, p, 4, None, 2, p, None, 2, 8, *[p] * 6, p, 0, 1.0,
                                 None) == E_SHAPE
    assert lib.wkv7_prefill_into(None, 0, None, p, 1, None, 2, p, None, 2, 8, *[p] * 6, p, 0,
                                 1.0, None) == E_SHAPE
    assert lib.wkv7_prefill_into(None, 0, None, None, 0, None, 2, p, None, 2, 8, *[p] * 6, p, 4,
                                 1.0, None) == E_ARG
    assert lib.wkv7_prefill_into(None, 0, None, None, 0, None, 2, None, None, 2, 8, *[p] * 6, p,
                                 0, 1.0, None) == E_ARG
    assert lib.wkv7_prefill_into(None, 0, None, None, 0, None, 2, p, None, 2, 8, *[p] * 6, p + 4,
                                 0, 1.0, None) == E_SHAPE
    assert lib.wkv7_prefill_into(None, 0, None, None, 0, None, 2, p, None, 0, 8, *[p] * 6, p, 0,
                                 1.0, None) == 0
    assert lib.wkv7_prefill_varlen(p, 4, 2, p, p, None, 2, 8, *[p] * 6, p + 2, 0, 0, 1.0,
                                   None) == E_SHAPE
    assert lib.wkv7_prefill_varlen(p, 4, 2, p, p, None, 2, 8, *[p] * 6, p + 8, 1, 0, 1.0,
                                   None) == E_SHAPE
    # chain: segments without their tables; misaligned hin
    assert lib.wkv7_segment_chain(p, 4, 2, None, 0, p, 1, None, 1, p, None) == E_ARG
    assert lib.wkv7_segment_chain(p, 4, 2, p, 2, p, 1, p, 1, p + 4, None) == E_SHAPE
    # correct: bad dtype, missing q with segments, misaligned fp32 y
    assert lib.wkv7_segment_correct(8, 2, p, p, p, 1, p, 0, p, 5, None) == E_ARG
    assert lib.wkv7_segment_correct(8, 2, p, None, p, 1, p, 1, p, 0, None) == E_ARG
    assert lib.wkv7_segment_correct(8, 2, p, p, p, 1, p, 1, p + 8, 1, None) == E_SHAPE
