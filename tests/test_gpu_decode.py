"""Decode-step parity: wkv7_decode_slots (HIP, through the C ABI) against the
float64 oracle on the same seeded inputs.

Bars (north star): the fp32 state matches to max relative error 1e-5 per step,
measured normwise per (slot, head) 64x64 tile as max|d| / max|ref|; y in fp32
matches to the same bar per (slot, head) vector; a bf16 y is within that bar
plus one bf16 ulp of the float64 result (its own rounding). Rows not in the
batch, including pad slot 0, stay bit-identical."""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import oracle as O
from tests import util as U
from tests.golden import make_golden as G
from wkvm_amd import ops, synthetic
from wkvm_amd.layout import RWKV7StateLayout
from wkvm_amd.runner import WKV7Runner
from wkvm_amd.state import RWKV7StateBank

pytestmark = pytest.mark.gpu

STATE_TOL = 1e-5
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "wkv7_golden.npz")


def _check_step(pool_before: np.ndarray, ids, vec_bits, pool_after: torch.Tensor, y: torch.Tensor,
                scale: float = 1.0):
    y_ref, h_ref = O.scan_bf16(np.arange(len(ids) + 1), *vec_bits, pool=pool_before,
                               slot_ids=ids, scale=scale)
    h = U.f64(pool_after[ids])
    err = U.normwise_max(h, h_ref)
    assert err <= STATE_TOL, f"state normwise error {err:.3e}"
    if y.dtype == torch.float32:
        yerr = U.normwise_max(U.f64(y), y_ref, tile_dims=1)
        assert yerr <= STATE_TOL, f"y normwise error {yerr:.3e}"
    else:
        excess = U.bf16_y_excess(U.bits(y), y_ref)
        assert excess <= 1, f"bf16 y at {excess:.2f} x its bar"
    return err


@pytest.mark.parametrize("y_dtype", [torch.bfloat16, torch.float32])
def test_cfg0_decode_matches_oracle_and_golden(dev, y_dtype):
    pool, ids, vecs = G.cfg0_inputs()
    gpool = pool.to(dev)
    xs = [vecs[n].to(dev) for n in "rwkvab"]
    y = ops.wkv7_decode_slots(gpool, ids, *xs, out_dtype=y_dtype)
    torch.cuda.synchronize()
    _check_step(pool.numpy(), ids, U.vec_bits(vecs), gpool, y)
    others = [i for i in range(pool.shape[0]) if i not in ids]
    assert torch.equal(gpool[others].cpu(), pool[others]), "rows outside the batch changed"
    g = np.load(GOLDEN)
    if y_dtype == torch.float32:
        assert U.normwise_max(U.f64(y), g["cfg0_y"], tile_dims=1) <= STATE_TOL
    h = U.f64(gpool[ids])
    assert U.normwise_max(h @ G.projection_vector(), g["cfg0_state_proj"], 1) <= 1e-4
    assert U.normwise_max(h[0, 0], g["cfg0_state_block"]) <= STATE_TOL


def test_cfg1_full_layer_multi_step(dev):
    """1.5B shape (H=32), 256 active slots scattered in a 512-slot pool, three
    consecutive steps; each step is checked against the oracle run from the
    GPU's own previous state (per-step bar), and the 3-step drift against an
    oracle chain is reported."""
    H, S, B = 32, 512, 256
    gen = synthetic.make_generator(101)
    pool = torch.zeros((S + 1, H, 64, 64))
    pool[1:] = synthetic.initial_states((S, H, 64, 64), gen)
    ids = synthetic.active_slots(S, B, gen)
    gpool = pool.to(dev)
    chain = pool.numpy().astype(np.float64)
    for step in range(3):
        vecs = synthetic.wkv7_vectors((B, H, 64), gen)
        before = gpool.cpu().numpy()
        y = ops.wkv7_decode_slots(gpool, ids, *(vecs[n].to(dev) for n in "rwkvab"),
                                  out_dtype=torch.float32)
        torch.cuda.synchronize()
        err = _check_step(before, ids, U.vec_bits(vecs), gpool, y)
        _, chain_h = O.scan_f64(np.arange(B + 1), *(O.bf16_bits_to_f64(b) for b in U.vec_bits(vecs)),
                                h0=chain[ids])
        chain[ids] = chain_h
        print(f"step {step}: per-step normwise {err:.2e}, "
              f"drift vs f64 chain {U.normwise_max(U.f64(gpool[ids]), chain[ids]):.2e}")
    untouched = [i for i in range(S + 1) if i not in set(ids)]
    assert torch.equal(gpool[untouched].cpu(), pool[untouched])


def test_delta_rule_orientation_on_gpu(dev):
    """CF3 through the kernel: decay 1, a = -k^, b = k^ (bf16), k = k^:
    S_1 k^ = (1 - k^.k^) S_0 k^ + (k^.k^) v in exact arithmetic with the bf16
    vectors; a transposed kernel misses this for a non-symmetric S_0."""
    H = 8
    g = torch.Generator().manual_seed(12)
    kh = torch.nn.functional.normalize(torch.randn((1, H, 64), generator=g), dim=-1).bfloat16()
    v = torch.randn((1, H, 64), generator=g).bfloat16()
    r = torch.randn((1, H, 64), generator=g).bfloat16()
    zero = torch.zeros((1, H, 64), dtype=torch.bfloat16)
    pool = torch.randn((2, H, 64, 64), generator=g)
    gpool = pool.to(dev)
    ops.wkv7_decode_slots(gpool, [1], *(x.to(dev) for x in (r, zero, kh, v, -kh, kh)))
    k64 = kh.double().numpy()[0]
    kk = np.sum(k64 * k64, -1)[:, None]
    S0k = np.einsum("hji,hj->hi", pool.double().numpy()[1], k64)
    S1k = np.einsum("hji,hj->hi", U.f64(gpool[1]), k64)
    expect = (1 - kk) * S0k + kk * v.double().numpy()[0]
    assert np.max(np.abs(S1k - expect)) <= 1e-4 * np.max(np.abs(expect))


def test_permutation_equivariance_and_scale(dev):
    """CF7: the same rows in another batch order give identical bits; scale
    multiplies r, so y(scale=0.5) == 0.5 * y(scale=1) exactly in fp32."""
    H, S = 4, 12
    gen = synthetic.make_generator(13)
    base = synthetic.initial_states((S + 1, H, 64, 64), gen).to(dev)
    ids = [3, 9, 1, 12, 6]
    vecs = synthetic.wkv7_vectors((5, H, 64), gen, device=dev)
    perm = [2, 0, 4, 1, 3]
    p1, p2, p3 = base.clone(), base.clone(), base.clone()
    y1 = ops.wkv7_decode_slots(p1, ids, *synthetic.order(vecs), out_dtype=torch.float32)
    y2 = ops.wkv7_decode_slots(p2, [ids[i] for i in perm],
                               *(vecs[n][perm] for n in "rwkvab"), out_dtype=torch.float32)
    assert torch.equal(p1, p2)
    assert torch.equal(y1[perm], y2)
    y3 = ops.wkv7_decode_slots(p3, ids, *synthetic.order(vecs), scale=0.5, out_dtype=torch.float32)
    assert torch.equal(p3, p1)
    assert torch.equal(y3, y1 * 0.5)


def test_decode_argument_errors(dev):
    pool = torch.zeros((5, 2, 64, 64), device=dev)
    vecs = synthetic.order(synthetic.wkv7_vectors((2, 2, 64), synthetic.make_generator(0),
                                                  device=dev))
    with pytest.raises(ValueError, match="duplicate"):
        ops.wkv7_decode_slots(pool, [1, 1], *vecs)
    with pytest.raises(ValueError, match="out of range"):
        ops.wkv7_decode_slots(pool, [1, 5], *vecs)
    with pytest.raises(ValueError, match="bfloat16"):
        ops.wkv7_decode_slots(pool, [1, 2], *(x.float() for x in vecs))
    with pytest.raises(ValueError):
        ops.wkv7_decode_slots(pool, [1, 2, 3], *vecs)
    with pytest.raises(ValueError):
        ops.wkv7_decode_slots(pool.double(), [1, 2], *vecs)
    y = ops.wkv7_decode_slots(pool, [], *(x[:0] for x in vecs))
    assert y.shape == (0, 2, 64)


def test_runner_decode_step_all_layers(dev):
    """WKV7Runner.decode_step over a 4-layer bank equals per-layer oracle steps;
    the pad slot and idle slots stay untouched."""
    lay = RWKV7StateLayout(n_layer=4, hidden_size=384, num_heads=6, head_dim=64, head_v_dim=64,
                           dtype=torch.bfloat16)
    bank = RWKV7StateBank(lay, num_slots=10, device=dev)
    gen = synthetic.make_generator(21)
    bank.wkv[:, 1:] = synthetic.initial_states((4, 10, 6, 64, 64), gen).to(dev)
    before = bank.wkv.cpu().numpy()
    batch = [{"wkv": s, "shift": s} for s in (4, 2, 9)]
    layer_vecs = [synthetic.wkv7_vectors((3, 6, 64), gen) for _ in range(4)]
    run = WKV7Runner(bank)
    ys = run.decode_step(batch, [[v[n].to(dev) for n in "rwkvab"] for v in layer_vecs],
                         out_dtype=torch.float32)
    torch.cuda.synchronize()
    for layer in range(4):
        _check_step(before[layer], [4, 2, 9], U.vec_bits(layer_vecs[layer]), bank.wkv[layer],
                    ys[layer])
    idle = [0, 1, 3, 5, 6, 7, 8, 10]
    assert np.array_equal(bank.wkv[:, idle].cpu().numpy(), before[:, idle])


def test_row_order_changes_visiting_order_only(dev):
    """The slot-sorted visiting order (computed for host ids) and any other
    permutation passed as row_order give bit-identical states and outputs."""
    H, S = 8, 40
    gen = synthetic.make_generator(77)
    base = synthetic.initial_states((S + 1, H, 64, 64), gen).to(dev)
    ids = synthetic.active_slots(S, 17, gen)
    vecs = synthetic.order(synthetic.wkv7_vectors((17, H, 64), gen, device=dev))
    ids_t = torch.tensor(ids, dtype=torch.int32, device=dev)
    outs = []
    for order in (None, list(range(17)), list(range(16, -1, -1))):
        p = base.clone()
        ro = None if order is None else torch.tensor(order, dtype=torch.int32, device=dev)
        src = ids if order is None else ids_t
        y = ops.wkv7_decode_slots(p, src, *vecs, out_dtype=torch.float32, row_order=ro)
        outs.append((p, y))
    for p, y in outs[1:]:
        assert torch.equal(p, outs[0][0]) and torch.equal(y, outs[0][1])
    with pytest.raises(ValueError):
        ops.wkv7_decode_slots(base.clone(), ids_t, *vecs,
                              row_order=torch.arange(16, dtype=torch.int32, device=dev))


def test_7b_shape_decode_matches_oracle(dev):
    """7B head count (H = 64, config 3's shape): 48 slots scattered in a
    160-slot pool, bf16 and fp32 y, two steps against the oracle."""
    H, S, B = 64, 160, 48
    gen = synthetic.make_generator(171)
    pool = torch.zeros((S + 1, H, 64, 64))
    pool[1:] = synthetic.initial_states((S, H, 64, 64), gen)
    ids = synthetic.active_slots(S, B, gen)
    gpool = pool.to(dev)
    for y_dtype in (torch.bfloat16, torch.float32):
        vecs = synthetic.wkv7_vectors((B, H, 64), gen)
        before = gpool.cpu().numpy()
        y = ops.wkv7_decode_slots(gpool, ids, *(vecs[n].to(dev) for n in "rwkvab"),
                                  out_dtype=y_dtype)
        torch.cuda.synchronize()
        _check_step(before, ids, U.vec_bits(vecs), gpool, y)
    untouched = [i for i in range(S + 1) if i not in set(ids)]
    assert torch.equal(gpool[untouched].cpu(), pool[untouched])


def test_fla_recurrent_decode_cfg1_shape(dev):
    """fused_recurrent_rwkv7 at T = 1 (the reference model layer's decode
    call, wkvm/models/rwkv7.py:108-111) at config-1 shape (B = 256, H = 32):
    it runs the decode kernel out of place -- initial_state read, a new
    final_state written, the caller's tensor untouched -- and matches the
    oracle; initial_state=None is the zero state; output_final_state=False
    gives the same o; the packed form (cu_seqlens as fla's device int64
    tensor) and head_first give the same bits."""
    B, H = 256, 32
    gen = synthetic.make_generator(301)
    vecs = synthetic.wkv7_vectors((B, 1, H, 64), gen)
    h0 = synthetic.initial_states((B, H, 64, 64), gen)
    xs = [vecs[n].to(dev) for n in "rwkvab"]
    h0d = h0.to(dev)
    o, hT = ops.fused_recurrent_rwkv7(*xs, initial_state=h0d, output_final_state=True)
    torch.cuda.synchronize()
    assert o.shape == (B, 1, H, 64) and o.dtype == torch.bfloat16
    assert hT.shape == (B, H, 64, 64) and hT.data_ptr() != h0d.data_ptr()
    assert torch.equal(h0d.cpu(), h0)
    flat = [U.bits(vecs[n][:, 0]) for n in "rwkvab"]
    y_ref, h_ref = O.scan_bf16(np.arange(B + 1), *flat, pool=h0.numpy(), slot_ids=list(range(B)))
    assert U.normwise_max(U.f64(hT), h_ref) <= STATE_TOL
    assert U.bf16_y_excess(U.bits(o[:, 0]), y_ref) <= 1
    o_nf, none = ops.fused_recurrent_rwkv7(*xs, initial_state=h0d, output_final_state=False)
    assert none is None and torch.equal(o_nf, o)
    cu = torch.arange(B + 1, dtype=torch.int64, device=dev)
    o_p, h_p = ops.fused_recurrent_rwkv7(*(x.transpose(0, 1) for x in xs), initial_state=h0d,
                                         cu_seqlens=cu)
    assert torch.equal(o_p[0], o[:, 0]) and torch.equal(h_p, hT)
    o_hf, h_hf = ops.fused_recurrent_rwkv7(*(x.transpose(1, 2) for x in xs), initial_state=h0d,
                                           head_first=True)
    assert torch.equal(o_hf.transpose(1, 2), o) and torch.equal(h_hf, hT)
    o0, h00 = ops.fused_recurrent_rwkv7(*xs)
    y0, hz = O.scan_bf16(np.arange(B + 1), *flat)
    assert U.normwise_max(U.f64(h00), hz) <= STATE_TOL
    assert U.bf16_y_excess(U.bits(o0[:, 0]), y0) <= 1


def test_fla_recurrent_short_packed_sequences(dev):
    """fused_recurrent_rwkv7 over packed sequences of 1-40 tokens with fla's
    device int64 cu_seqlens (the chunked scan on a copy of initial_state)."""
    H = 8
    lens = [1, 40, 7, 1, 23]
    cu = np.concatenate([[0], np.cumsum(lens)])
    gen = synthetic.make_generator(303)
    vecs = synthetic.wkv7_vectors((1, int(cu[-1]), H, 64), gen)
    h0 = synthetic.initial_states((len(lens), H, 64, 64), gen)
    h0d = h0.to(dev)
    o, hT = ops.fused_recurrent_rwkv7(*(vecs[n].to(dev) for n in "rwkvab"), initial_state=h0d,
                                      cu_seqlens=torch.tensor(cu, device=dev))
    torch.cuda.synchronize()
    y_ref, h_ref = O.scan_bf16(cu, *(U.bits(vecs[n][0]) for n in "rwkvab"), pool=h0.numpy(),
                               slot_ids=list(range(len(lens))))
    assert U.rel_l2(U.f64(hT), h_ref) <= 1e-3
    assert U.rel_l2(U.f64(o[0]), O.round_f64_to_bf16(y_ref)) <= 1e-3
    assert torch.equal(h0d.cpu(), h0)


def test_decode_into_ids_zero_state_and_no_output_state(dev):
    """wkv7_decode_into with id lists on both sides (reading one pool, writing
    another), with no source (zero state) and with no destination: each
    against the oracle; rows of the destination outside out_ids untouched."""
    H, S, B = 4, 20, 6
    gen = synthetic.make_generator(305)
    src = synthetic.initial_states((S, H, 64, 64), gen)
    vecs = synthetic.wkv7_vectors((B, H, 64), gen)
    xs = [vecs[n].to(dev) for n in "rwkvab"]
    in_ids = [3, 17, 0, 9, 12, 3]      # a source row may be read twice
    out_ids = [5, 1, 14, 2, 19, 7]
    gsrc = src.to(dev)
    dst = torch.full((S, H, 64, 64), 2.5, device=dev)
    y = ops.wkv7_decode_into(gsrc, dst, *xs, in_ids=in_ids, out_ids=out_ids,
                             out_dtype=torch.float32)
    torch.cuda.synchronize()
    y_ref, h_ref = O.scan_bf16(np.arange(B + 1), *U.vec_bits(vecs), pool=src.numpy(),
                               slot_ids=in_ids)
    assert U.normwise_max(U.f64(dst[out_ids]), h_ref) <= STATE_TOL
    assert U.normwise_max(U.f64(y), y_ref, tile_dims=1) <= STATE_TOL
    assert torch.equal(gsrc.cpu(), src)
    rest = [i for i in range(S) if i not in out_ids]
    assert bool((dst[rest] == 2.5).all())
    y_z = ops.wkv7_decode_into(None, dst, *xs, out_ids=out_ids, out_dtype=torch.float32)
    yz_ref, hz_ref = O.scan_bf16(np.arange(B + 1), *U.vec_bits(vecs))
    assert U.normwise_max(U.f64(dst[out_ids]), hz_ref) <= STATE_TOL
    assert U.normwise_max(U.f64(y_z), yz_ref, tile_dims=1) <= STATE_TOL
    y_n = ops.wkv7_decode_into(gsrc, None, *xs, in_ids=in_ids, out_dtype=torch.float32)
    assert torch.equal(y_n, y)
    with pytest.raises(ValueError, match="reads"):
        ops.wkv7_decode_into(gsrc, gsrc, *xs, in_ids=[1, 2, 3, 4, 5, 6],
                             out_ids=[2, 8, 9, 10, 11, 0])


def test_rejected_device_ids_read_out_zero(dev):
    """Device id tensors are not validated on the host. A row whose id the
    kernel's bounds check rejects touches no state and gets y = 0 (decode in
    place, out of place, and the fused time-mix decode alike)."""
    H, S, B = 2, 6, 3
    gen = synthetic.make_generator(307)
    pool = synthetic.initial_states((S + 1, H, 64, 64), gen).to(dev)
    before = pool.clone()
    vecs = synthetic.order(synthetic.wkv7_vectors((B, H, 64), gen, device=dev))
    bad = torch.tensor([2, S + 1, 4], dtype=torch.int32, device=dev)
    y = ops.wkv7_decode_slots(pool, bad, *vecs, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert not torch.any(y[1]) and torch.all(y[0] != 0)
    assert torch.equal(pool[[0, 1, 3, 5, 6]], before[[0, 1, 3, 5, 6]])
    ref = before.clone()
    y_ok = ops.wkv7_decode_slots(ref, [2, 4], *(x[[0, 2]] for x in vecs), out_dtype=torch.float32)
    assert torch.equal(y[[0, 2]], y_ok) and torch.equal(pool, ref)
    dst = torch.zeros_like(pool)
    y2 = ops.wkv7_decode_into(before, dst, *vecs, in_ids=torch.tensor([1, 2, -1], dtype=torch.int32,
                                                                       device=dev),
                              out_ids=torch.tensor([1, 2, 3], dtype=torch.int32, device=dev),
                              out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert not torch.any(y2[2]) and not torch.any(dst[3]) and torch.any(dst[1])
    D = H * 64
    rows = [torch.randn((B, D), generator=torch.Generator().manual_seed(i)).bfloat16().to(dev)
            for i in range(8)]
    par = [torch.rand(D, generator=torch.Generator().manual_seed(10 + i)).bfloat16().to(dev)
           for i in range(5)]
    blk_pool = before.clone()
    out, v_out = ops.wkv7_decode_block(blk_pool, bad, H, *rows[:6], *par, 64e-5,
                                       v_lora=rows[6], v_first=rows[7], want_v=True)
    torch.cuda.synchronize()
    assert not torch.any(out[1]) and not torch.any(v_out[1]) and torch.any(out[0])
    assert torch.equal(blk_pool[[0, 1, 3, 5, 6]], before[[0, 1, 3, 5, 6]])


def test_requests_in_one_batch_match_each_request_alone(dev):
    """State isolation as the reference checks it (two requests decoded as one
    batch give what each gives alone, tests/test_rwkv7_gpu.py:254-276), at the
    WKV level and bit for bit: two prompts (150 and 77 tokens) prefilled through
    WKV7Runner.prefill, then 12 decode steps with both rows in one batch, equal
    each request run alone on a fresh bank (every step's y and the final
    states); and a mixed step in which one request decodes while the other
    prefills equals the two calls made separately (the reference engine's
    decode / prefill split, engine.py:142-170)."""
    lay = RWKV7StateLayout(n_layer=3, hidden_size=256, num_heads=4, head_dim=64, head_v_dim=64,
                           dtype=torch.bfloat16)
    H, L, steps = 4, 3, 12
    gen = synthetic.make_generator(401)
    lens = [150, 77]
    prompts = [[synthetic.order(synthetic.wkv7_vectors((n, H, 64), gen)) for _ in range(L)]
               for n in lens]
    dec = [[[synthetic.order(synthetic.wkv7_vectors((1, H, 64), gen)) for _ in range(L)]
            for _ in range(steps)] for _ in lens]
    slots = [{"wkv": 2, "shift": 2}, {"wkv": 5, "shift": 5}]

    def on_dev(layer_inputs):
        return [[x.to(dev) for x in xs] for xs in layer_inputs]

    def run(reqs):
        bank = RWKV7StateBank(lay, num_slots=6, device=dev)
        runner = WKV7Runner(bank, prefill_chunk=64)
        for i in reqs:
            runner.prefill(on_dev(prompts[i]), slots[i], out_dtype=torch.float32)
        ys = []
        for s in range(steps):
            inputs = [[torch.cat([dec[i][s][layer][n] for i in reqs]).to(dev) for n in range(6)]
                      for layer in range(L)]
            ys.append(runner.decode_step([slots[i] for i in reqs], inputs,
                                         out_dtype=torch.float32))
        torch.cuda.synchronize()
        return bank.wkv.clone(), ys

    both, y_both = run([0, 1])
    for i in (0, 1):
        alone, y_alone = run([i])
        sl = slots[i]["wkv"]
        assert torch.equal(both[:, sl], alone[:, sl]), f"request {i}: final state"
        for s in range(steps):
            for layer in range(L):
                assert torch.equal(y_both[s][layer][i], y_alone[s][layer][0]), (i, s, layer)

    # request 0 decodes one token while request 1 prefills, in one mixed step
    bank = RWKV7StateBank(lay, num_slots=6, device=dev)
    runner = WKV7Runner(bank, prefill_chunk=64)
    runner.prefill(on_dev(prompts[0]), slots[0], out_dtype=torch.float32)
    sep = bank.wkv.clone()
    dec_y, pre_y = runner.mixed_step([slots[0]], on_dev(dec[0][0]), [slots[1]], [lens[1]],
                                     on_dev(prompts[1]), out_dtype=torch.float32)
    torch.cuda.synchronize()
    bank2 = RWKV7StateBank(lay, num_slots=6, device=dev)
    bank2.wkv.copy_(sep)
    runner2 = WKV7Runner(bank2, prefill_chunk=64)
    y_dec = runner2.decode_step([slots[0]], on_dev(dec[0][0]), out_dtype=torch.float32)
    y_pre = runner2.prefill(on_dev(prompts[1]), slots[1], out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(bank.wkv, bank2.wkv)
    for layer in range(L):
        assert torch.equal(dec_y[layer], y_dec[layer])
        assert torch.equal(pre_y[layer], y_pre[layer])


def test_cfg3_fork_then_decode_at_full_size(dev):
    """Config 3 at its own size, one layer: 7B heads (H = 64), 1153 slot rows,
    1024 live slots scattered over rows 1..1024. 128 seeded live slots are
    forked into the free rows 1025..1152 (bit-exact copies), then one decode
    step of all 1024 live slots is checked against the oracle (every live
    slot's state and its fp32 y); the forked children keep their sources'
    pre-step state and pad row 0 stays zero."""
    H, S, B = 64, 1152, 1024
    gen = synthetic.make_generator(331)
    pool = torch.zeros((S + 1, H, 64, 64))
    pool[1:B + 1] = synthetic.initial_states((B, H, 64, 64), gen)
    live = synthetic.active_slots(B, B, gen)
    src = [live[i] for i in torch.randperm(B, generator=gen)[:128].tolist()]
    dst = list(range(B + 1, S + 1))
    gpool = pool.to(dev)
    del pool
    ops.slot_copy(gpool, dst, gpool, src, slot_dim=0)
    torch.cuda.synchronize()
    before = gpool.cpu().numpy()
    assert np.array_equal(before[dst], before[src])
    vecs = synthetic.wkv7_vectors((B, H, 64), gen)
    y = ops.wkv7_decode_slots(gpool, live, *(vecs[n].to(dev) for n in "rwkvab"),
                              out_dtype=torch.float32)
    torch.cuda.synchronize()
    _check_step(before, live, U.vec_bits(vecs), gpool, y)
    assert torch.equal(gpool[dst].cpu(), torch.from_numpy(before[dst]))
    assert not torch.any(gpool[0])
