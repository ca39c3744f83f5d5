"""Time-mix stages on the GPU (HIP kernels through the C ABI) against the CPU
oracle (oracle/timemix.py), plus the composed RWKV-7 time-mix block.

Bars: ``token_shift_mix`` is bit-exact (outputs and the slot rows it writes;
rows outside the batch, pad row 0 included, untouched). ``time_mix_inputs``
and ``time_mix_output`` compute in fp32 with hardware exp / reciprocal, so a
bf16 output may land one bf16 ulp from the float64 value rounded to bf16:
inputs are held to <= 1 ulp (absolute 2^-8 |ref| at the rounding edge),
except the v lerp, which can cancel and is held to 2^-8 of its summands'
magnitude; the output to 2^-7 of its summands' magnitude (the GroupNorm and
the bonus term can cancel).

The composed block must give the same shift rows (bit-exact) whether a prompt
runs as one prefill, as two chunks through the slot, or token by token as
decode steps, and the same wkv state and outputs to 1e-2. The projections
are vendor-BLAS GEMMs whose accumulation order depends on the row count, so
their bf16 outputs (the WKV inputs) differ by an ulp here and there between
those runs (state differences ~5e-4 measured); a broken hand-off through the
slot (a stale shift row, a reset or double-applied state) differs by O(0.1)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import timemix as TM
from tests import util as U
from wkvm_amd import ops
from wkvm_amd.layout import RWKV7StateLayout
from wkvm_amd.state import RWKV7StateBank
from wkvm_amd.timemix import RWKV7TimeMix, TokenBatch

pytestmark = pytest.mark.gpu


def _bf(shape, dev, seed, scale=1.0):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return (torch.randn(shape, generator=g, device=dev) * scale).to(torch.bfloat16)


@pytest.mark.parametrize("D,rows,slots,cu,M", [
    (768, 17, [3, 9, 1, 16], None, 6),                   # decode, 0.1B width
    (2048, 9, [2, 7, 4, 5, 8], [0, 5, 5, 40, 41, 57], 6),  # ragged prefill, an empty sequence
    (2048, 9, [6], [0, 1], 1),                           # one token, channel-mix family (M = 1)
    (4096, 5, [1, 3], [0, 130, 131], 6),                 # 7B width, D = 2 block passes
    # 2-token tiles: boundaries inside tiles, a one-token sequence
    (2048, 9, [3, 8, 1], [0, 2999, 3000, 5001], 6),
    # 8-token tiles: boundaries at odd offsets, one-token and empty sequences
    (2048, 9, [4, 2, 6, 7, 1, 5], [0, 1, 5003, 5003, 5006, 12001, 16390], 6),
])
def test_token_shift_mix_bit_exact(dev, D, rows, slots, cu, M):
    T = len(slots) if cu is None else cu[-1]
    x = _bf((T, D), dev, 1)
    shift = _bf((3, 2, rows, D), dev, 2)  # [L, 2, S+1, D] like bank.shift
    mix = (torch.rand((M, D), generator=torch.Generator(device=dev).manual_seed(3), device=dev)
           ).to(torch.bfloat16)
    fam = 1 if M == 1 else 0
    before = shift.clone()
    out = ops.token_shift_mix(x, shift[1, fam], slots, mix, cu)
    torch.cuda.synchronize()
    ref_out, ref_shift = TM.token_shift_mix(U.bits(x), U.bits(before[1, fam]), slots,
                                            cu if cu is not None else range(T + 1), U.bits(mix))
    assert np.array_equal(U.bits(out), ref_out)
    assert np.array_equal(U.bits(shift[1, fam]), ref_shift)
    # other layers and the other family are untouched
    keep = shift.clone()
    keep[1, fam] = before[1, fam]
    assert torch.equal(keep, before)


def test_token_shift_mix_full_decode_shape(dev):
    """Config-1 shape: 256 slots of a 512-slot pool, D = 2048, six mixes."""
    D, rows = 2048, 513
    gen = torch.Generator().manual_seed(11)
    slots = (torch.randperm(512, generator=gen)[:256] + 1).tolist()
    x = _bf((256, D), dev, 4)
    shift = _bf((rows, D), dev, 5)
    mix = _bf((6, D), dev, 6, 0.5)
    before = U.bits(shift)
    out = ops.token_shift_mix(x, shift, slots, mix)
    torch.cuda.synchronize()
    ref_out, ref_shift = TM.token_shift_mix(U.bits(x), before, slots, range(257), U.bits(mix))
    assert np.array_equal(U.bits(out), ref_out)
    assert np.array_equal(U.bits(shift), ref_shift)


def _input_args(T, H, dev, seed, with_v=True):
    D = H * 64
    names = ["k", "v", "w_lora", "a_lora"]
    a = {n: _bf((T, D), dev, seed + i) for i, n in enumerate(names)}
    a["k_k"] = (0.5 + torch.rand(D, generator=torch.Generator(device=dev).manual_seed(seed + 9),
                                 device=dev)).to(torch.bfloat16)
    a["k_a"] = torch.rand(D, generator=torch.Generator(device=dev).manual_seed(seed + 10),
                          device=dev).to(torch.bfloat16)
    if with_v:
        a["v_lora"] = _bf((T, D), dev, seed + 11)
        a["v_first"] = _bf((T, D), dev, seed + 12)
    return a


def _ulp_ok(got: torch.Tensor, ref: np.ndarray) -> None:
    ulps = U.bf16_ulp_distance(U.bits(got), ref)
    edge = np.abs(U.f64(got) - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-30
    assert np.all((ulps <= 1) | edge), f"max {ulps.max()} ulps"


@pytest.mark.parametrize("T,H,with_v", [(7, 12, False), (256, 32, True), (3000, 32, True)])
def test_time_mix_inputs_match_oracle(dev, T, H, with_v):
    a = _input_args(T, H, dev, 20, with_v)
    outs = ops.time_mix_inputs(H, **a)
    torch.cuda.synchronize()
    f = {n: U.f64(t) for n, t in a.items()}
    ref = TM.time_mix_inputs(H, **f)
    for name, got in zip("wkvab", outs):
        if name == "v" and with_v:
            # the lerp can cancel: bound by its summands' magnitude
            s = 1.0 / (1.0 + np.exp(-f["v_lora"]))
            scale = np.abs(f["v"]) + np.abs(f["v_first"] - f["v"]) * s
            assert np.all(np.abs(U.f64(got) - ref["v"]) <= 2.0 ** -8 * scale + 1e-30)
        else:
            _ulp_ok(got, ref[name])


@pytest.mark.parametrize("T,H,y_dtype", [(5, 12, torch.float32), (256, 32, torch.bfloat16),
                                         (2000, 32, torch.float32)])
def test_time_mix_output_matches_oracle(dev, T, H, y_dtype):
    D = H * 64
    y = (torch.randn((T, H, 64), generator=torch.Generator(device=dev).manual_seed(30),
                     device=dev) * 2 + 0.3).to(y_dtype)
    r, k, v, g = (_bf((T, D), dev, 31 + i) for i in range(4))
    r_k = _bf((D,), dev, 40, 0.3)
    ln_w = (0.8 + 0.4 * torch.rand(D, generator=torch.Generator(device=dev).manual_seed(41),
                                   device=dev)).to(torch.bfloat16)
    ln_b = _bf((D,), dev, 42, 0.1)
    eps = 64e-5
    out = ops.time_mix_output(H, y, r, k, v, g, r_k, ln_w, ln_b, eps)
    torch.cuda.synchronize()
    ref, scale = TM.time_mix_output(H, U.f64(y), *(U.f64(t) for t in (r, k, v, g, r_k, ln_w,
                                                                       ln_b)), eps)
    err = np.abs(U.f64(out) - ref)
    assert np.all(err <= 2.0 ** -7 * scale + 1e-30), f"max err/scale {np.max(err / scale):.2e}"


# -- the composed block ------------------------------------------------------------------

def _block(dev, shape="0.1B", slots=6):
    layout = RWKV7StateLayout.for_shape(shape)
    bank = RWKV7StateBank(layout, slots, device=dev)
    bank.wkv.normal_(0.0, 0.1, generator=torch.Generator(device=dev).manual_seed(50))
    bank.shift.copy_(_bf(bank.shift.shape, dev, 51))
    layers = [RWKV7TimeMix.random(layout, l, dev, seed=3) for l in range(2)]
    return layout, bank, layers


def _run(bank, layers, x, slots, cu):
    batch = TokenBatch.plan(bank, slots, cu)
    v_first = None
    outs = []
    for layer in layers:
        o, v_first = layer.forward(bank, x, batch, v_first)
        outs.append(o)
    return outs


def test_block_prefill_equals_chunks_and_decode(dev):
    layout, bank0, layers = _block(dev)
    T, slot = 40, 4
    x = _bf((T, layout.hidden_size), dev, 60)
    banks = []
    for _ in range(3):
        b = RWKV7StateBank(layout, bank0.num_slots, device=dev)
        b.wkv.copy_(bank0.wkv)
        b.shift.copy_(bank0.shift)
        banks.append(b)
    # one prefill
    full = _run(banks[0], layers, x, [slot], [0, T])
    # two chunks threaded through the slot
    c1 = _run(banks[1], layers, x[:17], [slot], [0, 17])
    c2 = _run(banks[1], layers, x[17:], [slot], [0, T - 17])
    # token by token as decode steps
    steps = [_run(banks[2], layers, x[t:t + 1], [slot], None) for t in range(T)]
    torch.cuda.synchronize()
    for name, b in zip(("chunked", "decode"), banks[1:]):
        assert torch.equal(b.shift, banks[0].shift), "shift rows differ"
        err = U.normwise_max(U.f64(b.wkv[:, slot]), U.f64(banks[0].wkv[:, slot]))
        print(f"{name}: wkv state normwise difference {err:.2e}")
        assert err <= 1e-2, f"{name}: wkv state differs by {err:.2e}"
    others = [i for i in range(bank0.num_slots + 1) if i != slot]
    assert torch.equal(banks[0].wkv[:, others], bank0.wkv[:, others])
    assert torch.equal(banks[0].shift[:, :, others], bank0.shift[:, :, others])
    for l in range(len(layers)):
        ref = U.f64(full[l])
        chunked = np.concatenate([U.f64(c1[l]), U.f64(c2[l])])
        dec = np.concatenate([U.f64(s[l]) for s in steps])
        print(f"layer {l}: output rel-L2 chunked {U.rel_l2(chunked, ref):.2e}, "
              f"decode {U.rel_l2(dec, ref):.2e}")
        assert U.rel_l2(chunked, ref) <= 1e-2, f"layer {l}: chunked {U.rel_l2(chunked, ref):.2e}"
        assert U.rel_l2(dec, ref) <= 1e-2, f"layer {l}: decode {U.rel_l2(dec, ref):.2e}"


def test_block_ragged_batch_equals_separate_requests(dev):
    """One ragged launch over three requests (one of them a single token)
    equals running each request alone (wkvm/engine.py:142-170 runs them one by
    one)."""
    layout, bank0, layers = _block(dev)
    lens, slots = [9, 1, 22], [2, 5, 3]
    cu = [0, 9, 10, 32]
    x = _bf((32, layout.hidden_size), dev, 70)
    together = RWKV7StateBank(layout, bank0.num_slots, device=dev)
    together.wkv.copy_(bank0.wkv)
    together.shift.copy_(bank0.shift)
    outs = _run(together, layers, x, slots, cu)
    alone = RWKV7StateBank(layout, bank0.num_slots, device=dev)
    alone.wkv.copy_(bank0.wkv)
    alone.shift.copy_(bank0.shift)
    parts = [_run(alone, layers, x[cu[i]:cu[i + 1]], [slots[i]], [0, lens[i]]) for i in range(3)]
    torch.cuda.synchronize()
    assert torch.equal(together.shift, alone.shift)
    err = U.normwise_max(U.f64(together.wkv), U.f64(alone.wkv))
    print(f"ragged vs separate: wkv state normwise difference {err:.2e}")
    assert err <= 1e-2
    for l in range(len(layers)):
        sep = np.concatenate([U.f64(p[l]) for p in parts])
        assert U.rel_l2(U.f64(outs[l]), sep) <= 1e-2


def test_time_mix_decode_graph_replays_match_eager(dev):
    """Replays of the captured all-layer time-mix decode step equal the eager
    blocks bit for bit (outputs, shift rows, wkv state), over several steps with
    different slot batches and unrelated eager GPU work between replays."""
    from wkvm_amd.timemix import TimeMixDecodeGraph

    layout = RWKV7StateLayout(n_layer=3, hidden_size=256, num_heads=4, head_dim=64,
                              head_v_dim=64, dtype=torch.bfloat16)
    eager = RWKV7StateBank(layout, 20, device=dev)
    eager.wkv.normal_(0.0, 0.1, generator=torch.Generator(device=dev).manual_seed(80))
    eager.shift.copy_(_bf(eager.shift.shape, dev, 81))
    graphed = RWKV7StateBank(layout, 20, device=dev)
    graphed.wkv.copy_(eager.wkv)
    graphed.shift.copy_(eager.shift)
    layers = [RWKV7TimeMix.random(layout, l, dev, seed=5) for l in range(3)]
    B = 6
    tg = TimeMixDecodeGraph(graphed, layers, B)
    gen = torch.Generator().manual_seed(82)
    for step in range(4):
        slots = (torch.randperm(20, generator=gen)[:B] + 1).tolist()
        xs = _bf((3, B, 256), dev, 90 + step)
        batch = TokenBatch.plan(eager, slots)
        v_first, ref = None, []
        for l, layer in enumerate(layers):
            o, v_first = layer.forward(eager, xs[l], batch, v_first)
            ref.append(o)
        tg.set_slots(slots)
        tg.x.copy_(xs)
        out = tg.replay()
        torch.cuda.synchronize()
        assert torch.equal(torch.stack(out), torch.stack(ref)), f"step {step}: outputs differ"
        assert torch.equal(graphed.shift, eager.shift), f"step {step}: shift rows differ"
        assert torch.equal(graphed.wkv, eager.wkv), f"step {step}: wkv state differs"
        scratch = torch.randn(1 << 16, device=dev).sum()
        torch.cuda.synchronize()
        del scratch


def test_block_side_streams_give_the_same_bytes(dev, monkeypatch):
    """The block's independent GEMM chains on side streams (eager) produce the
    same outputs and state as the single-stream block (vendor-BLAS path, as
    taken above PROJ_MAX_ROWS tokens)."""
    monkeypatch.setattr(RWKV7TimeMix, "PROJ_MAX_ROWS", 0)
    layout = RWKV7StateLayout(n_layer=2, hidden_size=256, num_heads=4, head_dim=64,
                              head_v_dim=64, dtype=torch.bfloat16)
    banks = [RWKV7StateBank(layout, 12, device=dev) for _ in range(2)]
    banks[0].wkv.normal_(0.0, 0.1, generator=torch.Generator(device=dev).manual_seed(95))
    banks[0].shift.copy_(_bf(banks[0].shift.shape, dev, 96))
    banks[1].wkv.copy_(banks[0].wkv)
    banks[1].shift.copy_(banks[0].shift)
    layers = [RWKV7TimeMix.random(layout, l, dev, seed=7) for l in range(2)]
    streams = [torch.cuda.Stream(dev) for _ in range(3)]
    slots = [3, 7, 1, 11, 5]
    x = _bf((2, len(slots), 256), dev, 97)
    outs = []
    for bank, st in zip(banks, (None, streams)):
        batch = TokenBatch.plan(bank, slots)
        v_first, o = None, []
        for l, layer in enumerate(layers):
            y, v_first = layer.forward(bank, x[l], batch, v_first, streams=st)
            o.append(y)
        outs.append(torch.stack(o))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    assert torch.equal(banks[0].wkv, banks[1].wkv) and torch.equal(banks[0].shift, banks[1].shift)


def test_block_grouped_projections_match_vendor_path(dev, monkeypatch):
    """The block with its projections on wkv7_proj_grouped (decode-sized
    batches) against the same block on the vendor BLAS: both round every
    GEMM output to bf16 once (the grouped path applies the LoRA tanh/sigmoid
    before that rounding), so outputs and state agree to bf16 rounding."""
    layout = RWKV7StateLayout(n_layer=3, hidden_size=512, num_heads=8, head_dim=64,
                              head_v_dim=64, dtype=torch.bfloat16)
    banks = [RWKV7StateBank(layout, 40, device=dev) for _ in range(2)]
    banks[0].wkv.normal_(0.0, 0.1, generator=torch.Generator(device=dev).manual_seed(105))
    banks[0].shift.copy_(_bf(banks[0].shift.shape, dev, 106))
    banks[1].wkv.copy_(banks[0].wkv)
    banks[1].shift.copy_(banks[0].shift)
    layers = [RWKV7TimeMix.random(layout, l, dev, seed=9) for l in range(3)]
    slots = list(range(3, 35))
    x = _bf((3, len(slots), 512), dev, 107)
    outs = []
    for bank, rows in zip(banks, (RWKV7TimeMix.PROJ_MAX_ROWS, 0)):
        monkeypatch.setattr(RWKV7TimeMix, "PROJ_MAX_ROWS", rows)
        batch = TokenBatch.plan(bank, slots)
        v_first, o = None, []
        for l, layer in enumerate(layers):
            y, v_first = layer.forward(bank, x[l], batch, v_first)
            o.append(y)
        outs.append(torch.stack(o))
    torch.cuda.synchronize()
    assert torch.equal(banks[0].shift, banks[1].shift)
    err = U.normwise_max(U.f64(banks[0].wkv), U.f64(banks[1].wkv))
    rel = U.rel_l2(U.f64(outs[0]), U.f64(outs[1]))
    print(f"grouped vs vendor: state {err:.2e}, outputs rel-L2 {rel:.2e}")
    assert err <= 1e-2 and rel <= 1e-2


@pytest.mark.parametrize("first_layer,scale", [(True, 1.0), (False, 1.0), (False, 0.5)])
def test_decode_block_bit_identical_to_three_kernels(dev, first_layer, scale):
    """wkv7_decode_block equals time_mix_inputs -> wkv7_decode_slots (bf16 y)
    -> time_mix_output bit for bit: output, v, and the state of every slot
    (untouched slots included), with scattered slots in slot-sorted order.
    scale multiplies r in the state readout only (the bonus uses raw r)."""
    H, B, S = 8, 37, 60
    D = H * 64
    gen = torch.Generator(device=dev).manual_seed(120 + first_layer)

    def bf(shape, std=1.0):
        return (torch.randn(shape, generator=gen, device=dev) * std).to(torch.bfloat16)

    r, k, v, wl, al, g = (bf((B, D)) for _ in range(6))
    vl, vf = (None, None) if first_layer else (bf((B, D)), bf((B, D)))
    k_k = (torch.rand(D, generator=gen, device=dev) + 0.5).to(torch.bfloat16)
    k_a, ln_w = ((torch.rand(D, generator=gen, device=dev)).to(torch.bfloat16) for _ in range(2))
    r_k, ln_b = bf(D, 0.1), bf(D, 0.05)
    eps = 64e-5
    pool = torch.randn((S + 1, H, 64, 64), generator=gen, device=dev) * 0.1
    slots = (torch.randperm(S, generator=torch.Generator().manual_seed(7))[:B] + 1).tolist()
    ids, order = ops.decode_plan(slots, S + 1, dev)
    ref_pool = pool.clone()
    w2, k2, v2, a2, b2 = ops.time_mix_inputs(H, k, v, wl, al, k_k, k_a, vl, vf)
    vec = [t.view(B, H, 64) for t in (r, w2, k2, v2, a2, b2)]
    y = ops.wkv7_decode_slots(ref_pool, ids, *vec, row_order=order, scale=scale)
    ref = ops.time_mix_output(H, y, r, k2, v2, g, r_k, ln_w, ln_b, eps)
    out, v_out = ops.wkv7_decode_block(pool, ids, H, r, k, v, wl, al, g, k_k, k_a, r_k, ln_w,
                                       ln_b, eps, v_lora=vl, v_first=vf, row_order=order,
                                       scale=scale, want_v=True)
    torch.cuda.synchronize()
    assert torch.equal(v_out, v2)
    assert torch.equal(out, ref)
    assert torch.equal(pool, ref_pool)
