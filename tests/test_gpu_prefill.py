"""Prefill parity: wkv7_prefill_varlen (HIP, through the C ABI) against the
float64 oracle on the same seeded inputs.

Bars (north star): relative L2 <= 1e-3 per sequence on the final state and on
the per-token y. A bf16 y is compared with the float64 y rounded to bf16 (the
rounding of the output alone is ~1.5e-3 relative L2, so comparing it with the
unrounded value would test the storage format, not the kernel); an fp32 y is
compared with the unrounded value."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from tests import util as U
from wkvm_amd import ops, synthetic
from wkvm_amd.layout import RWKV7StateLayout
from wkvm_amd.runner import WKV7Runner
from wkvm_amd.state import RWKV7StateBank

pytestmark = pytest.mark.gpu

REL_L2 = 1e-3


def _check(pool_before, ids, cu, vbits, gpool, y, zero_init, tol=REL_L2):
    y_ref, h_ref = O.scan_bf16(cu, *vbits, pool=None if zero_init else pool_before,
                               slot_ids=None if zero_init else ids)
    h = U.f64(gpool[ids])
    yv = U.f64(y)
    if y.dtype == torch.bfloat16:
        y_cmp = O.round_f64_to_bf16(y_ref)
    else:
        y_cmp = y_ref
    worst_h, worst_y = 0.0, 0.0
    for s in range(len(ids)):
        worst_h = max(worst_h, U.rel_l2(h[s], h_ref[s]))
        if cu[s + 1] > cu[s]:
            worst_y = max(worst_y, U.rel_l2(yv[cu[s]:cu[s + 1]], y_cmp[cu[s]:cu[s + 1]]))
    assert worst_h <= tol, f"final state rel L2 {worst_h:.3e}"
    assert worst_y <= tol, f"y rel L2 {worst_y:.3e}"
    return worst_h, worst_y


@pytest.mark.parametrize("zero_init", [False, True])
@pytest.mark.parametrize("y_dtype", [torch.bfloat16, torch.float32])
def test_ragged_lengths_from_slot_state(dev, zero_init, y_dtype):
    """Edge lengths around the chunk size, a zero-length and a length-1 row."""
    H, S = 4, 12
    lens = [1, 5, 0, 63, 64, 65, 130, 257]
    cu = np.concatenate([[0], np.cumsum(lens)])
    gen = synthetic.make_generator(31)
    pool = torch.zeros((S + 1, H, 64, 64))
    pool[1:] = synthetic.initial_states((S, H, 64, 64), gen)
    ids = synthetic.active_slots(S, len(lens), gen)
    vecs = synthetic.wkv7_vectors((int(cu[-1]), H, 64), gen)
    gpool = pool.to(dev)
    y = ops.wkv7_prefill_varlen(gpool, ids, cu.tolist(), *(vecs[n].to(dev) for n in "rwkvab"),
                                zero_init=zero_init, out_dtype=y_dtype)
    torch.cuda.synchronize()
    _check(pool.numpy(), ids, cu, U.vec_bits(vecs), gpool, y, zero_init)
    others = [i for i in range(S + 1) if i not in ids]
    assert torch.equal(gpool[others].cpu(), pool[others])
    if zero_init:  # the zero-length row leaves an all-zero (fresh) state
        assert gpool[ids[2]].abs().sum().item() == 0.0
    else:          # ... or its slot state untouched
        assert torch.equal(gpool[ids[2]].cpu(), pool[ids[2]])


def test_sequence_order_changes_nothing(dev):
    """The visiting order of the sequences (``seq_order``) only schedules the
    workgroups: identity, reversed and longest-first launches give the same
    bytes, final states and y alike."""
    H, S = 4, 10
    lens = [3, 300, 0, 64, 129, 17, 640]
    cu = np.concatenate([[0], np.cumsum(lens)]).tolist()
    gen = synthetic.make_generator(33)
    pool = torch.zeros((S + 1, H, 64, 64))
    pool[1:] = synthetic.initial_states((S, H, 64, 64), gen)
    ids = synthetic.active_slots(S, len(lens), gen)
    vecs = [x.to(dev) for x in synthetic.order(synthetic.wkv7_vectors((cu[-1], H, 64), gen))]
    n = len(lens)
    orders = [None, list(range(n)), list(range(n))[::-1], ops.longest_first(cu)]
    assert ops.longest_first(cu)[:2] == [6, 1]
    outs = []
    for order in orders:
        gpool = pool.to(dev)
        seq = None if order is None else torch.tensor(order, dtype=torch.int32, device=dev)
        y = ops.wkv7_prefill_varlen(gpool, ids, cu, *vecs, seq_order=seq)
        torch.cuda.synchronize()
        outs.append((gpool.cpu(), y.cpu()))
    for p, y in outs[1:]:
        assert torch.equal(p, outs[0][0]) and torch.equal(y, outs[0][1])
    with pytest.raises(ValueError):
        ops.wkv7_prefill_varlen(pool.to(dev), ids, cu, *vecs,
                                seq_order=torch.arange(n - 1, dtype=torch.int32, device=dev))


def test_cfg2_full_size_zero_init(dev):
    """Config 2: 1.5B shape (H=32), 8 sequences x 4096 tokens from zero state,
    final states written to 8 seeded slots of a 16-slot pool; every token's y
    and every final state checked."""
    H, S, nseq, T = 32, 16, 8, 4096
    gen = synthetic.make_generator(2)
    ids = synthetic.active_slots(S, nseq, gen)
    vecs = synthetic.wkv7_vectors((nseq * T, H, 64), gen)
    cu = np.arange(nseq + 1) * T
    gpool = torch.full((S + 1, H, 64, 64), 7.0, device=dev)  # stale contents must be ignored
    y = ops.wkv7_prefill_varlen(gpool, ids, cu.tolist(), *(vecs[n].to(dev) for n in "rwkvab"),
                                zero_init=True)
    torch.cuda.synchronize()
    eh, ey = _check(None, ids, cu, U.vec_bits(vecs), gpool, y, zero_init=True)
    print(f"cfg2: worst final-state rel L2 {eh:.2e}, worst y rel L2 (bf16) {ey:.2e}")
    others = [i for i in range(S + 1) if i not in ids]
    assert bool((gpool[others] == 7.0).all())


@pytest.mark.parametrize("batch", ["ragged", "cfg4_rows", "segmented", "one_request"])
def test_repeated_runs_are_bit_identical(dev, batch):
    """The same batch (slot state in, fp32 y) run six times gives bit-identical
    y and final states every time: no result may depend on timing
    (matrix-core results read back by vector instructions before they are
    ready, LDS reads racing a tick's writes). Four batches: eight ragged
    sequences; config 4's prefill rows (64 lengths uniform in [1, 2048] at the
    1.5B head count, longest first); the segmented form (runs from zero
    and identity state, the chain and the correction) on few long sequences;
    and one 4096-token request, which runs on the quarter-head kernel.
    Re-entry determinism is what the reference relies on when a preempted
    request resumes from its slot (wkvm/runner/runner.py:30-33)."""
    H, S = 32, 72
    gen = synthetic.make_generator(5)
    if batch == "cfg4_rows":
        lens = torch.randint(1, 2049, (64,), generator=gen).tolist()
    elif batch == "segmented":
        lens = [4096, 3000, 17]
    elif batch == "one_request":
        lens = [4096]
    else:
        lens = [4096, 4001, 17, 1, 100, 2000, 33, 3000]
    cu = np.concatenate([[0], np.cumsum(lens)]).tolist()
    gdev = synthetic.make_generator(6, dev)  # config 4's ~65k tokens are drawn on the GPU
    vecs = synthetic.wkv7_vectors((cu[-1], H, 64), gdev)
    xs = [vecs[n] for n in "rwkvab"]
    pool0 = torch.zeros((S + 1, H, 64, 64), device=dev)
    pool0[1:] = synthetic.initial_states((S, H, 64, 64), gdev)
    ids = list(range(1, len(lens) + 1))
    ref = None
    for rep in range(6):
        pool = pool0.clone()
        if batch == "segmented":
            y = ops.wkv7_prefill_segments(pool, ids, cu, *xs, segments=4,
                                          out_dtype=torch.float32)
        else:
            y = ops.wkv7_prefill_varlen(pool, ids, cu, *xs, out_dtype=torch.float32)
        torch.cuda.synchronize()
        if ref is None:
            ref = (y, pool)
        else:
            assert torch.equal(y, ref[0]), f"run {rep}: y differs"
            assert torch.equal(pool, ref[1]), f"run {rep}: final states differ"


def test_chunk_split_invariance_through_the_slot(dev):
    """CF6: one call over T tokens equals the runner's chunked re-entry through
    the slot (prefill_chunk 64, 100 and 4096), as a preempted request's would.
    Chunks on the kernel's 16-token sub-chunk grid (64) reproduce the one-call
    result bit for bit; other chunks (100) shift the grid, and the operands the
    kernel takes as one bf16 each (A^, T) then round differently, so they
    agree to the parity bar."""
    lay = RWKV7StateLayout(n_layer=2, hidden_size=512, num_heads=8, head_dim=64, head_v_dim=64,
                           dtype=torch.bfloat16)
    T = 700
    gen = synthetic.make_generator(41)
    layer_vecs = [synthetic.wkv7_vectors((T, 8, 64), gen, device=dev) for _ in range(2)]
    inputs = [synthetic.order(v) for v in layer_vecs]
    finals, outs = [], []
    for chunk in (4096, 64, 100):
        bank = RWKV7StateBank(lay, num_slots=3, device=dev)
        run = WKV7Runner(bank, prefill_chunk=chunk)
        ys = run.prefill(inputs, {"wkv": 2, "shift": 2}, out_dtype=torch.float32)
        finals.append(bank.wkv[:, 2].clone())
        outs.append(torch.stack(ys))
    assert torch.equal(finals[1], finals[0]) and torch.equal(outs[1], outs[0])
    assert U.rel_l2(U.f64(finals[2]), U.f64(finals[0])) <= REL_L2
    assert U.rel_l2(U.f64(outs[2]), U.f64(outs[0])) <= REL_L2


def test_fla_signatures(dev):
    """chunk_rwkv7 / fused_recurrent_rwkv7 with [B, T, H, K] tensors, an initial
    state, packed cu_seqlens and head_first, against the oracle."""
    B, T, H = 3, 80, 4
    gen = synthetic.make_generator(51)
    vecs = synthetic.wkv7_vectors((B, T, H, 64), gen)
    h0 = synthetic.initial_states((B, H, 64, 64), gen)
    xs = [vecs[n].to(dev) for n in "rwkvab"]
    h0d = h0.to(dev)
    o, hT = ops.chunk_rwkv7(*xs, scale=1.0, initial_state=h0d, output_final_state=True)
    flat_bits = [U.bits(vecs[n].reshape(B * T, H, 64)) for n in "rwkvab"]
    cu = np.arange(B + 1) * T
    y_ref, h_ref = O.scan_bf16(cu, *flat_bits, pool=h0.numpy(), slot_ids=list(range(B)))
    assert o.shape == (B, T, H, 64) and o.dtype == torch.bfloat16
    assert U.rel_l2(U.f64(hT), h_ref) <= REL_L2
    assert U.rel_l2(U.f64(o).reshape(B * T, H, 64), O.round_f64_to_bf16(y_ref)) <= REL_L2
    assert torch.equal(h0d.cpu(), h0)  # the caller's initial_state is not modified
    o2, h2 = ops.fused_recurrent_rwkv7(*(x.transpose(1, 2) for x in xs), initial_state=h0.to(dev),
                                       head_first=True)
    assert torch.equal(o2.transpose(1, 2), o) and torch.equal(h2, hT)
    # packed sequences of lengths 30, 0, 120 with no initial state
    lens = [30, 0, 120]
    packed = synthetic.wkv7_vectors((1, sum(lens), H, 64), gen)
    cu = [0, 30, 30, 150]
    o3, h3 = ops.chunk_rwkv7(*(packed[n].to(dev) for n in "rwkvab"), cu_seqlens=cu)
    y_ref, h_ref = O.scan_bf16(np.array(cu), *(U.bits(packed[n][0]) for n in "rwkvab"))
    assert U.rel_l2(U.f64(h3), h_ref) <= REL_L2
    assert U.rel_l2(U.f64(o3[0]), O.round_f64_to_bf16(y_ref)) <= REL_L2
    assert h3[1].abs().sum().item() == 0.0
    _, none = ops.chunk_rwkv7(*xs, output_final_state=False)
    assert none is None


def test_chunk_rwkv7_cfg2_shape_out_of_place(dev):
    """chunk_rwkv7 at config 2's shape (8 x 4096 tokens, H = 32) from an
    initial state: the state is read from initial_state and written to a new
    final_state by one kernel launch (no copy of the state), both against the
    float64 oracle; initial_state keeps its bytes, and output_final_state=False
    runs the same y with no state written (wkvm/models/rwkv7.py:108-109)."""
    B, T, H = 8, 4096, 32
    gen = synthetic.make_generator(53)
    vecs = synthetic.wkv7_vectors((B, T, H, 64), gen)
    h0 = synthetic.initial_states((B, H, 64, 64), gen)
    xs = [vecs[n].to(dev) for n in "rwkvab"]
    h0d = h0.to(dev)
    o, hT = ops.chunk_rwkv7(*xs, initial_state=h0d, output_final_state=True)
    torch.cuda.synchronize()
    assert hT.data_ptr() != h0d.data_ptr()
    assert torch.equal(h0d.cpu(), h0)  # initial_state is only read
    cu = np.arange(B + 1) * T
    flat = [U.bits(vecs[n].reshape(B * T, H, 64)) for n in "rwkvab"]
    y_ref, h_ref = O.scan_bf16(cu, *flat, pool=h0.numpy(), slot_ids=list(range(B)))
    y_cmp = O.round_f64_to_bf16(y_ref)
    hv, yv = U.f64(hT), U.f64(o).reshape(B * T, H, 64)
    eh = max(U.rel_l2(hv[s], h_ref[s]) for s in range(B))
    ey = max(U.rel_l2(yv[s * T:(s + 1) * T], y_cmp[s * T:(s + 1) * T]) for s in range(B))
    print(f"chunk_rwkv7 cfg2 shape: worst state rel L2 {eh:.2e}, y {ey:.2e}")
    assert eh <= REL_L2 and ey <= REL_L2
    o2, none = ops.chunk_rwkv7(*xs, initial_state=h0d, output_final_state=False)
    torch.cuda.synchronize()
    assert none is None and torch.equal(o2, o)


def test_prefill_into_rows_and_in_place(dev):
    """wkv7_prefill_into: sequences read states from permuted rows of one
    tensor and write them to other rows of another; the result equals the
    in-place slot prefill bit for bit, and the same tensor with in_ids ==
    out_ids is the in-place call. No state_in means zero state; no state_out
    writes nothing."""
    H, S = 4, 9
    lens = [100, 0, 1, 333]
    cu = np.concatenate([[0], np.cumsum(lens)]).tolist()
    gen = synthetic.make_generator(57)
    src = synthetic.initial_states((S, H, 64, 64), gen).to(dev)
    vecs = [x.to(dev) for x in synthetic.order(synthetic.wkv7_vectors((cu[-1], H, 64), gen))]
    in_ids, out_ids = [5, 0, 8, 2], [1, 7, 3, 6]
    dst = torch.full((S, H, 64, 64), 3.0, device=dev)
    y = ops.wkv7_prefill_into(src, dst, cu, *vecs, in_ids=in_ids, out_ids=out_ids,
                              out_dtype=torch.float32)
    pool = src.clone()
    y_ref = ops.wkv7_prefill_varlen(pool, in_ids, cu, *vecs, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref)
    assert torch.equal(dst[out_ids], pool[in_ids])
    assert torch.equal(dst[7], src[0])  # the empty sequence's state passes through
    assert bool((dst[[0, 2, 4, 5, 8]] == 3.0).all())
    same = src.clone()
    y2 = ops.wkv7_prefill_into(same, same, cu, *vecs, in_ids=in_ids, out_ids=in_ids,
                               out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(y2, y_ref) and torch.equal(same, pool)
    zero = torch.zeros_like(src)
    y_zero_ref = ops.wkv7_prefill_varlen(zero, [1, 2, 3, 4], cu, *vecs, out_dtype=torch.float32)
    y3 = ops.wkv7_prefill_into(None, None, cu, *vecs, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(y3, y_zero_ref)
    with pytest.raises(ValueError, match="reads"):
        ops.wkv7_prefill_into(same, same, cu, *vecs, in_ids=[0, 1, 2, 3], out_ids=[1, 2, 3, 4])


@pytest.mark.parametrize("H", [2, 64])
def test_rejected_device_slot_ids_zero_the_prefill_y(dev, H):
    """A device slot id the kernel's bounds check rejects leaves that
    sequence's state untouched and writes y = 0 for its tokens (as the decode
    step does), so a caller's uninitialised output never leaks; the other
    sequences are unaffected. Same for wkv7_prefill_into's in and out ids.
    H = 2 runs the quarter-head kernel (few busy heads), H = 64 the
    whole-head one."""
    S = 6
    lens = [40, 100, 17]
    cu = [0, 40, 140, 157]
    gen = synthetic.make_generator(309)
    pool = synthetic.initial_states((S + 1, H, 64, 64), gen).to(dev)
    before = pool.clone()
    vecs = [x.to(dev) for x in synthetic.order(synthetic.wkv7_vectors((cu[-1], H, 64), gen))]
    for y_dtype in (torch.bfloat16, torch.float32):
        pool.copy_(before)
        bad = torch.tensor([2, S + 1, 4], dtype=torch.int32, device=dev)
        y = torch.full((cu[-1], H, 64), 5.0, dtype=y_dtype, device=dev)
        ops.wkv7_prefill_varlen(pool, bad, torch.tensor(cu, dtype=torch.int32, device=dev),
                                *vecs, out=y)
        ref = before.clone()
        y_ok = ops.wkv7_prefill_varlen(ref, [2, 4], [0, 40, 57],
                                       *(torch.cat([x[0:40], x[140:157]]) for x in vecs),
                                       out_dtype=y_dtype)
        torch.cuda.synchronize()
        assert not torch.any(y[40:140])
        assert torch.equal(y[0:40], y_ok[0:40]) and torch.equal(y[140:157], y_ok[40:57])
        assert torch.equal(pool, ref)
    dst = torch.zeros_like(before)
    y2 = torch.full((cu[-1], H, 64), 5.0, device=dev)
    ops.wkv7_prefill_into(before, dst, cu, *vecs, out=y2,
                          in_ids=torch.tensor([1, -1, 3], dtype=torch.int32, device=dev),
                          out_ids=torch.tensor([1, 2, 99], dtype=torch.int32, device=dev))
    torch.cuda.synchronize()
    assert torch.any(y2[0:40]) and not torch.any(y2[40:157])
    assert torch.any(dst[1]) and not torch.any(dst[2:])


@pytest.mark.parametrize("zero_init", [False, True])
@pytest.mark.parametrize("y_dtype", [torch.bfloat16, torch.float32])
def test_quarter_heads_bit_identical_to_whole_heads(dev, zero_init, y_dtype):
    """A launch that would keep at most a quarter of the compute units busy
    (4 x sequences x heads <= CUs) runs each (sequence, head) on four
    workgroups, one per 16 value columns, each repeating the operand, score
    and inverse work. The same sequences launched beside enough empty ones to
    fill the GPU run one workgroup per pair. Both give the same bits, and
    both match the oracle."""
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    H = 4
    lens = [700, 1, 33, 0, 256, 64]
    assert 4 * len(lens) * H <= cus
    n_pad = cus // (4 * H) + 1 - len(lens)
    S = len(lens) + n_pad + 2
    gen = synthetic.make_generator(83)
    pool = torch.zeros((S + 1, H, 64, 64))
    pool[1:] = synthetic.initial_states((S, H, 64, 64), gen)
    cu = np.concatenate([[0], np.cumsum(lens)]).tolist()
    vecs = synthetic.wkv7_vectors((cu[-1], H, 64), gen)
    xs = [vecs[n].to(dev) for n in "rwkvab"]
    ids = list(range(1, len(lens) + 1))
    few = pool.to(dev)
    y_few = ops.wkv7_prefill_varlen(few, ids, cu, *xs, zero_init=zero_init, out_dtype=y_dtype)
    full = pool.to(dev)
    ids_full = ids + list(range(len(lens) + 1, len(lens) + 1 + n_pad))
    assert 4 * len(ids_full) * H > cus
    y_full = ops.wkv7_prefill_varlen(full, ids_full, cu + [cu[-1]] * n_pad, *xs,
                                     zero_init=zero_init, out_dtype=y_dtype)
    torch.cuda.synchronize()
    assert torch.equal(y_few, y_full)
    assert torch.equal(few[:len(lens) + 1], full[:len(lens) + 1])
    _check(pool.numpy(), ids, np.array(cu), U.vec_bits(vecs), few, y_few, zero_init)


def test_prefill_argument_errors(dev):
    pool = torch.zeros((5, 2, 64, 64), device=dev)
    vecs = synthetic.order(synthetic.wkv7_vectors((10, 2, 64), synthetic.make_generator(0),
                                                  device=dev))
    with pytest.raises(ValueError):
        ops.wkv7_prefill_varlen(pool, [1, 2], [0, 4, 9], *vecs)        # does not end at T
    with pytest.raises(ValueError):
        ops.wkv7_prefill_varlen(pool, [1, 2], [0, 6, 4, 10], *vecs)   # wrong count
    with pytest.raises(ValueError, match="duplicate"):
        ops.wkv7_prefill_varlen(pool, [1, 1], [0, 4, 10], *vecs)
    with pytest.raises(ValueError, match="bfloat16"):
        ops.wkv7_prefill_varlen(pool, [1, 2], [0, 4, 10], *(x.float() for x in vecs))
    # y rows are stored as vectors: a contiguous out view 2 bytes off alignment is refused
    skew = torch.empty(10 * 2 * 64 + 1, dtype=torch.bfloat16, device=dev)[1:].view(10, 2, 64)
    with pytest.raises(ValueError, match="aligned"):
        ops.wkv7_prefill_varlen(pool, [1, 2], [0, 4, 10], *vecs, out=skew)


def test_mixed_step_equals_separate_calls(dev):
    """Config 4's shape at reduced size: one decode launch + one varlen prefill
    launch per layer equals running every row on its own (the reference
    engine's own decomposition, wkvm/engine.py:142-170)."""
    lay = RWKV7StateLayout(n_layer=2, hidden_size=256, num_heads=4, head_dim=64, head_v_dim=64,
                           dtype=torch.bfloat16)
    gen = synthetic.make_generator(61)
    S = 20
    init = synthetic.initial_states((2, S + 1, 4, 64, 64), gen).to(dev)
    dec_slots = [3, 7, 11, 15, 19]
    pre_slots = [1, 9, 18]
    lens = [1, 97, 200]
    dec_in = [synthetic.order(synthetic.wkv7_vectors((5, 4, 64), gen, device=dev)) for _ in range(2)]
    pre_in = [synthetic.order(synthetic.wkv7_vectors((sum(lens), 4, 64), gen, device=dev))
              for _ in range(2)]
    bank = RWKV7StateBank(lay, num_slots=S, device=dev)
    bank.wkv.copy_(init)
    run = WKV7Runner(bank)
    dys, pys = run.mixed_step([{"wkv": s, "shift": s} for s in dec_slots], dec_in,
                              [{"wkv": s, "shift": s} for s in pre_slots], lens, pre_in,
                              out_dtype=torch.float32)
    ref = RWKV7StateBank(lay, num_slots=S, device=dev)
    ref.wkv.copy_(init)
    cu = [0, 1, 98, 298]
    for layer in range(2):
        for i, s in enumerate(dec_slots):
            y = ref.decode_wkv(layer, [{"wkv": s, "shift": s}], *(x[i:i + 1] for x in dec_in[layer]),
                               out_dtype=torch.float32)
            assert torch.equal(y, dys[layer][i:i + 1])
        for i, s in enumerate(pre_slots):
            y = ref.prefill_wkv(layer, [{"wkv": s, "shift": s}], [0, lens[i]],
                                *(x[cu[i]:cu[i + 1]] for x in pre_in[layer]),
                                out_dtype=torch.float32)
            assert U.rel_l2(U.f64(y), U.f64(pys[layer][cu[i]:cu[i + 1]])) <= 1e-6
    assert U.rel_l2(U.f64(bank.wkv), U.f64(ref.wkv)) <= 1e-6
    with pytest.raises(ValueError, match="same step"):
        run.mixed_step([{"wkv": 1, "shift": 1}], [[x[:1] for x in d] for d in dec_in],
                       [{"wkv": 1, "shift": 1}], [1], [[x[:1] for x in p] for p in pre_in])


@pytest.mark.parametrize("y_dtype", [torch.bfloat16, torch.float32])
def test_7b_shape_prefill_matches_oracle(dev, y_dtype):
    """7B head count (H = 64): ragged sequences from slot state, lengths
    around the sub-chunk and chunk sizes."""
    H, S = 64, 10
    lens = [17, 300, 1, 64, 129]
    cu = np.concatenate([[0], np.cumsum(lens)])
    gen = synthetic.make_generator(181)
    pool = torch.zeros((S + 1, H, 64, 64))
    pool[1:] = synthetic.initial_states((S, H, 64, 64), gen)
    ids = synthetic.active_slots(S, len(lens), gen)
    vecs = synthetic.wkv7_vectors((int(cu[-1]), H, 64), gen)
    gpool = pool.to(dev)
    y = ops.wkv7_prefill_varlen(gpool, ids, cu.tolist(), *(vecs[n].to(dev) for n in "rwkvab"),
                                out_dtype=y_dtype)
    torch.cuda.synchronize()
    _check(pool.numpy(), ids, cu, U.vec_bits(vecs), gpool, y, zero_init=False)


def test_mixed_step_concurrent_equals_serial(dev):
    """The decode launches on a side stream (forked from and joined into the
    current stream) give the same bits as the single-stream step."""
    lay = RWKV7StateLayout(n_layer=3, hidden_size=512, num_heads=8, head_dim=64, head_v_dim=64,
                           dtype=torch.bfloat16)
    gen = synthetic.make_generator(62)
    S = 40
    init = synthetic.initial_states((3, S + 1, 8, 64, 64), gen).to(dev)
    dec_slots = list(range(2, 34, 2))
    pre_slots = [1, 5, 39]
    lens = [700, 33, 1]
    dec_in = [synthetic.order(synthetic.wkv7_vectors((16, 8, 64), gen, device=dev))
              for _ in range(3)]
    pre_in = [synthetic.order(synthetic.wkv7_vectors((sum(lens), 8, 64), gen, device=dev))
              for _ in range(3)]
    out = []
    for concurrent in (True, False):
        bank = RWKV7StateBank(lay, num_slots=S, device=dev)
        bank.wkv.copy_(init)
        ys = WKV7Runner(bank).mixed_step([{"wkv": s, "shift": s} for s in dec_slots], dec_in,
                                         [{"wkv": s, "shift": s} for s in pre_slots], lens, pre_in,
                                         concurrent=concurrent)
        torch.cuda.synchronize()
        out.append((bank.wkv.clone(), ys))
    assert torch.equal(out[0][0], out[1][0])
    for a, b in zip(out[0][1][0] + out[0][1][1], out[1][1][0] + out[1][1][1]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("H", [64, 8])
def test_large_batch_uses_the_64bit_input_path(dev, H):
    """A batch whose input bytes exceed 31-bit offsets runs the operand waves'
    global-load path instead of the buffer-resource one; the first (checked)
    sequence must match the oracle there too. The second sequence is zero
    input and only makes the batch large: 262,144 tokens at H = 64 (one
    workgroup per head) or 2,097,152 at H = 8 (few heads: the quarter-head
    kernel)."""
    S = 4
    lens = [300, (1 << 24) // H]
    cu = [0, lens[0], lens[0] + lens[1]]
    gen = synthetic.make_generator(191)
    pool = torch.zeros((S + 1, H, 64, 64))
    pool[1:] = synthetic.initial_states((S, H, 64, 64), gen)
    small = synthetic.wkv7_vectors((lens[0], H, 64), gen)
    xs = []
    for n in "rwkvab":
        t = torch.zeros((cu[-1], H, 64), dtype=torch.bfloat16, device=dev)
        t[:lens[0]] = small[n].to(dev)
        xs.append(t)
    gpool = pool.to(dev)
    y = ops.wkv7_prefill_varlen(gpool, [2, 3], cu, *xs, out_dtype=torch.float32)
    torch.cuda.synchronize()
    y_ref, h_ref = O.scan_bf16(np.array([0, lens[0]]), *U.vec_bits(small), pool=pool.numpy(),
                               slot_ids=[2])
    assert U.rel_l2(U.f64(y[:lens[0]]), y_ref) <= REL_L2
    assert U.rel_l2(U.f64(gpool[2]), h_ref[0]) <= REL_L2
    # all-zero input: log-decay 0 is a decay of 1 and every update term is a
    # product with zero, so the second slot keeps its state and reads out 0
    assert not torch.any(y[lens[0]:])
    assert U.rel_l2(U.f64(gpool[3]), pool[3].double().numpy()) <= 1e-6
    assert torch.equal(gpool[[0, 1, 4]].cpu(), pool[[0, 1, 4]])


@pytest.mark.parametrize("H", [2, 72])
@pytest.mark.parametrize("pattern", ["channels", "tokens", "all_max", "limit"])
def test_decay_extremes_and_scale(dev, pattern, H):
    """RWKV-7's log-decay lies in (-exp(-0.5), 0]. Both ends of that range
    (no decay, and the strongest decay, whose 16-token products reach
    e^{+-9.7} inside a sub-chunk) against the oracle, with scale = 1/8:
    per key channel, per token, or the strongest decay everywhere; and the
    documented limit of the chunked form, w = -5 everywhere (e^{+-80}).
    H = 2 runs the quarter-head kernel, H = 72 the whole-head one."""
    S = 6
    lens = [300, 333]
    cu = np.concatenate([[0], np.cumsum(lens)])
    T = int(cu[-1])
    gen = synthetic.make_generator(77)
    pool = torch.zeros((S + 1, H, 64, 64))
    pool[1:] = synthetic.initial_states((S, H, 64, 64), gen)
    ids = [4, 2]
    vecs = synthetic.wkv7_vectors((T, H, 64), gen)
    wmax = -synthetic.DECAY_SCALE
    if pattern == "channels":
        w = torch.where(torch.arange(64) % 2 == 0, 0.0, wmax).expand(T, H, 64)
    elif pattern == "tokens":
        w = torch.where(torch.arange(T) % 3 == 0, 0.0, wmax)[:, None, None].expand(T, H, 64)
    elif pattern == "all_max":
        w = torch.full((T, H, 64), wmax)
    else:
        w = torch.full((T, H, 64), -5.0)
    vecs["w"] = w.to(torch.bfloat16).contiguous()
    scale = 0.125
    gpool = pool.to(dev)
    y = ops.wkv7_prefill_varlen(gpool, ids, cu.tolist(), *(vecs[n].to(dev) for n in "rwkvab"),
                                scale=scale, out_dtype=torch.float32)
    torch.cuda.synchronize()
    y_ref, h_ref = O.scan_bf16(cu, *U.vec_bits(vecs), pool=pool.numpy(), slot_ids=ids,
                               scale=scale)
    assert np.all(np.isfinite(U.f64(y)))
    for s in range(len(ids)):
        sl = slice(int(cu[s]), int(cu[s + 1]))
        assert U.rel_l2(U.f64(y[sl]), y_ref[sl]) <= REL_L2
        assert U.rel_l2(U.f64(gpool[ids[s]]), h_ref[s]) <= REL_L2


@pytest.mark.parametrize("pattern", ["channels", "tokens"])
def test_slow_decay_long_sequence(dev, pattern):
    """Where state accumulates most: 4,096 tokens with no decay (w = 0) on half
    the key channels, or on every third token, from slot state, at the unit
    scale of the shipped fast path. The operands the kernel rounds to one bf16
    (A^, T) must keep the state and y within the parity bar over the whole
    length, per sequence; h as one bf16 in the A^ h product did not (y 1.7e-3
    against the bf16-rounded oracle, state 8e-4, on the "channels" pattern)."""
    H, S = 4, 4
    lens = [4096, 4096]
    cu = np.concatenate([[0], np.cumsum(lens)])
    T = int(cu[-1])
    gen = synthetic.make_generator(79)
    pool = torch.zeros((S + 1, H, 64, 64))
    pool[1:] = synthetic.initial_states((S, H, 64, 64), gen)
    ids = [3, 1]
    vecs = synthetic.wkv7_vectors((T, H, 64), gen)
    wmax = -synthetic.DECAY_SCALE
    if pattern == "channels":
        w = torch.where(torch.arange(64) % 2 == 0, 0.0, wmax).expand(T, H, 64)
    else:
        w = torch.where(torch.arange(T) % 3 == 0, 0.0, wmax)[:, None, None].expand(T, H, 64)
    vecs["w"] = w.to(torch.bfloat16).contiguous()
    gpool = pool.to(dev)
    y = ops.wkv7_prefill_varlen(gpool, ids, cu.tolist(), *(vecs[n].to(dev) for n in "rwkvab"))
    torch.cuda.synchronize()
    eh, ey = _check(pool.numpy(), ids, cu, U.vec_bits(vecs), gpool, y, zero_init=False)
    print(f"slow decay ({pattern}), 4096 tokens: worst state rel L2 {eh:.2e}, y {ey:.2e}")


@pytest.mark.parametrize("zero_init", [False, True])
@pytest.mark.parametrize("y_dtype", [torch.bfloat16, torch.float32])
def test_segmented_prefill_matches_oracle_and_one_pass(dev, zero_init, y_dtype):
    """Sequences cut into up to 4 segments that run side by side (transition
    runs from the identity, combined by linearity in the initial state) give
    the oracle's y and final states, and the one-pass kernel's to 1e-4 (the
    segments' own sub-chunk grids and the linear combination round differently;
    measured 1.9e-6 on the states, 3.5e-5 on an fp32 y); an empty sequence and
    a 10-token one (a single segment) ride along."""
    H, S = 4, 10
    lens = [700, 0, 10, 333]
    cu = np.concatenate([[0], np.cumsum(lens)])
    gen = synthetic.make_generator(61)
    pool = torch.zeros((S + 1, H, 64, 64))
    pool[1:] = synthetic.initial_states((S, H, 64, 64), gen)
    ids = [7, 2, 9, 4]
    vecs = synthetic.wkv7_vectors((int(cu[-1]), H, 64), gen)
    xs = [vecs[n].to(dev) for n in "rwkvab"]
    gpool = pool.to(dev)
    y = ops.wkv7_prefill_segments(gpool, ids, cu.tolist(), *xs, segments=4, zero_init=zero_init,
                                  out_dtype=y_dtype)
    torch.cuda.synchronize()
    _check(pool.numpy(), ids, cu, U.vec_bits(vecs), gpool, y, zero_init)
    others = [i for i in range(S + 1) if i not in ids]
    assert torch.equal(gpool[others].cpu(), pool[others])
    one = pool.to(dev)
    y1 = ops.wkv7_prefill_varlen(one, ids, cu.tolist(), *xs, zero_init=zero_init,
                                 out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert U.rel_l2(U.f64(gpool), U.f64(one)) <= 1e-4
    if y_dtype == torch.float32:
        assert U.rel_l2(U.f64(y), U.f64(y1)) <= 1e-4


def test_runner_segmented_prefill_matches_one_pass(dev):
    """WKV7Runner with prefill_segments: chunks of at least 2048 tokens run
    segmented, shorter ones in one pass; every layer's y and the slot state
    agree with the one-pass runner to 1e-4 (measured 1.6e-5 on y)."""
    lay = RWKV7StateLayout(n_layer=2, hidden_size=256, num_heads=4, head_dim=64, head_v_dim=64,
                           dtype=torch.bfloat16)
    T = 2048 + 300
    gen = synthetic.make_generator(67)
    inputs = [synthetic.order(synthetic.wkv7_vectors((T, 4, 64), gen, device=dev))
              for _ in range(2)]
    outs, finals = [], []
    for segs in (None, 4, "auto"):
        bank = RWKV7StateBank(lay, num_slots=3, device=dev)
        bank.wkv[:, 2].normal_(0.0, 0.1, generator=torch.Generator(device=dev).manual_seed(68))
        run = WKV7Runner(bank, prefill_chunk=2048, prefill_segments=segs)
        ys = run.prefill(inputs, {"wkv": 2, "shift": 2}, out_dtype=torch.float32)
        outs.append(torch.stack(ys))
        finals.append(bank.wkv[:, 2].clone())
    for i in (1, 2):
        assert U.rel_l2(U.f64(outs[i]), U.f64(outs[0])) <= 1e-4
        assert U.rel_l2(U.f64(finals[i]), U.f64(finals[0])) <= 1e-4


def test_fla_signature_long_single_sequence_runs_segmented(dev):
    """chunk_rwkv7 with one long sequence picks the segmented form (few busy
    compute units) and still matches the oracle, from an initial state and
    from zero."""
    B, T, H = 1, 2100, 4
    assert ops.auto_segments(H, [T], dev) > 1 and ops.auto_segments(H, [500], dev) == 1
    gen = synthetic.make_generator(71)
    vecs = synthetic.wkv7_vectors((B, T, H, 64), gen)
    h0 = synthetic.initial_states((B, H, 64, 64), gen)
    xs = [vecs[n].to(dev) for n in "rwkvab"]
    bits = [U.bits(vecs[n][0]) for n in "rwkvab"]
    for init in (h0, None):
        o, hT = ops.chunk_rwkv7(*xs, scale=1.0, initial_state=None if init is None else init.to(dev))
        y_ref, h_ref = O.scan_bf16(np.array([0, T]), *bits,
                                   pool=None if init is None else init.numpy(),
                                   slot_ids=None if init is None else [0])
        assert U.rel_l2(U.f64(hT), h_ref) <= REL_L2
        assert U.rel_l2(U.f64(o[0]), O.round_f64_to_bf16(y_ref)) <= REL_L2


@pytest.mark.parametrize("chunk,segments", [(512, None), (4096, "auto")])
def test_runner_prefill_matches_oracle(dev, chunk, segments):
    """WKV7Runner.prefill (wkvm/runner/runner.py:41-63): one 4,096-token
    request at the 1.5B head count, two layers, from a non-zero slot state,
    in 512-token chunks re-entering through the slot (and in one 4,096-token
    chunk that runs segmented); every layer's y and the final slot state
    against the float64 oracle, the pad row and the other slots untouched."""
    Lr, H, T = 2, 32, 4096
    lay = RWKV7StateLayout(n_layer=Lr, hidden_size=H * 64, num_heads=H, head_dim=64,
                           head_v_dim=64, dtype=torch.bfloat16)
    bank = RWKV7StateBank(lay, num_slots=4, device=dev)
    gen = synthetic.make_generator(421)
    bank.wkv[:, 1:] = synthetic.initial_states((Lr, 4, H, 64, 64), gen).to(dev)
    before = bank.wkv.cpu()
    vecs = [synthetic.wkv7_vectors((T, H, 64), gen) for _ in range(Lr)]
    run = WKV7Runner(bank, prefill_chunk=chunk, prefill_segments=segments)
    ys = run.prefill([[v[n].to(dev) for n in "rwkvab"] for v in vecs], {"wkv": 3, "shift": 3})
    torch.cuda.synchronize()
    for layer in range(Lr):
        y_ref, h_ref = O.scan_bf16(np.array([0, T]), *U.vec_bits(vecs[layer]),
                                   pool=before[layer].numpy(), slot_ids=[3])
        eh = U.rel_l2(U.f64(bank.wkv[layer, 3]), h_ref[0])
        ey = U.rel_l2(U.f64(ys[layer]), O.round_f64_to_bf16(y_ref))
        print(f"layer {layer}: state rel L2 {eh:.2e}, y {ey:.2e}")
        assert eh <= REL_L2 and ey <= REL_L2
    assert torch.equal(bank.wkv[:, [0, 1, 2, 4]].cpu(), before[:, [0, 1, 2, 4]])


@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")
def test_cached_offsets_under_graph_capture(dev):
    """Host offsets are uploaded once and cached per (device, offsets). A
    launch captured in a HIP graph reads the cached copy on every replay, so
    that copy must outlive the cache's eviction of it; offsets that are not
    cached yet cannot be uploaded under capture and raise before any launch
    is recorded. Every replay (with eager launches of other offsets between,
    which evict the entry) equals the eager result."""
    H, S = 4, 8
    lens = [37, 200, 5]
    cu = np.concatenate([[0], np.cumsum(lens)]).tolist()
    gen = synthetic.make_generator(101)
    pool0 = synthetic.initial_states((S + 1, H, 64, 64), gen).to(dev)
    xs = [x.to(dev) for x in synthetic.order(synthetic.wkv7_vectors((cu[-1], H, 64), gen))]
    ids = torch.tensor([2, 5, 7], dtype=torch.int32, device=dev)
    y = torch.empty((cu[-1], H, 64), dtype=torch.bfloat16, device=dev)
    pool = pool0.clone()
    ops.wkv7_prefill_varlen(pool, ids, cu, *xs, out=y)  # caches the plan of `cu`
    torch.cuda.synchronize()
    ref_y, ref_pool = y.clone(), pool.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.wkv7_prefill_varlen(pool, ids, cu, *xs, out=y)
    other = [0, 1, 2, 3]  # a one-token-per-sequence batch over slots 1..3
    for rep in range(3):
        # more distinct offsets than the cache holds: the captured entry is evicted
        for n in range(ops._PLAN_CACHE_SIZE + 8):
            ops._device_plan([0, 1000 + n, 2000 + 1000 * rep + n], dev)
        pool.copy_(pool0)
        y.fill_(7.0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref_y), f"replay {rep}: y differs"
        assert torch.equal(pool, ref_pool), f"replay {rep}: state differs"
        # eager work between replays on the same tensors
        tmp = pool0.clone()
        ops.wkv7_prefill_varlen(tmp, [1, 2, 3], other, *(x[:3] for x in xs))
    g2 = torch.cuda.CUDAGraph()
    fresh = [0, 11, 12, cu[-1]]
    with pytest.raises(RuntimeError, match="graph capture"):
        with torch.cuda.graph(g2):
            ops.wkv7_prefill_varlen(pool, ids, fresh, *xs, out=y)
