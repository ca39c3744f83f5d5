"""Config 4 against the oracle at its own workload: one scheduler step of the
1.5B shape (H = 32) over a 1024-slot pool with 64 prefill rows of seeded
lengths U[1, 2048] and 448 decode rows, through WKV7Runner.mixed_step with
the decode launches on a side stream (the schedule bench.py times).

The reference runs such a step as per-request prefill plus one batched decode
(wkvm/engine.py:142-170) over ragged offsets (wkvm/core/mixed_batch.py:
213-230); each row is therefore checked against the float64 oracle on its
own: prefill rows (y and final state, relative L2 <= 1e-3 per row, a bf16 y
against the rounded oracle), decode rows (state normwise <= 1e-5 per (slot,
head) tile; a bf16 y within that bar plus one ulp of its own rounding). Every other row of the pool, pad slot 0
included, must keep its bytes."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from tests import util as U
from wkvm_amd import synthetic
from wkvm_amd.layout import RWKV7StateLayout
from wkvm_amd.runner import WKV7Runner
from wkvm_amd.state import RWKV7StateBank

pytestmark = pytest.mark.gpu

L, H, S, NP, ND = 2, 32, 1024, 64, 448


@pytest.mark.parametrize("zero_init", [False, True])
def test_cfg4_mixed_step_matches_oracle(dev, zero_init):
    gen = synthetic.make_generator(401 + int(zero_init))
    slots = synthetic.active_slots(S, NP + ND, gen)
    pre, dec = slots[:NP], slots[NP:]
    lens = synthetic.ragged_lengths(NP, 1, 2048, gen)
    cu = np.concatenate([[0], np.cumsum(lens)])
    T = int(cu[-1])
    print(f"cfg4: {T} prefill tokens in {NP} rows, {ND} decode rows, zero_init={zero_init}",
          flush=True)
    lay = RWKV7StateLayout(n_layer=L, hidden_size=H * 64, num_heads=H, head_dim=64,
                           head_v_dim=64, dtype=torch.bfloat16)
    bank = RWKV7StateBank(lay, S, device=dev)
    gdev = synthetic.make_generator(411, dev)
    bank.wkv.normal_(0.0, 0.1, generator=gdev)
    dec_in = [synthetic.wkv7_vectors((ND, H, 64), gdev) for _ in range(L)]
    pre_in = [synthetic.wkv7_vectors((T, H, 64), gdev) for _ in range(L)]
    before = bank.wkv.cpu()
    run = WKV7Runner(bank)
    dys, pys = run.mixed_step([{"wkv": s, "shift": s} for s in dec], [synthetic.order(x) for x in dec_in],
                              [{"wkv": s, "shift": s} for s in pre], lens,
                              [synthetic.order(x) for x in pre_in], zero_init=zero_init,
                              concurrent=True)
    torch.cuda.synchronize()
    after = bank.wkv.cpu()
    untouched = sorted(set(range(S + 1)) - set(slots))
    assert 0 in untouched
    assert torch.equal(after[:, untouched], before[:, untouched])
    for layer in range(L):
        pool_np = before[layer].numpy()
        # decode rows, one step each from their slot state
        y_ref, h_ref = O.scan_bf16(np.arange(ND + 1), *U.vec_bits(dec_in[layer]), pool=pool_np,
                                   slot_ids=dec)
        err = U.normwise_max(after[layer, dec].double().numpy(), h_ref)
        excess = U.bf16_y_excess(U.bits(dys[layer]), y_ref)
        assert err <= 1e-5, f"layer {layer}: decode state normwise {err:.2e}"
        assert excess <= 1, f"layer {layer}: decode bf16 y at {excess:.2f} x its bar"
        # prefill rows, each from its slot state (or zero)
        y_ref, h_ref = O.scan_bf16(cu, *U.vec_bits(pre_in[layer]),
                                   pool=None if zero_init else pool_np,
                                   slot_ids=None if zero_init else pre)
        y_cmp = O.round_f64_to_bf16(y_ref)
        del y_ref
        yv = U.f64(pys[layer])
        hs = after[layer, pre].double().numpy()
        worst_h = max(U.rel_l2(hs[s], h_ref[s]) for s in range(NP))
        worst_y = max(U.rel_l2(yv[cu[s]:cu[s + 1]], y_cmp[cu[s]:cu[s + 1]]) for s in range(NP))
        print(f"layer {layer}: decode state {err:.2e}, y {excess:.2f} x bar; prefill worst state "
              f"rel L2 {worst_h:.2e}, worst y {worst_y:.2e}", flush=True)
        assert worst_h <= 1e-3 and worst_y <= 1e-3
        del y_cmp, yv
