"""HIP-graph decode step: replays of the captured step must equal the eager
launches bit for bit (same kernels, same inputs), across several replays with
different slot batches and with eager GPU work and synchronisations between
them. The graph holds no memset nodes (the decode kernels need none)."""

from __future__ import annotations

import pytest
import torch

from wkvm_amd import synthetic
from wkvm_amd.graph import DecodeGraph
from wkvm_amd.layout import RWKV7StateLayout
from wkvm_amd.state import RWKV7StateBank

pytestmark = pytest.mark.gpu


def _banks(dev, L=3, H=4, S=24, seed=11):
    layout = RWKV7StateLayout(n_layer=L, hidden_size=H * 64, num_heads=H, head_dim=64,
                              head_v_dim=64, dtype=torch.bfloat16)
    a = RWKV7StateBank(layout, S, device=dev)
    g = synthetic.make_generator(seed, dev)
    a.wkv.normal_(0.0, 0.1, generator=g)
    b = RWKV7StateBank(layout, S, device=dev)
    b.wkv.copy_(a.wkv)
    return layout, a, b


@pytest.mark.parametrize("y_dtype", [torch.bfloat16, torch.float32])
def test_graph_replays_match_eager(dev, y_dtype):
    layout, eager, graphed = _banks(dev)
    L, H, B = layout.n_layer, layout.num_heads, 5
    dg = DecodeGraph(graphed, B, out_dtype=y_dtype)
    gcpu = synthetic.make_generator(12)
    gdev = synthetic.make_generator(13, dev)
    for step in range(4):
        slots = synthetic.active_slots(graphed.num_slots, B, gcpu)
        xs = [synthetic.order(synthetic.wkv7_vectors((B, H, 64), gdev)) for _ in range(L)]
        y_eager = torch.stack([eager.decode_wkv(l, [{"wkv": s} for s in slots], *xs[l],
                                                out_dtype=y_dtype) for l in range(L)])
        torch.cuda.synchronize()
        y_graph = dg.step([{"wkv": s, "shift": s} for s in slots], xs)
        torch.cuda.synchronize()
        assert torch.equal(y_graph, y_eager), f"step {step}: y differs"
        assert torch.equal(graphed.wkv, eager.wkv), f"step {step}: state differs"
        # unrelated eager work between replays
        scratch = torch.randn(1 << 16, device=dev).sum()
        torch.cuda.synchronize()
        del scratch


def test_graph_replays_match_oracle(dev):
    """DecodeGraph replays (the role of the reference's GraphedDecode,
    experiments/m2_engine_bench.py:44-131) at the 1.5B head count: three
    replays with different slot batches, every layer's state and y checked
    against the float64 oracle from the state before the replay."""
    import numpy as np

    import oracle as O
    from tests import util as U

    layout, _, graphed = _banks(dev, L=2, H=32, S=96, seed=21)
    L, H, B = layout.n_layer, layout.num_heads, 48
    dg = DecodeGraph(graphed, B, out_dtype=torch.float32)
    gcpu = synthetic.make_generator(22)
    for step in range(3):
        slots = synthetic.active_slots(graphed.num_slots, B, gcpu)
        vecs = [synthetic.wkv7_vectors((B, H, 64), gcpu) for _ in range(L)]
        before = graphed.wkv.cpu().numpy()
        y = dg.step(slots, [[v[n].to(dev) for n in "rwkvab"] for v in vecs])
        torch.cuda.synchronize()
        for layer in range(L):
            y_ref, h_ref = O.scan_bf16(np.arange(B + 1), *U.vec_bits(vecs[layer]),
                                       pool=before[layer], slot_ids=slots)
            assert U.normwise_max(U.f64(graphed.wkv[layer, slots]), h_ref) <= 1e-5, step
            assert U.normwise_max(U.f64(y[layer]), y_ref, tile_dims=1) <= 1e-5, step
        idle = sorted(set(range(graphed.num_slots + 1)) - set(slots))
        assert np.array_equal(graphed.wkv[:, idle].cpu().numpy(), before[:, idle])


def test_graph_rejects_wrong_batch(dev):
    _, _, graphed = _banks(dev)
    dg = DecodeGraph(graphed, 3)
    with pytest.raises(ValueError):
        dg.set_slots([1, 2])
    with pytest.raises(ValueError):
        dg.set_slots([1, 1, 2])
    with pytest.raises(ValueError):
        dg.set_slots([1, 2, graphed.num_slots + 1])
