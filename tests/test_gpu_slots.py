"""Slot copy / zero / gather / scatter kernels: bit-exact against the
reference's torch slot views (wkvm/runner/state.py:50-97, wkvm/store.py:130-152)
and the fork invariants (wkvm/core/arena.py:82-93; tests/test_store_gpu.py:107-126
of the reference for isolation)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from wkvm_amd import ops, synthetic
from wkvm_amd.layout import RWKV7StateLayout
from wkvm_amd.state import RWKV7StateBank

pytestmark = pytest.mark.gpu


def _small_bank(dev, head_dim=32):
    # The reference's own bank test layout (tests/test_rwkv7_gpu.py:74-80).
    layout = RWKV7StateLayout(n_layer=3, hidden_size=64, num_heads=2, head_dim=head_dim,
                              head_v_dim=head_dim, dtype=torch.bfloat16)
    return RWKV7StateBank(layout, num_slots=4, device=dev)


def test_gather_scatter_roundtrip(dev):
    """Mirrors TestStateBankRoundTrip.test_gather_scatter_roundtrip."""
    bank = _small_bank(dev)
    batch = [{"wkv": 2, "shift": 2}, {"wkv": 4, "shift": 4}]
    cache = bank.gather_cache(batch)
    for i in range(bank.layout.n_layer):
        cache[i]["recurrent_state"].normal_()
        cache[i]["conv_state"].normal_()
        cache[i]["ffn_state"].normal_()
    expected = [(cache[i]["recurrent_state"].clone(), cache[i]["conv_state"].clone(),
                 cache[i]["ffn_state"].clone()) for i in range(bank.layout.n_layer)]
    bank.scatter_cache(batch, cache)
    back = bank.gather_cache(batch)
    for i, (wkv, conv, ffn) in enumerate(expected):
        assert torch.equal(back[i]["recurrent_state"], wkv)
        assert torch.equal(back[i]["conv_state"], conv)
        assert torch.equal(back[i]["ffn_state"], ffn)
    # and the rows landed where index_copy_ would put them
    ids = torch.tensor([2, 4], device=dev)
    assert torch.equal(bank.wkv.index_select(1, ids), torch.stack([e[0] for e in expected]))


def test_scatter_leaves_other_slots_untouched(dev):
    """Mirrors TestStateBankRoundTrip.test_scatter_leaves_other_slots_untouched."""
    bank = _small_bank(dev)
    cache = bank.gather_cache([{"wkv": 3, "shift": 3}])
    for i in range(bank.layout.n_layer):
        cache[i]["recurrent_state"].fill_(1.0)
        cache[i]["conv_state"].fill_(1.0)
        cache[i]["ffn_state"].fill_(1.0)
    bank.scatter_cache([{"wkv": 3, "shift": 3}], cache)
    for s in (0, 1, 2, 4):
        assert bank.wkv[:, s].abs().sum().item() == 0.0, f"slot {s}"
        assert bank.shift[:, :, s].abs().sum().item() == 0.0, f"slot {s}"
    assert bank.wkv[:, 3].abs().sum().item() > 0.0


def test_scatter_of_replaced_cache_entries(dev):
    """A forward that replaces cache tensors (fla's Cache.update does) takes
    the per-layer path; bytes must still equal index_copy_."""
    bank = _small_bank(dev)
    batch = [{"wkv": 1, "shift": 1}, {"wkv": 3, "shift": 3}]
    cache = bank.gather_cache(batch)
    ref_wkv, ref_shift = bank.wkv.clone(), bank.shift.clone()
    ids = torch.tensor([1, 3], device=dev)
    for i in range(bank.layout.n_layer):
        st = torch.randn_like(cache[i]["recurrent_state"], dtype=torch.float64)
        conv = torch.randn_like(cache[i]["conv_state"])
        cache.update(recurrent_state=st, conv_state=conv, layer_idx=i)
        ref_wkv[i].index_copy_(0, ids, st.to(torch.float32))
        ref_shift[i, 0].index_copy_(0, ids, conv)
        ref_shift[i, 1].index_copy_(0, ids, cache[i]["ffn_state"])
    bank.scatter_cache(batch, cache)
    assert torch.equal(bank.wkv, ref_wkv)
    assert torch.equal(bank.shift, ref_shift)


def test_zero_slots(dev):
    bank = _small_bank(dev)
    bank.wkv.normal_()
    bank.shift.normal_()
    before_w, before_s = bank.wkv.clone(), bank.shift.clone()
    bank.zero_slots({"wkv": 2, "shift": 3})
    assert bank.wkv[:, 2].abs().sum().item() == 0.0
    assert bank.shift[:, :, 3].abs().sum().item() == 0.0
    keep_w = [s for s in range(5) if s != 2]
    keep_s = [s for s in range(5) if s != 3]
    assert torch.equal(bank.wkv[:, keep_w], before_w[:, keep_w])
    assert torch.equal(bank.shift[:, :, keep_s], before_s[:, :, keep_s])


def test_fork_is_bit_exact_and_isolated(dev):
    """CF8: dst bytes == src bytes, src unchanged, other rows unchanged, and a
    decode from dst equals a decode from src bit for bit."""
    layout = RWKV7StateLayout(n_layer=2, hidden_size=256, num_heads=4, head_dim=64,
                              head_v_dim=64, dtype=torch.bfloat16)
    bank = RWKV7StateBank(layout, num_slots=8, device=dev)
    bank.wkv.normal_()
    bank.shift.normal_()
    before_w, before_s = bank.wkv.clone(), bank.shift.clone()
    src = [{"wkv": 2, "shift": 2}, {"wkv": 2, "shift": 2}, {"wkv": 5, "shift": 5}]
    dst = [{"wkv": 7, "shift": 7}, {"wkv": 1, "shift": 1}, {"wkv": 8, "shift": 8}]
    bank.fork_slots(src, dst)
    exp_w = O.slot_copy_np(before_w.cpu().numpy(), 1, [2, 2, 5], [7, 1, 8])
    exp_s = O.slot_copy_np(before_s.view(torch.int16).cpu().numpy(), 2, [2, 2, 5], [7, 1, 8])
    assert np.array_equal(bank.wkv.cpu().numpy().view(np.uint32), exp_w.view(np.uint32))
    assert np.array_equal(bank.shift.view(torch.int16).cpu().numpy(), exp_s)
    # a decode from the fork equals a decode from its parent
    g = synthetic.make_generator(5)
    vecs = synthetic.order(synthetic.wkv7_vectors((1, 4, 64), g, device=dev))
    y_parent = bank.decode_wkv(0, [{"wkv": 5, "shift": 5}], *vecs, out_dtype=torch.float32)
    y_child = bank.decode_wkv(0, [{"wkv": 8, "shift": 8}], *vecs, out_dtype=torch.float32)
    assert torch.equal(y_parent, y_child)
    assert torch.equal(bank.wkv[0, 5], bank.wkv[0, 8])


def test_fork_rejects_overlap_and_duplicate_destinations(dev):
    bank = _small_bank(dev)
    with pytest.raises(ValueError, match="overlap"):
        bank.fork_slots([{"wkv": 1, "shift": 1}], [{"wkv": 1, "shift": 1}])
    with pytest.raises(ValueError, match="duplicate"):
        bank.fork_slots([{"wkv": 1, "shift": 1}, {"wkv": 2, "shift": 2}],
                        [{"wkv": 3, "shift": 3}, {"wkv": 3, "shift": 3}])
    with pytest.raises(ValueError, match="out of range"):
        bank.fork_slots([{"wkv": 1, "shift": 1}], [{"wkv": 5, "shift": 5}])


@pytest.mark.parametrize("row_elems,dtype", [(3, torch.bfloat16), (5, torch.float32),
                                             (7, torch.uint8), (1000, torch.bfloat16),
                                             (4096 + 3, torch.float32)])
def test_copy_odd_row_sizes_pick_narrower_vectors(dev, row_elems, dtype):
    g = torch.Generator(device=dev).manual_seed(row_elems)
    t = torch.randint(0, 100, (3, 9, row_elems), generator=g, device=dev).to(dtype)
    before = t.cpu().view(torch.uint8).numpy()   # raw bytes: [3, 9, row_bytes]
    ops.slot_copy(t, [0, 8, 4], t, [3, 3, 6], slot_dim=1)
    exp = O.slot_copy_np(before, 1, [3, 3, 6], [0, 8, 4])
    assert np.array_equal(t.cpu().view(torch.uint8).numpy(), exp)


def test_copy_between_tensors_gather_and_scatter(dev):
    g = torch.Generator(device=dev).manual_seed(1)
    bank = torch.randn((4, 10, 3, 8), generator=g, device=dev)
    stage = torch.empty((4, 5, 3, 8), device=dev)
    ids = [9, 0, 4, 4, 2]
    ops.slot_copy(stage, None, bank, ids, slot_dim=1)
    assert torch.equal(stage, bank.index_select(1, torch.tensor(ids, device=dev)))
    upd = torch.randn((4, 3, 3, 8), generator=g, device=dev)
    ref = bank.clone()
    ref.index_copy_(1, torch.tensor([1, 7, 3], device=dev), upd)
    ops.slot_copy(bank, [1, 7, 3], upd, None, slot_dim=1)
    assert torch.equal(bank, ref)


def test_fork_7b_shape_128_slots(dev):
    """Config 3's fork round at full size: 128 seeded sources into free slots of
    a 7B-shape pool (32 layers, 64 heads, 1153 slot rows: ~38.7 GB of wkv)."""
    lay = RWKV7StateLayout.for_shape("7B")
    S = 1152
    wkv = torch.empty((lay.n_layer, S + 1, *lay.wkv_shape), dtype=torch.float32, device=dev)
    shift = torch.empty((lay.n_layer, 2, S + 1, lay.hidden_size), dtype=torch.bfloat16, device=dev)
    g = torch.Generator(device=dev).manual_seed(3)
    wkv.normal_(generator=g)
    shift.normal_(generator=g)
    gen = synthetic.make_generator(3)
    live = synthetic.active_slots(1024, 1024, gen)
    src = [live[i] for i in torch.randperm(1024, generator=gen)[:128].tolist()]
    dst = list(range(1025, 1153))
    src_w = wkv[:, src].clone()
    src_s = shift[:, :, src].clone()
    keep = wkv[:, 1:1025].sum(dim=(2, 3, 4))
    ops.slot_copy(wkv, dst, wkv, src, slot_dim=1)
    ops.slot_copy(shift, dst, shift, src, slot_dim=2)
    assert torch.equal(wkv[:, dst], src_w)
    assert torch.equal(shift[:, :, dst], src_s)
    assert torch.equal(wkv[:, 1:1025].sum(dim=(2, 3, 4)), keep)
    del wkv, shift
    torch.cuda.empty_cache()
