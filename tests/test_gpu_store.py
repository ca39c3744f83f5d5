"""StateStore HOT <-> WARM <-> COLD on the GPU (wkv7_slot_transfer DMA copies).

The bar is bit-exactness: a saved WARM record equals the slot's rows of every
layer as torch slicing reads them (``bank.wkv[:, slot]``,
``bank.shift[:, :, slot]``, the reference's snapshot views,
wkvm/store.py:130-131); a load writes exactly those bytes into the target slot
and leaves every other row, pad row 0 included, untouched
(tests/test_store_gpu.py of the reference checks the same through
token-identical continuations); the round trip through COLD and through a
fresh store rebuilt from the index is exact; a rejected load moves no byte."""

from __future__ import annotations

import pytest
import torch

from wkvm_amd import ops, synthetic
from wkvm_amd.layout import RWKV7StateLayout
from wkvm_amd.state import RWKV7StateBank
from wkvm_amd.store import FingerprintMismatch, StateStore

pytestmark = pytest.mark.gpu


def _bank(dev, shape="0.1B", slots=6, seed=21):
    layout = RWKV7StateLayout.for_shape(shape)
    bank = RWKV7StateBank(layout, slots, device=dev)
    g = synthetic.make_generator(seed, dev)
    bank.wkv.normal_(0.0, 1.0, generator=g)
    bank.shift.copy_(torch.randn(bank.shift.shape, device=dev, generator=g).to(bank.shift.dtype))
    return bank


def test_save_is_the_slot_view(dev, tmp_path):
    bank = _bank(dev)
    st = StateStore(bank, tmp_path)
    h = st.save("s", {"wkv": 3, "shift": 4}, 5, [1, 2, 3, 4, 5, 6])
    t = st.host_tensors(h)
    assert t["wkv"].is_pinned() and t["shift"].is_pinned()
    assert torch.equal(t["wkv"], bank.wkv[:, 3].cpu())
    assert torch.equal(t["shift"], bank.shift[:, :, 4].cpu())
    rec = st.get(h)
    assert (rec.num_computed_tokens, rec.token_ids) == (5, (1, 2, 3, 4, 5, 6))


def test_load_writes_only_the_target_slot(dev, tmp_path):
    bank = _bank(dev)
    st = StateStore(bank, tmp_path)
    h = st.save("s", {"wkv": 2, "shift": 2}, 0, [0])
    saved = {k: v.clone() for k, v in st.host_tensors(h).items()}
    before_w, before_s = bank.wkv.clone(), bank.shift.clone()
    st.load(h, {"wkv": 5, "shift": 1})
    assert torch.equal(bank.wkv[:, 5].cpu(), saved["wkv"])
    assert torch.equal(bank.shift[:, :, 1].cpu(), saved["shift"])
    keep_w = [i for i in range(bank.num_slots + 1) if i != 5]
    keep_s = [i for i in range(bank.num_slots + 1) if i != 1]
    assert torch.equal(bank.wkv[:, keep_w], before_w[:, keep_w])
    assert torch.equal(bank.shift[:, :, keep_s], before_s[:, :, keep_s])


def test_cold_roundtrip_and_rebuild(dev, tmp_path):
    bank = _bank(dev, shape="1.5B", slots=3)
    st = StateStore(bank, tmp_path)
    h = st.save("durable", {"wkv": 1, "shift": 1}, 3, [7, 8, 9, 10])
    ref_w, ref_s = bank.wkv[:, 1].clone(), bank.shift[:, :, 1].clone()
    st.evict(h)  # persist + drop WARM
    assert h not in st._warm
    fresh = StateStore(bank, tmp_path)  # index + safetensors only
    assert h in {r.handle for r in fresh.list()}
    bank.wkv[:, 3].zero_()
    bank.shift[:, :, 3].zero_()
    fresh.load(h, {"wkv": 3, "shift": 3})
    assert torch.equal(bank.wkv[:, 3], ref_w)
    assert torch.equal(bank.shift[:, :, 3], ref_s)


def test_fork_and_mutate_then_load(dev, tmp_path):
    bank = _bank(dev)
    st = StateStore(bank, tmp_path)
    parent = st.save("p", {"wkv": 1, "shift": 1}, 0, [0])
    ref_w, ref_s = bank.wkv[:, 1].clone(), bank.shift[:, :, 1].clone()
    child = st.fork(parent, "c")
    mut = st.mutate(parent, "decay", {"alpha": 0.25})
    st.load(child, {"wkv": 2, "shift": 2})
    st.load(mut, {"wkv": 3, "shift": 3})
    assert torch.equal(bank.wkv[:, 2], ref_w) and torch.equal(bank.shift[:, :, 2], ref_s)
    assert torch.equal(bank.wkv[:, 3], ref_w * 0.25)  # exact: fp32 multiply by 0.25
    assert torch.equal(bank.shift[:, :, 3], ref_s)
    st.load(parent, {"wkv": 4, "shift": 4})  # parent untouched by fork and mutate
    assert torch.equal(bank.wkv[:, 4], ref_w)


def test_rejected_load_moves_nothing(dev, tmp_path):
    bank = _bank(dev)
    st = StateStore(bank, tmp_path)
    h = st.save("fp", {"wkv": 1, "shift": 1}, 0, [0])
    object.__setattr__(st.get(h), "fingerprint", "bogus")
    before_w, before_s = bank.wkv.clone(), bank.shift.clone()
    with pytest.raises(FingerprintMismatch):
        st.load(h, {"wkv": 2, "shift": 2})
    with pytest.raises(ValueError):
        ops.slot_from_host(bank.wkv, bank.num_slots + 1, 1, st.host_tensors(h)["wkv"])
    torch.cuda.synchronize()
    assert torch.equal(bank.wkv, before_w) and torch.equal(bank.shift, before_s)


@pytest.mark.parametrize("staged", [False, True])
def test_transfer_paths_bit_exact(dev, staged):
    """Both transfer paths (strided DMA; device gather/scatter through a
    staging buffer plus a contiguous DMA) move exactly the slot view's bytes,
    for fp32 rows, bf16 rows and rows whose size allows only 2-byte vectors."""
    g = synthetic.make_generator(5, dev)
    cases = [(torch.randn(3, 7, 4, 64, 64, device=dev, generator=g), 1),
             (torch.randn(2, 2, 9, 96, device=dev, generator=g).to(torch.bfloat16), 2),
             (torch.randn(4, 5, 33, device=dev, generator=g).to(torch.bfloat16), 1)]
    for t, dim in cases:
        slot = t.shape[dim] - 2
        view = t.select(dim, slot)
        nbytes = view.numel() * t.element_size()
        staging = torch.empty(nbytes + 64, dtype=torch.uint8, device=dev) if staged else None
        host = ops.slot_to_host(t, slot, dim, staging=staging)
        dense = torch.empty(view.shape, dtype=t.dtype, device=dev)
        ops.slot_gather_dense(t, slot, dim, dense)
        torch.cuda.synchronize(dev)
        assert torch.equal(host, view.cpu())
        assert torch.equal(dense, view)
        before = t.clone()
        src = torch.randn(view.shape, generator=torch.Generator().manual_seed(1)).to(t.dtype)
        src = src.pin_memory()
        ops.slot_from_host(t, 1, dim, src, staging=staging)
        torch.cuda.synchronize(dev)
        assert torch.equal(t.select(dim, 1).cpu(), src)
        keep = [i for i in range(t.shape[dim]) if i != 1]
        assert torch.equal(t.index_select(dim, torch.tensor(keep, device=dev)),
                           before.index_select(dim, torch.tensor(keep, device=dev)))
    small = torch.empty(16, dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError):
        ops.slot_to_host(cases[0][0], 1, 1, staging=small)
