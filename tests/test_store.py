"""StateStore host logic (no GPU): record lineage, the JSON index and
restart persistence, the COLD safetensors format, the model fingerprint and
the mutation rules' arithmetic. The HOT <-> WARM transfers need the GPU and
are covered by test_gpu_store.py.

Pinned against the reference's behaviour (wkvm/store.py): the fingerprint is
the sha256 of the same key string; handles are ``name@version``; COLD files
are the handle with '@' replaced by '_v' plus ``.safetensors``, holding
tensors "wkv" and "shift"; the
index maps handles to record fields plus a ``cold`` flag; ``decay`` is an
fp32 multiply of wkv only; ``merge`` is (1 - w) a + w b in fp32 with one
rounding per operation, cast back to each family's dtype."""

from __future__ import annotations

import hashlib
import json

import numpy as np
import pytest
import torch
from safetensors.torch import load_file

import oracle as O
from wkvm_amd.layout import RWKV7StateLayout
from wkvm_amd.state import RWKV7StateBank
from wkvm_amd.store import FingerprintMismatch, StateRecord, StateStore, rule_decay


def _bank(n_layer=2, heads=2, slots=3):
    layout = RWKV7StateLayout(n_layer=n_layer, hidden_size=heads * 64, num_heads=heads,
                              head_dim=64, head_v_dim=64, dtype=torch.bfloat16)
    return RWKV7StateBank(layout, slots, device="cpu")


def _tensors(bank, seed):
    g = torch.Generator().manual_seed(seed)
    L, H, D = bank.layout.n_layer, bank.layout.num_heads, bank.layout.hidden_size
    return {"wkv": torch.randn((L, H, 64, 64), generator=g),
            "shift": torch.randn((L, 2, D), generator=g).to(torch.bfloat16)}


def _put(store, name, tensors, tokens=(1, 2, 3)):
    return store.save_host(name, tensors, len(tokens) - 1, list(tokens))


def test_fingerprint_is_the_reference_key_hash(tmp_path):
    bank = RWKV7StateBank(RWKV7StateLayout.for_shape("1.5B"), 1, device="cpu")
    key = "rwkv7:L24:wkv(32, 64, 64):shift(2048,):torch.bfloat16"
    assert StateStore(bank, tmp_path).fingerprint == hashlib.sha256(key.encode()).hexdigest()[:16]


def test_versions_lineage_and_index_rebuild(tmp_path):
    bank = _bank()
    st = StateStore(bank, tmp_path)
    h0 = _put(st, "sess", _tensors(bank, 0))
    h1 = _put(st, "sess", _tensors(bank, 1))
    assert (h0, h1) == ("sess@0", "sess@1")
    child = st.fork(h1, "kid")
    assert child == "kid@0" and st.get(child).parent == h1
    assert st.host_tensors(child) is st.host_tensors(h1)  # fork moves no bytes
    mut = st.mutate(h0, "decay", {"alpha": 0.5})
    rec = st.get(mut)
    assert (mut, rec.parent, rec.rule, rec.rule_params) == ("sess@2", h0, "decay", {"alpha": 0.5})
    st.persist(h1)
    idx = json.loads((tmp_path / "index.json").read_text())
    assert set(idx) == {h0, h1, child, mut}
    assert idx[h1]["cold"] and not idx[h0]["cold"]
    assert idx[h1]["token_ids"] == [1, 2, 3]
    # a fresh store over the same directory: index + safetensors only
    st2 = StateStore(bank, tmp_path)
    assert [r.handle for r in st2.list()] == [child, h0, h1, mut]
    assert st2.get(mut) == rec
    for k, v in st.host_tensors(h1).items():
        assert torch.equal(st2.host_tensors(h1)[k], v)
    with pytest.raises(KeyError):
        st2.host_tensors(h0)  # WARM-only record of the old process
    st2.delete(h1)
    assert not (tmp_path / "sess_v1.safetensors").exists()
    assert h1 not in json.loads((tmp_path / "index.json").read_text())


def test_cold_file_format(tmp_path):
    bank = _bank()
    st = StateStore(bank, tmp_path)
    t = _tensors(bank, 3)
    h = _put(st, "fmt", t)
    path = st.persist(h)
    assert path.name == "fmt_v0.safetensors"
    assert st.persist(h) == path  # idempotent
    data = load_file(str(path))
    assert set(data) == {"wkv", "shift"}
    assert data["wkv"].dtype == torch.float32 and tuple(data["wkv"].shape) == (2, 2, 64, 64)
    assert data["shift"].dtype == torch.bfloat16 and tuple(data["shift"].shape) == (2, 2, 128)
    assert torch.equal(data["wkv"], t["wkv"]) and torch.equal(data["shift"], t["shift"])
    st.evict(h)
    assert h not in st._warm and torch.equal(st.host_tensors(h)["wkv"], t["wkv"])


def test_decay_rule_arithmetic():
    bank = _bank()
    t = _tensors(bank, 4)
    out = rule_decay({k: v.clone() for k, v in t.items()}, {"alpha": 0.2})
    expect = t["wkv"].numpy() * np.float32(0.2)
    assert np.array_equal(out["wkv"].numpy(), expect)
    assert torch.equal(out["shift"], t["shift"])
    out = rule_decay({k: v.clone() for k, v in t.items()}, {})
    assert np.array_equal(out["wkv"].numpy(), t["wkv"].numpy() * np.float32(0.9))


def test_merge_rule_arithmetic(tmp_path):
    bank = _bank()
    st = StateStore(bank, tmp_path)
    a, b = _tensors(bank, 5), _tensors(bank, 6)
    ha, hb = _put(st, "a", a), _put(st, "b", b)
    hm = st.mutate(ha, "merge", {"other": hb, "weight": 0.3})
    m = st.host_tensors(hm)
    w1, w = np.float32(1.0 - 0.3), np.float32(0.3)
    assert np.array_equal(m["wkv"].numpy(), w1 * a["wkv"].numpy() + w * b["wkv"].numpy())
    sa = O.bf16_bits_to_f64(a["shift"].view(torch.int16).numpy().view(np.uint16)).astype(np.float32)
    sb = O.bf16_bits_to_f64(b["shift"].view(torch.int16).numpy().view(np.uint16)).astype(np.float32)
    expect_bits = O.f32_to_bf16_bits(w1 * sa + w * sb)
    assert np.array_equal(m["shift"].view(torch.int16).numpy().view(np.uint16), expect_bits)
    assert st.get(hm).parent == ha and st.get(hm).rule == "merge"


def test_errors(tmp_path):
    bank = _bank()
    st = StateStore(bank, tmp_path)
    h = _put(st, "x", _tensors(bank, 7))
    with pytest.raises(KeyError):
        st.get("nope@0")
    with pytest.raises(KeyError):
        st.mutate(h, "no-such-rule")
    object.__setattr__(st.get(h), "fingerprint", "bogus")
    with pytest.raises(FingerprintMismatch):
        st.load(h, {"wkv": 1, "shift": 1})
    with pytest.raises(ValueError):  # transfers need a GPU bank
        StateStore(bank, tmp_path / "other").save("y", {"wkv": 1, "shift": 1}, 0, [0])


def test_index_rows_and_version_numbers(tmp_path):
    """Each index row holds exactly the record fields plus ``cold`` (what the
    reference's reader rebuilds a record from), and an index in that layout
    written by hand loads here. A name's next version is 1 + its highest
    live version, so deleting the newest version frees its number."""
    bank = _bank()
    st = StateStore(bank, tmp_path)
    h0 = _put(st, "s", _tensors(bank, 0))
    h1 = _put(st, "s", _tensors(bank, 1))
    row = json.loads((tmp_path / "index.json").read_text())[h1]
    assert set(row) == {f for f in StateRecord.__dataclass_fields__} | {"cold"}
    st.delete(h1)
    assert _put(st, "s", _tensors(bank, 2)) == "s@1"
    st.delete("s@7")  # unknown: no-op
    assert [r.handle for r in st.list()] == [h0, "s@1"]
    other = tmp_path / "other"
    other.mkdir()
    hand = {"x@3": {"name": "x", "version": 3, "fingerprint": st.fingerprint,
                    "num_computed_tokens": 2, "token_ids": [7, 8, 9], "parent": None,
                    "rule": "decay", "rule_params": {"alpha": 0.5}, "cold": False}}
    (other / "index.json").write_text(json.dumps(hand))
    st2 = StateStore(bank, other)
    rec = st2.get("x@3")
    assert rec.token_ids == (7, 8, 9) and rec.rule_params == {"alpha": 0.5}
    assert st2._next_version("x") == 4


def test_save_host_validation_warm_view_and_shared_forks(tmp_path):
    bank = _bank()
    st = StateStore(bank, tmp_path)
    t = _tensors(bank, 8)
    with pytest.raises(ValueError):
        st.save_host("bad", {"wkv": t["wkv"][:1], "shift": t["shift"]}, 0, [0])
    with pytest.raises(ValueError):
        st.save_host("bad", {"wkv": t["wkv"].double(), "shift": t["shift"]}, 0, [0])
    h = _put(st, "p", t)
    kid = st.fork(h, "kid")
    assert set(st._warm) == {h, kid}
    st.evict(h)
    assert set(st._warm) == {kid}
    st.delete(h)  # the fork keeps the shared tensors
    assert torch.equal(st.host_tensors(kid)["wkv"], t["wkv"])
    assert not (tmp_path / "p_v0.safetensors").exists()


def test_cold_file_name_of_a_name_with_at_sign(tmp_path):
    """The COLD file name is the handle with every '@' replaced by '_v'
    (wkvm/store.py:257-258), so a name that holds '@' maps to the file the
    reference writes: 'u@h' version 1 -> 'u_vh_v1.safetensors'. A directory
    laid out that way (index + file, written here by hand) opens and loads."""
    bank = _bank()
    st = StateStore(bank, tmp_path)
    t = _tensors(bank, 9)
    st.save_host("u@h", t, 2, [4, 5, 6])
    h = _put(st, "u@h", t)
    assert h == "u@h@1"
    path = st.persist(h)
    assert path.name == "u_vh_v1.safetensors" and path.exists()
    assert not list(tmp_path.glob("*.partial"))  # the temporary name was renamed away
    st.delete(h)
    assert not path.exists()

    ref_dir = tmp_path / "ref"
    ref_dir.mkdir()
    from safetensors.torch import save_file
    save_file({k: v.contiguous() for k, v in t.items()}, str(ref_dir / "u_vh_v0.safetensors"))
    row = {"name": "u@h", "version": 0, "fingerprint": st.fingerprint,
           "num_computed_tokens": 2, "token_ids": [4, 5, 6], "parent": None, "rule": None,
           "rule_params": {}, "cold": True}
    (ref_dir / "index.json").write_text(json.dumps({"u@h@0": row}))
    st2 = StateStore(bank, ref_dir)
    got = st2.host_tensors("u@h@0")
    assert torch.equal(got["wkv"], t["wkv"]) and torch.equal(got["shift"], t["shift"])
