"""StateStore restart recovery after a process is killed (CPU only).

The reference survives a kill -9 by rebuilding its store from the COLD index
(wkvm/store.py:275-296; the SIGKILL demo, experiments/wkvm_demo_video.py:463-493).
Here a child process builds a store and is SIGKILLed:
* right after ``persist``: a fresh store over the same directory holds the
  persisted record, byte for byte, with its lineage;
* in the middle of an index rewrite (killed between writing the temporary
  file and replacing ``index.json``): the index is still the previous complete
  version, so a restart sees every record up to the last finished write and
  nothing half-written."""

from __future__ import annotations

import os
import signal
import subprocess
import sys
import textwrap

import torch

from wkvm_amd.layout import RWKV7StateLayout
from wkvm_amd.state import RWKV7StateBank
from wkvm_amd.store import StateStore

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = textwrap.dedent("""
    import os, signal, sys
    sys.path.insert(0, {root!r})
    import torch
    from wkvm_amd.layout import RWKV7StateLayout
    from wkvm_amd.state import RWKV7StateBank
    from wkvm_amd.store import StateStore

    layout = RWKV7StateLayout(n_layer=2, hidden_size=128, num_heads=2, head_dim=64,
                              head_v_dim=64, dtype=torch.bfloat16)
    bank = RWKV7StateBank(layout, 3, device="cpu")
    st = StateStore(bank, {store!r})

    def tensors(seed):
        g = torch.Generator().manual_seed(seed)
        return {{"wkv": torch.randn((2, 2, 64, 64), generator=g),
                 "shift": torch.randn((2, 2, 128), generator=g).to(torch.bfloat16)}}

    def put(name, seed, tokens):
        return st.save_host(name, tensors(seed), len(tokens) - 1, tokens)

    a = put("sess", 1, [5, 6, 7])
    st.persist(a)
    b = st.fork(a, "kid")
    if {mode!r} == "mid_index":
        import wkvm_amd.store as S
        def die(*args, **kwargs):
            os.kill(os.getpid(), signal.SIGKILL)
        S.os.replace = die      # killed after the temporary index is written
        c = put("late", 2, [1])
    os.kill(os.getpid(), signal.SIGKILL)
""")


def _tensors(seed):
    g = torch.Generator().manual_seed(seed)
    return {"wkv": torch.randn((2, 2, 64, 64), generator=g),
            "shift": torch.randn((2, 2, 128), generator=g).to(torch.bfloat16)}


def _bank():
    layout = RWKV7StateLayout(n_layer=2, hidden_size=128, num_heads=2, head_dim=64,
                              head_v_dim=64, dtype=torch.bfloat16)
    return RWKV7StateBank(layout, 3, device="cpu")


def _run_child(store_dir, mode):
    code = CHILD.format(root=ROOT, store=str(store_dir), mode=mode)
    proc = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                          timeout=120)
    assert proc.returncode == -signal.SIGKILL, proc.stderr


def test_kill_after_persist_rebuilds_from_index(tmp_path):
    _run_child(tmp_path, "after_persist")
    st = StateStore(_bank(), tmp_path)
    assert [r.handle for r in st.list()] == ["kid@0", "sess@0"]
    assert st.get("kid@0").parent == "sess@0"
    assert st.get("sess@0").token_ids == (5, 6, 7)
    got, want = st.host_tensors("sess@0"), _tensors(1)
    for k in ("wkv", "shift"):
        assert torch.equal(got[k], want[k])


def test_kill_mid_index_write_keeps_last_complete_index(tmp_path):
    _run_child(tmp_path, "mid_index")
    assert (tmp_path / "index.json.partial").exists()  # the interrupted write
    st = StateStore(_bank(), tmp_path)
    assert [r.handle for r in st.list()] == ["kid@0", "sess@0"]  # no "late@0"
    for k in ("wkv", "shift"):
        assert torch.equal(st.host_tensors("sess@0")[k], _tensors(1)[k])
    # the store keeps working after the restart
    st.save_host("late", _tensors(2), 0, [1])
    st.persist("late@0")
    assert [r.handle for r in StateStore(_bank(), tmp_path).list()] == ["kid@0", "late@0",
                                                                          "sess@0"]
