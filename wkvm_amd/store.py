"""StateStore over the slot pool: named, versioned, forkable state handles in
three tiers, drop-in for wkvm/store.py.

* HOT  -- the session's slot rows in ``RWKV7StateBank`` (``wkv`` and ``shift``
  families, every layer).
* WARM -- pinned host tensors held here, one per family, shaped like the
  reference's (``wkv [L, H, 64, 64]`` fp32, ``shift [L, 2, D]`` model dtype).
* COLD -- one safetensors file per handle plus ``index.json`` under
  ``store_dir``, rewritten atomically; a new process rebuilds the store from
  the index alone.

Interface, record fields, handle strings (``name@version``), file names, the
index format and the model fingerprint follow the reference
(wkvm/store.py:39-57, 63-86, 108-176, 195-243) so that stores written by
either implementation load in the other. What changes is the HOT <-> WARM
path, where the reference copies a non-contiguous slot view with
``Tensor.copy_`` (wkvm/store.py:130-131, 151-152, 230-233): a save gathers
both families' strided slot rows into a device staging buffer
(``wkv7_slot_copy``) and then moves each to its pinned WARM tensor as one
contiguous DMA; a load is one strided host-to-device DMA per family straight
into the slot rows (``wkv7_slot_transfer``). Mutation rules act on WARM host tensors with the
reference's arithmetic: ``decay`` scales ``wkv`` (wkvm/store.py:298-305),
``merge`` blends two records in fp32 (wkvm/store.py:260-268).

Single-threaded and synchronous like the reference (wkvm/store.py:21-22):
transfers synchronise the device before returning.
"""

from __future__ import annotations

import hashlib
import json
import math
import os
from dataclasses import asdict, dataclass, field
from pathlib import Path
from typing import Callable

import torch

from . import ops
from .state import RWKV7StateBank

MutationRule = Callable[[dict[str, torch.Tensor], dict], dict[str, torch.Tensor]]

# slot dimension of each family in the bank (wkv [L, S+1, ...], shift [L, 2, S+1, D])
_SLOT_DIM = {"wkv": 1, "shift": 2}


@dataclass(frozen=True)
class StateRecord:
    """Metadata of one immutable snapshot (fields as wkvm/store.py:39-57)."""

    name: str
    version: int
    fingerprint: str
    num_computed_tokens: int
    token_ids: tuple[int, ...]
    parent: str | None = None
    rule: str | None = None
    rule_params: dict = field(default_factory=dict)

    @property
    def handle(self) -> str:
        return f"{self.name}@{self.version}"


class FingerprintMismatch(RuntimeError):
    """A record saved for a different model layout (wkvm/store.py:60-61)."""


def layout_fingerprint(bank: RWKV7StateBank) -> str:
    """Model binding of a record: a hash of the state layout, computed from
    the same key string as the reference (wkvm/store.py:80-84)."""
    lay = bank.layout
    key = (f"rwkv7:L{lay.n_layer}:wkv{tuple(lay.wkv_shape)}:shift{tuple(lay.shift_shape)}:"
           f"{lay.dtype}")
    return hashlib.sha256(key.encode()).hexdigest()[:16]


class StateStore:
    def __init__(self, bank: RWKV7StateBank, store_dir: str | Path) -> None:
        self.bank = bank
        self.store_dir = Path(store_dir)
        self.store_dir.mkdir(parents=True, exist_ok=True)
        self.fingerprint = layout_fingerprint(bank)
        self._warm: dict[str, dict[str, torch.Tensor]] = {}
        self._meta: dict[str, StateRecord] = {}
        self._cold: set[str] = set()
        self._rules: dict[str, MutationRule] = {}
        self._stage: torch.Tensor | None = None
        self.register_rule("decay", rule_decay)
        self.register_rule("merge", self._rule_merge)
        self._load_index()

    # -- records ---------------------------------------------------------------

    def _next_version(self, name: str) -> int:
        return 1 + max((r.version for r in self._meta.values() if r.name == name), default=-1)

    def get(self, handle: str) -> StateRecord:
        if handle not in self._meta:
            raise KeyError(f"unknown state handle {handle!r}")
        return self._meta[handle]

    def list(self) -> list[StateRecord]:
        return sorted(self._meta.values(), key=lambda r: (r.name, r.version))

    def _add(self, record: StateRecord, tensors: dict[str, torch.Tensor]) -> str:
        self._warm[record.handle] = tensors
        self._meta[record.handle] = record
        self._write_index()
        return record.handle

    # -- HOT <-> WARM ------------------------------------------------------------

    def _family(self, name: str) -> torch.Tensor:
        return self.bank.wkv if name == "wkv" else self.bank.shift

    def _staging(self) -> torch.Tensor:
        """Device buffer holding one slot's rows of both families (12.2 MiB
        at the 1.5B shape), allocated on first use: a save gathers the slot's
        strided rows into it and each family crosses the host link as one
        contiguous DMA."""
        if self._stage is None:
            nbytes = sum(-(-self._family(f).select(_SLOT_DIM[f], 0).numel()
                           * self._family(f).element_size() // 256) * 256
                         for f in ("wkv", "shift"))
            self._stage = torch.empty(nbytes, dtype=torch.uint8, device=self.bank.device)
        return self._stage

    def save(self, name: str, slots: dict[str, int], num_computed_tokens: int,
             token_ids: list[int], parent: str | None = None, rule: str | None = None,
             rule_params: dict | None = None) -> str:
        """Snapshot a session's HOT slot rows into a new WARM record: device
        gathers of both families into the staging buffer, one contiguous DMA
        per family, then one synchronise (wkvm/store.py:108-137)."""
        record = StateRecord(name=name, version=self._next_version(name),
                             fingerprint=self.fingerprint,
                             num_computed_tokens=num_computed_tokens,
                             token_ids=tuple(token_ids), parent=parent, rule=rule,
                             rule_params=rule_params or {})
        # Both families' rows are gathered into the staging buffer first, then
        # moved to the host back to back: one kernel -> DMA hand-off per save.
        staged = {}
        offset = 0
        staging = self._staging()
        for fam in ("wkv", "shift"):
            t = self._family(fam)
            shape = t.shape[:_SLOT_DIM[fam]] + t.shape[_SLOT_DIM[fam] + 1:]
            nbytes = math.prod(shape) * t.element_size()
            staged[fam] = staging[offset:offset + nbytes].view(t.dtype).view(shape)
            ops.slot_gather_dense(t, slots[fam], _SLOT_DIM[fam], staged[fam])
            offset += -(-nbytes // 256) * 256
        tensors = {}
        for fam in ("wkv", "shift"):
            tensors[fam] = torch.empty(staged[fam].shape, dtype=staged[fam].dtype,
                                       pin_memory=True)
            tensors[fam].copy_(staged[fam], non_blocking=True)
        torch.cuda.synchronize(self.bank.device)
        return self._add(record, tensors)

    def load(self, handle: str, slots: dict[str, int]) -> StateRecord:
        """Restore a record into allocated slots: one DMA per family, then one
        synchronise (wkvm/store.py:139-156). A fingerprint mismatch raises
        before any byte moves."""
        record = self.get(handle)
        if record.fingerprint != self.fingerprint:
            raise FingerprintMismatch(f"{handle}: saved for model {record.fingerprint}, "
                                      f"engine is {self.fingerprint}")
        tensors = self._tensors(handle)
        for fam in ("wkv", "shift"):
            ops.slot_from_host(self._family(fam), slots[fam], _SLOT_DIM[fam],
                               _pinned(tensors[fam]))
        torch.cuda.synchronize(self.bank.device)
        return record

    # -- lineage -----------------------------------------------------------------

    def fork(self, handle: str, new_name: str) -> str:
        """A new name sharing the parent's bytes: records are immutable, so no
        state data moves (wkvm/store.py:158-176)."""
        parent = self.get(handle)
        record = StateRecord(name=new_name, version=self._next_version(new_name),
                             fingerprint=parent.fingerprint,
                             num_computed_tokens=parent.num_computed_tokens,
                             token_ids=parent.token_ids, parent=handle)
        return self._add(record, self._tensors(handle))

    def mutate(self, handle: str, rule: str, params: dict | None = None) -> str:
        """Apply a registered rule to a copy of the record's tensors; the
        result is a new version of the same name whose provenance is
        ``(parent, rule, params)`` (wkvm/store.py:178-204)."""
        params = params or {}
        if rule not in self._rules:
            raise KeyError(f"unknown mutation rule {rule!r}")
        parent = self.get(handle)
        src = self._tensors(handle)
        out = self._rules[rule]({k: v.clone() for k, v in src.items()}, params)
        record = StateRecord(name=parent.name, version=self._next_version(parent.name),
                             fingerprint=parent.fingerprint,
                             num_computed_tokens=parent.num_computed_tokens,
                             token_ids=parent.token_ids, parent=handle, rule=rule,
                             rule_params=params)
        return self._add(record, {k: _pinned(v) for k, v in out.items()})

    def register_rule(self, name: str, fn: MutationRule) -> None:
        self._rules[name] = fn

    # -- WARM <-> COLD ------------------------------------------------------------

    def _cold_path(self, handle: str) -> Path:
        return self.store_dir / f"{handle.replace('@', '_v')}.safetensors"

    def persist(self, handle: str) -> Path:
        """WARM -> COLD (safetensors + index); idempotent (wkvm/store.py:208-220)."""
        from safetensors.torch import save_file

        self.get(handle)
        path = self._cold_path(handle)
        if handle not in self._cold:
            save_file({k: v.contiguous() for k, v in self._tensors(handle).items()}, str(path))
            self._cold.add(handle)
            self._write_index()
        return path

    def evict(self, handle: str) -> None:
        """Drop the WARM copy, persisting it first (wkvm/store.py:222-225)."""
        self.persist(handle)
        self._warm.pop(handle, None)

    def delete(self, handle: str) -> None:
        self._warm.pop(handle, None)
        self._meta.pop(handle, None)
        if handle in self._cold:
            self._cold.discard(handle)
            self._cold_path(handle).unlink(missing_ok=True)
        self._write_index()

    def _tensors(self, handle: str) -> dict[str, torch.Tensor]:
        if handle in self._warm:
            return self._warm[handle]
        if handle in self._cold:
            from safetensors.torch import load_file

            tensors = {k: _pinned(v) for k, v in load_file(str(self._cold_path(handle))).items()}
            self._warm[handle] = tensors  # promoted to WARM
            return tensors
        raise KeyError(f"{handle}: metadata present but no WARM or COLD data")

    # -- rules ---------------------------------------------------------------------

    def _rule_merge(self, tensors: dict[str, torch.Tensor], params: dict) -> dict[str, torch.Tensor]:
        """(1 - w) * self + w * other in fp32, cast back to each family's dtype
        (wkvm/store.py:260-268)."""
        other = self._tensors(params["other"])
        w = float(params.get("weight", 0.5))
        return {k: ((1.0 - w) * v.float() + w * other[k].float()).to(v.dtype)
                for k, v in tensors.items()}

    # -- index (restart persistence) ---------------------------------------------------

    def _index_path(self) -> Path:
        return self.store_dir / "index.json"

    def _write_index(self) -> None:
        data = {h: {**asdict(r), "token_ids": list(r.token_ids), "cold": h in self._cold}
                for h, r in self._meta.items()}
        tmp = self._index_path().with_suffix(".tmp")
        tmp.write_text(json.dumps(data))
        os.replace(tmp, self._index_path())

    def _load_index(self) -> None:
        path = self._index_path()
        if not path.exists():
            return
        for handle, entry in json.loads(path.read_text()).items():
            cold = bool(entry.pop("cold", False))
            entry["token_ids"] = tuple(entry["token_ids"])
            entry["rule_params"] = entry.get("rule_params") or {}
            self._meta[handle] = StateRecord(**entry)
            if cold:
                self._cold.add(handle)
            # WARM-only records of an ended process keep their lineage; loading
            # them fails until they are saved again.


def rule_decay(tensors: dict[str, torch.Tensor], params: dict) -> dict[str, torch.Tensor]:
    """Scale the wkv memory by ``alpha`` (default 0.9) in fp32; the
    token-shift caches are unchanged (wkvm/store.py:298-305)."""
    alpha = float(params.get("alpha", 0.9))
    out = dict(tensors)
    out["wkv"] = (tensors["wkv"].float() * alpha).to(tensors["wkv"].dtype)
    return out


def _pinned(t: torch.Tensor) -> torch.Tensor:
    """Contiguous page-locked copy for the DMA path (host memory is left
    pageable when no GPU is present: there is nothing to copy to then)."""
    t = t.contiguous()
    if t.is_pinned() or not torch.cuda.is_available():
        return t
    return t.pin_memory()
