"""StateStore over the slot pool: named, versioned, forkable state handles in
three tiers, drop-in for the reference's StateStore (wkvm/store.py).

* HOT  -- the session's slot rows in ``RWKV7StateBank`` (``wkv`` and ``shift``
  families, every layer).
* WARM -- pinned host tensors, one per family, in the dense layout of one
  slot's rows (``wkv [L, H, 64, 64]`` fp32, ``shift [L, 2, D]`` model dtype).
* COLD -- one safetensors file per handle plus an index file under
  ``store_dir``; a new process rebuilds the store from the index alone.

Design. Every handle owns one ``_Entry``: its immutable ``StateRecord``, the
WARM tensors (or None once evicted) and whether its COLD file exists. Forks
share the parent's WARM dict, which is safe because no path writes into a
stored tensor: rules work on copies and loads only read. The index is a
``_Catalog`` that rewrites one JSON file atomically (write a temporary file,
flush and fsync it, rename it over the index, fsync the directory), so a
process killed at any point leaves either the previous or the next complete
index. HOT -> WARM gathers both families' strided slot rows into a device
staging buffer (``wkv7_slot_copy``) and moves each to the host as one
contiguous DMA; WARM -> HOT is one strided host-to-device DMA per family
straight into the slot rows (``wkv7_slot_transfer``).

What the on-disk format and the caller contract fix, and so stays as the
reference has it (wkvm/store.py:39-57, 80-84, 228-256):
* the record fields and the ``name@version`` handle; versions of a name are
  1 + the highest live version (0 for a new name);
* the index file ``index.json``: handle -> record fields (``token_ids`` as a
  list) plus a boolean ``cold``;
* COLD files named by the handle with every ``@`` replaced by ``_v``
  (``<name>_v<version>.safetensors`` for a name without ``@``), holding
  tensors ``wkv`` and ``shift``; the file is fsync'd and renamed into place
  before the index marks the record ``cold``;
* the model fingerprint: the first 16 hex digits of the sha256 of
  ``rwkv7:L{n_layer}:wkv{wkv_shape}:shift{shift_shape}:{dtype}``;
* the two built-in rules: ``decay`` scales ``wkv`` by ``alpha`` (default
  0.9) in fp32; ``merge`` is ``(1 - weight) self + weight other`` (default
  weight 0.5) in fp32, one rounding per product and one for the sum, cast
  back to each family's dtype.

Single-threaded and synchronous like the reference (wkvm/store.py:21-22):
transfers synchronise the device before returning.
"""

from __future__ import annotations

import dataclasses
import hashlib
import json
import math
import os
from dataclasses import dataclass, field
from pathlib import Path
from typing import Callable, Iterable

import torch

from . import ops
from .state import RWKV7StateBank

MutationRule = Callable[[dict[str, torch.Tensor], dict], dict[str, torch.Tensor]]

FAMILIES = ("wkv", "shift")
# slot dimension of each family in the bank (wkv [L, S+1, ...], shift [L, 2, S+1, D])
_SLOT_DIM = {"wkv": 1, "shift": 2}


@dataclass(frozen=True)
class StateRecord:
    """Metadata of one immutable snapshot: which session (``name``) and
    version, the model it belongs to (``fingerprint``), the tokens whose
    effect it holds (``num_computed_tokens`` of ``token_ids``) and, for forks
    and mutations, where it came from (``parent``, ``rule``, ``rule_params``)."""

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
    """Loading a record saved for another state layout into this bank."""


_RECORD_FIELDS = tuple(f.name for f in dataclasses.fields(StateRecord))


def layout_fingerprint(bank: RWKV7StateBank) -> str:
    """The model binding of a record: a short hash of the bank's state layout
    (layer count, per-slot shapes and model dtype)."""
    lay = bank.layout
    text = "rwkv7:L%d:wkv%s:shift%s:%s" % (lay.n_layer, tuple(lay.wkv_shape),
                                          tuple(lay.shift_shape), lay.dtype)
    return hashlib.sha256(text.encode()).hexdigest()[:16]


@dataclass
class _Entry:
    record: StateRecord
    host: dict[str, torch.Tensor] | None  # WARM tensors; shared with forks
    on_disk: bool                          # the COLD file is written


class _Catalog:
    """The index file: one JSON object, handle -> record fields + ``cold``."""

    def __init__(self, directory: Path) -> None:
        self.path = directory / "index.json"
        self._partial = directory / "index.json.partial"

    @staticmethod
    def _row(entry: _Entry) -> dict:
        rec = entry.record
        row = {name: getattr(rec, name) for name in _RECORD_FIELDS}
        row["token_ids"] = [int(t) for t in rec.token_ids]
        row["rule_params"] = dict(rec.rule_params)
        row["cold"] = bool(entry.on_disk)
        return row

    def store(self, entries: Iterable[_Entry]) -> None:
        payload = json.dumps({e.record.handle: self._row(e) for e in entries})
        with open(self._partial, "w") as f:
            f.write(payload)
            f.flush()
            os.fsync(f.fileno())
        os.replace(self._partial, self.path)
        _fsync_dir(self.path.parent)

    def entries(self) -> list[_Entry]:
        """Records of the last complete index; their WARM tensors died with
        the process that held them, so only ``cold`` ones keep their data."""
        if not self.path.exists():
            return []
        out = []
        for row in json.loads(self.path.read_text()).values():
            fields = {k: row[k] for k in _RECORD_FIELDS if k in row}
            fields["token_ids"] = tuple(fields.get("token_ids", ()))
            fields["rule_params"] = dict(fields.get("rule_params") or {})
            out.append(_Entry(StateRecord(**fields), None, bool(row.get("cold", False))))
        return out


class StateStore:
    def __init__(self, bank: RWKV7StateBank, store_dir: str | Path) -> None:
        self.bank = bank
        self.store_dir = Path(store_dir)
        self.store_dir.mkdir(parents=True, exist_ok=True)
        self.fingerprint = layout_fingerprint(bank)
        self._catalog = _Catalog(self.store_dir)
        self._entries: dict[str, _Entry] = {e.record.handle: e for e in self._catalog.entries()}
        self._rules: dict[str, MutationRule] = {"decay": rule_decay, "merge": self._merge}
        self._stage: torch.Tensor | None = None

    # -- records ---------------------------------------------------------------

    def get(self, handle: str) -> StateRecord:
        entry = self._entries.get(handle)
        if entry is None:
            raise KeyError(f"no state record {handle!r} in this store")
        return entry.record

    def list(self) -> list[StateRecord]:
        return [self._entries[h].record for h in sorted(
            self._entries, key=lambda h: (self._entries[h].record.name,
                                          self._entries[h].record.version))]

    @property
    def _warm(self) -> dict[str, dict[str, torch.Tensor]]:
        """Handles whose tensors are in host memory (the WARM tier) -> tensors."""
        return {h: e.host for h, e in self._entries.items() if e.host is not None}

    def _next_version(self, name: str) -> int:
        live = [e.record.version for e in self._entries.values() if e.record.name == name]
        return max(live) + 1 if live else 0

    def _new_record(self, name: str, base: StateRecord | None = None, **fields) -> StateRecord:
        if base is not None:
            fields.setdefault("num_computed_tokens", base.num_computed_tokens)
            fields.setdefault("token_ids", base.token_ids)
            fields.setdefault("fingerprint", base.fingerprint)
        fields.setdefault("fingerprint", self.fingerprint)
        fields["token_ids"] = tuple(int(t) for t in fields["token_ids"])
        fields["rule_params"] = dict(fields.get("rule_params") or {})
        return StateRecord(name=name, version=self._next_version(name), **fields)

    def _commit(self, record: StateRecord, host: dict[str, torch.Tensor]) -> str:
        self._entries[record.handle] = _Entry(record, host, False)
        self._catalog.store(self._entries.values())
        return record.handle

    def host_tensors(self, handle: str) -> dict[str, torch.Tensor]:
        """The record's WARM tensors, read back from its COLD file (and kept
        WARM) when it was evicted. Callers must not write into them."""
        self.get(handle)
        entry = self._entries[handle]
        if entry.host is None:
            if not entry.on_disk:
                raise KeyError(f"{handle}: its tensors were only in host memory of a process "
                               "that has ended; save the state again")
            from safetensors.torch import load_file

            loaded = load_file(str(self._cold_path(handle)))
            entry.host = {fam: _pinned(loaded[fam]) for fam in FAMILIES}
        return entry.host

    # -- HOT <-> WARM ------------------------------------------------------------

    def _family(self, fam: str) -> torch.Tensor:
        return self.bank.wkv if fam == "wkv" else self.bank.shift

    def _slot_shape(self, fam: str) -> torch.Size:
        t = self._family(fam)
        d = _SLOT_DIM[fam]
        return t.shape[:d] + t.shape[d + 1:]

    def _staging(self) -> torch.Tensor:
        """Device buffer for one slot's rows of both families (12.2 MiB at the
        1.5B shape, each family at a 256-byte boundary), allocated on first
        use."""
        if self._stage is None:
            total = sum(_round_up(math.prod(self._slot_shape(f)) * self._family(f).element_size(),
                                  256) for f in FAMILIES)
            self._stage = torch.empty(total, dtype=torch.uint8, device=self.bank.device)
        return self._stage

    def save(self, name: str, slots: dict[str, int], num_computed_tokens: int,
             token_ids: list[int], parent: str | None = None, rule: str | None = None,
             rule_params: dict | None = None) -> str:
        """Snapshot a session's HOT slot rows as the next version of ``name``
        (wkvm/store.py:108-137). Both families' rows are gathered on the
        device into the staging buffer, then each crosses the host link as
        one contiguous DMA into a pinned tensor: one kernel -> DMA hand-off
        per save and one synchronise."""
        record = self._new_record(name, num_computed_tokens=num_computed_tokens,
                                  token_ids=token_ids, parent=parent, rule=rule,
                                  rule_params=rule_params)
        stage, offset, staged = self._staging(), 0, {}
        for fam in FAMILIES:
            src = self._family(fam)
            shape = self._slot_shape(fam)
            nbytes = math.prod(shape) * src.element_size()
            view = stage[offset:offset + nbytes].view(src.dtype).view(shape)
            ops.slot_gather_dense(src, slots[fam], _SLOT_DIM[fam], view)
            staged[fam] = view
            offset += _round_up(nbytes, 256)
        host = {}
        for fam, view in staged.items():
            host[fam] = torch.empty(view.shape, dtype=view.dtype, pin_memory=True)
            host[fam].copy_(view, non_blocking=True)
        torch.cuda.synchronize(self.bank.device)
        return self._commit(record, host)

    def save_host(self, name: str, tensors: dict[str, torch.Tensor], num_computed_tokens: int,
                  token_ids: list[int], parent: str | None = None, rule: str | None = None,
                  rule_params: dict | None = None) -> str:
        """Record host tensors already in the WARM layout (a state computed
        elsewhere, or taken from another store) as the next version of
        ``name``; no device transfer. Shapes and dtypes must be the bank's."""
        host = {}
        for fam in FAMILIES:
            t = tensors[fam]
            want = self._slot_shape(fam)
            if tuple(t.shape) != tuple(want) or t.dtype != self._family(fam).dtype:
                raise ValueError(f"{fam} must be {tuple(want)} {self._family(fam).dtype}, "
                                 f"got {tuple(t.shape)} {t.dtype}")
            host[fam] = _pinned(t.detach().cpu())
        record = self._new_record(name, num_computed_tokens=num_computed_tokens,
                                  token_ids=token_ids, parent=parent, rule=rule,
                                  rule_params=rule_params)
        return self._commit(record, host)

    def load(self, handle: str, slots: dict[str, int]) -> StateRecord:
        """Write a record into already-allocated slots: one host-to-device DMA
        per family into the slot rows, then one synchronise
        (wkvm/store.py:139-156). A record of another model raises
        ``FingerprintMismatch`` before any byte moves."""
        record = self.get(handle)
        if record.fingerprint != self.fingerprint:
            raise FingerprintMismatch(f"{handle} belongs to state layout {record.fingerprint}; "
                                      f"this bank is {self.fingerprint}")
        host = self.host_tensors(handle)
        for fam in FAMILIES:
            ops.slot_from_host(self._family(fam), slots[fam], _SLOT_DIM[fam], _pinned(host[fam]))
        torch.cuda.synchronize(self.bank.device)
        return record

    # -- lineage -----------------------------------------------------------------

    def fork(self, handle: str, new_name: str) -> str:
        """The next version of ``new_name`` with ``handle``'s bytes and token
        history; no state data moves, the WARM tensors are shared
        (wkvm/store.py:158-176)."""
        base = self.get(handle)
        record = self._new_record(new_name, base, parent=handle)
        return self._commit(record, self.host_tensors(handle))

    def mutate(self, handle: str, rule: str, params: dict | None = None) -> str:
        """The next version of ``handle``'s name, holding ``rule`` applied to
        a copy of its tensors; provenance is ``(parent, rule, params)``
        (wkvm/store.py:178-204)."""
        fn = self._rules.get(rule)
        if fn is None:
            raise KeyError(f"no mutation rule {rule!r} (registered: {sorted(self._rules)})")
        params = dict(params or {})
        base = self.get(handle)
        result = fn({fam: t.clone() for fam, t in self.host_tensors(handle).items()}, params)
        record = self._new_record(base.name, base, parent=handle, rule=rule, rule_params=params)
        return self._commit(record, {fam: _pinned(t) for fam, t in result.items()})

    def register_rule(self, name: str, fn: MutationRule) -> None:
        """Add (or replace) a mutation rule: ``fn(tensors, params) -> tensors``
        on copies of a record's WARM tensors."""
        self._rules[name] = fn

    def _merge(self, tensors: dict[str, torch.Tensor], params: dict) -> dict[str, torch.Tensor]:
        other = self.host_tensors(params["other"])
        weight = float(params.get("weight", 0.5))
        out = {}
        for fam, mine in tensors.items():
            blend = mine.float().mul(1.0 - weight)
            blend.add_(other[fam].float().mul(weight))
            out[fam] = blend.to(mine.dtype)
        return out

    # -- WARM <-> COLD ------------------------------------------------------------

    def _cold_path(self, handle: str) -> Path:
        # The reference derives the file name from the handle by replacing
        # every '@' with '_v' (wkvm/store.py:257-258); a name that itself
        # holds '@' must map to the same file for a shared store directory.
        return self.store_dir / f"{self.get(handle).handle.replace('@', '_v')}.safetensors"

    def persist(self, handle: str) -> Path:
        """Write the record's COLD file and mark it in the index; a record
        already on disk is left as it is (wkvm/store.py:208-220)."""
        path = self._cold_path(handle)
        entry = self._entries[handle]
        if not entry.on_disk:
            from safetensors.torch import save_file

            host = self.host_tensors(handle)
            # The index must never name a file whose bytes are not durable:
            # write a temporary file, fsync it, rename it into place and fsync
            # the directory before the index marks the record COLD.
            partial = path.with_name(path.name + ".partial")
            save_file({fam: host[fam].contiguous() for fam in FAMILIES}, str(partial))
            _fsync_file(partial)
            os.replace(partial, path)
            _fsync_dir(self.store_dir)
            entry.on_disk = True
            self._catalog.store(self._entries.values())
        return path

    def evict(self, handle: str) -> None:
        """Release the WARM copy; the record stays loadable from its COLD
        file, which is written first if needed (wkvm/store.py:222-225)."""
        self.persist(handle)
        self._entries[handle].host = None

    def delete(self, handle: str) -> None:
        """Forget a record and remove its COLD file; unknown handles are a
        no-op. Forks that share its WARM tensors keep them."""
        entry = self._entries.pop(handle, None)
        if entry is None:
            return
        if entry.on_disk:
            (self.store_dir / f"{handle.replace('@', '_v')}.safetensors").unlink(missing_ok=True)
        self._catalog.store(self._entries.values())


def rule_decay(tensors: dict[str, torch.Tensor], params: dict) -> dict[str, torch.Tensor]:
    """Soft forgetting: the wkv memory times ``alpha`` (default 0.9) in fp32;
    the token-shift rows are kept."""
    alpha = float(params.get("alpha", 0.9))
    out = dict(tensors)
    wkv = tensors["wkv"]
    out["wkv"] = wkv.float().mul(alpha).to(wkv.dtype)
    return out


def _fsync_file(path: Path) -> None:
    fd = os.open(path, os.O_RDONLY)
    try:
        os.fsync(fd)
    finally:
        os.close(fd)


def _fsync_dir(directory: Path) -> None:
    # a rename is durable once the directory entry is
    _fsync_file(directory)


def _round_up(n: int, to: int) -> int:
    return (n + to - 1) // to * to


def _pinned(t: torch.Tensor) -> torch.Tensor:
    """Contiguous page-locked copy for the DMA path (host memory is left
    pageable when no GPU is present: there is nothing to copy to then)."""
    t = t.contiguous()
    if t.is_pinned() or not torch.cuda.is_available():
        return t
    return t.pin_memory()
