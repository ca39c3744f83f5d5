"""RWKV7StateBank: the slot pool, drop-in for wkvm/runner/state.py:23-100.

Same constructor, attributes and tensor layout as the reference:

* ``wkv``   ``[L, S+1, H, head_dim, head_v_dim]`` float32 (state.py:35-39)
* ``shift`` ``[L, 2, S+1, hidden]`` model dtype, ``[:, 0]`` = attention
  token-shift, ``[:, 1]`` = FFN token-shift (state.py:40-46)
* row 0 of every family is the reserved pad slot (wkvm/core/arena.py:32-37)

What changes is how the rows are touched. The WKV7 kernels read and write the
state at its slot row (``decode_wkv`` / ``prefill_wkv``), so the per-layer
``index_select`` -> forward -> ``index_copy_`` round trip of the reference
(state.py:63-97, runner.py:80-88) disappears from the hot path.
``gather_cache`` / ``scatter_cache`` are kept for callers that still stage
state through a cache object; they are single slot-copy launches over all
layers instead of 3 ``index_select`` + 3 ``index_copy_`` per layer.
``fork_slots`` is the device-side slot duplicate the reference leaves to the
runner (wkvm/core/arena.py:82-93) and performs through a host round trip
(wkvm/store.py:130-131, 151-152).
"""

from __future__ import annotations

import torch

from . import ops
from .layout import WKV_DTYPE, RWKV7StateLayout


class SlotCache:
    """Per-layer staging object with the fla ``Cache`` interface the reference
    uses (``update(recurrent_state=, conv_state=, ffn_state=, layer_idx=,
    offset=)`` and ``cache[i][name]``, wkvm/runner/state.py:74-97)."""

    def __init__(self) -> None:
        self._layers: list[dict[str, torch.Tensor]] = []
        self._dense: tuple[torch.Tensor, torch.Tensor] | None = None

    def update(self, recurrent_state=None, conv_state=None, ffn_state=None, layer_idx: int = 0,
               offset: int = 0) -> None:
        while len(self._layers) <= layer_idx:
            self._layers.append({})
        entry = self._layers[layer_idx]
        if recurrent_state is not None:
            entry["recurrent_state"] = recurrent_state
        if conv_state is not None:
            entry["conv_state"] = conv_state
        if ffn_state is not None:
            entry["ffn_state"] = ffn_state

    def __getitem__(self, i: int) -> dict[str, torch.Tensor]:
        return self._layers[i]

    def __len__(self) -> int:
        return len(self._layers)


class RWKV7StateBank:
    def __init__(self, layout: RWKV7StateLayout, num_slots: int,
                 device: torch.device | str = "cuda") -> None:
        if num_slots < 1:
            raise ValueError("num_slots must be >= 1")
        self.layout = layout
        self.num_slots = num_slots
        self.device = torch.device(device)
        self.wkv = torch.zeros((layout.n_layer, num_slots + 1, *layout.wkv_shape),
                               dtype=WKV_DTYPE, device=self.device)
        self.shift = torch.zeros((layout.n_layer, 2, num_slots + 1, *layout.shift_shape),
                                 dtype=layout.dtype, device=self.device)

    # -- slot lifecycle --------------------------------------------------------

    def zero_slots(self, slots: dict[str, int]) -> None:
        """Reset a freshly admitted request's slots (state.py:50-54): zero state
        is the empty prefix for every RWKV-7 state component."""
        ops.slot_zero(self.wkv, [slots["wkv"]], slot_dim=1)
        ops.slot_zero(self.shift, [slots["shift"]], slot_dim=2)

    def fork_slots(self, src_batch: list[dict[str, int]], dst_batch: list[dict[str, int]]) -> None:
        """Device copy of every layer's wkv and shift rows ``src -> dst``,
        bit-exact. Destinations must be distinct fresh slots (not sources)."""
        if len(src_batch) != len(dst_batch):
            raise ValueError("src_batch and dst_batch length mismatch")
        ops.slot_copy(self.wkv, ops.ids_list(dst_batch, "wkv"), self.wkv,
                      ops.ids_list(src_batch, "wkv"), slot_dim=1)
        ops.slot_copy(self.shift, ops.ids_list(dst_batch, "shift"), self.shift,
                      ops.ids_list(src_batch, "shift"), slot_dim=2)

    # -- gather / scatter (kept for cache-staging callers) ---------------------------

    def gather_cache(self, slot_batch: list[dict[str, int]]) -> SlotCache:
        """Copy the batch's states into a fresh staging cache (state.py:63-83)."""
        wkv_ids = ops.ids_list(slot_batch, "wkv")
        shift_ids = ops.ids_list(slot_batch, "shift")
        L, B = self.layout.n_layer, len(slot_batch)
        wkv = torch.empty((L, B, *self.layout.wkv_shape), dtype=WKV_DTYPE, device=self.device)
        shift = torch.empty((L, 2, B, *self.layout.shift_shape), dtype=self.shift.dtype,
                            device=self.device)
        if B:
            ops.slot_copy(wkv, None, self.wkv, wkv_ids, slot_dim=1)
            ops.slot_copy(shift, None, self.shift, shift_ids, slot_dim=2)
        cache = SlotCache()
        for i in range(L):
            cache.update(recurrent_state=wkv[i], conv_state=shift[i, 0], ffn_state=shift[i, 1],
                         layer_idx=i, offset=0)
        cache._dense = (wkv, shift)
        return cache

    def scatter_cache(self, slot_batch: list[dict[str, int]], cache: SlotCache) -> None:
        """Commit the cache's states back into the bank rows (state.py:85-97)."""
        wkv_ids = ops.ids_list(slot_batch, "wkv")
        shift_ids = ops.ids_list(slot_batch, "shift")
        if not slot_batch:
            return
        dense = getattr(cache, "_dense", None)
        if dense is not None and self._is_dense_view(cache, dense):
            ops.slot_copy(self.wkv, wkv_ids, dense[0], None, slot_dim=1)
            ops.slot_copy(self.shift, shift_ids, dense[1], None, slot_dim=2)
            return
        for i in range(self.layout.n_layer):
            state = cache[i]
            ops.slot_copy(self.wkv[i], wkv_ids,
                          state["recurrent_state"].to(WKV_DTYPE).contiguous(), None, slot_dim=0)
            ops.slot_copy(self.shift[i, 0], shift_ids,
                          state["conv_state"].to(self.shift.dtype).contiguous(), None, slot_dim=0)
            ops.slot_copy(self.shift[i, 1], shift_ids,
                          state["ffn_state"].to(self.shift.dtype).contiguous(), None, slot_dim=0)

    @staticmethod
    def _is_dense_view(cache: SlotCache, dense) -> bool:
        wkv, shift = dense
        for i in range(len(cache)):
            e = cache[i]
            if (e["recurrent_state"].data_ptr() != wkv[i].data_ptr()
                    or e["recurrent_state"].dtype != wkv.dtype
                    or e["conv_state"].data_ptr() != shift[i, 0].data_ptr()
                    or e["ffn_state"].data_ptr() != shift[i, 1].data_ptr()):
                return False
        return True

    # -- in-place WKV7 over slot rows (the hot path) ------------------------------------

    def decode_wkv(self, layer: int, slot_batch, r, w, k, v, a, b, *, scale: float = 1.0,
                   out=None, out_dtype: torch.dtype = torch.bfloat16,
                   row_order=None) -> torch.Tensor:
        """One decode token per slot for ``layer``; ``slot_batch`` is a list of
        arena slot dicts or a device int32 id tensor (then ``row_order`` may
        give the visiting order, see ``ops.decode_plan``). Returns ``y [B, H, 64]``."""
        ids = slot_batch if isinstance(slot_batch, torch.Tensor) else ops.ids_list(slot_batch, "wkv")
        return ops.wkv7_decode_slots(self.wkv[layer], ids, r, w, k, v, a, b, scale=scale,
                                     out=out, out_dtype=out_dtype, row_order=row_order)

    def prefill_wkv(self, layer: int, slot_batch, cu_seqlens, r, w, k, v, a, b, *,
                    zero_init: bool = False, scale: float = 1.0, out=None,
                    out_dtype: torch.dtype = torch.bfloat16,
                    seq_order=None) -> torch.Tensor:
        """Ragged prefill for ``layer``: sequence s of the packed ``[T, H, 64]``
        inputs continues from (or, with ``zero_init``, replaces) its slot state.
        ``seq_order`` (device int32) is the order the sequences are started in."""
        ids = slot_batch if isinstance(slot_batch, torch.Tensor) else ops.ids_list(slot_batch, "wkv")
        return ops.wkv7_prefill_varlen(self.wkv[layer], ids, cu_seqlens, r, w, k, v, a, b,
                                       zero_init=zero_init, scale=scale, out=out,
                                       out_dtype=out_dtype, seq_order=seq_order)

    def state_bytes(self) -> int:
        return (self.wkv.numel() * self.wkv.element_size()
                + self.shift.numel() * self.shift.element_size())
