"""wkvm_amd: MI355X-native (gfx950) WKV7 recurrence over a fixed-size slot pool.

The hot path of xiaol/wkvm -- the RWKV-7 WKV7 state update of every request,
held in a layer-major slot pool -- as hand-written HIP kernels behind a C ABI
(``include/wkv7.h``, ``libwkv7.so``), with a Python host layer that keeps the
reference's slot-tensor layout and op signatures:

* ``RWKV7StateLayout`` / ``RWKV7StateBank`` -- wkvm/models/rwkv7.py,
  wkvm/runner/state.py
* ``WKV7Runner`` -- the control flow of wkvm/runner/runner.py at op level
* ``wkv7_decode_slots`` / ``wkv7_prefill_varlen`` / ``slot_copy`` /
  ``slot_zero`` -- slot-indexed kernels
* ``fused_recurrent_rwkv7`` / ``chunk_rwkv7`` -- the fla wkv-op signatures the
  reference's model layer calls
* ``DecodeGraph`` -- a decode step's WKV launches captured as one HIP graph
  (the role of experiments/m2_engine_bench.py GraphedDecode)
* ``StateStore`` -- HOT/WARM/COLD state handles, wkvm/store.py, with the
  HOT <-> WARM copies as strided DMA transfers
"""

from .layout import HEAD_SIZE, WKV_DTYPE, ModelStateSpec, RWKV7StateLayout, StateFamilySpec
from .ops import (
    chunk_rwkv7,
    fused_recurrent_rwkv7,
    slot_copy,
    slot_zero,
    wkv7_decode_slots,
    wkv7_prefill_varlen,
)
from .graph import DecodeGraph
from .runner import WKV7Runner
from .state import RWKV7StateBank, SlotCache
from .store import FingerprintMismatch, StateRecord, StateStore

__all__ = [
    "HEAD_SIZE", "WKV_DTYPE", "ModelStateSpec", "RWKV7StateLayout", "StateFamilySpec",
    "RWKV7StateBank", "SlotCache", "WKV7Runner", "DecodeGraph",
    "StateStore", "StateRecord", "FingerprintMismatch",
    "wkv7_decode_slots", "wkv7_prefill_varlen", "slot_copy", "slot_zero",
    "chunk_rwkv7", "fused_recurrent_rwkv7",
]
