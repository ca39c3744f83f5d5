"""Tensor-level WKV7 ops over the slot pool, bound to libwkv7.so.

Everything here launches the hand-written gfx950 kernels through the C ABI on
the current torch stream; PyTorch only supplies device memory and the stream.
There is no CPU or eager fallback: a missing library or a CPU tensor raises.

Two layers of API:

* slot-indexed ops (the hot path): ``wkv7_decode_slots``,
  ``wkv7_prefill_varlen``, ``slot_copy``, ``slot_zero``;
* the time-mix stages either side of the WKV op: ``token_shift_mix`` (the
  slot-indexed token shift of a ``bank.shift`` family fused with its lerp
  mixes), ``time_mix_inputs`` and ``time_mix_output``;
* the fla wkv-op signatures the reference's model layer calls
  (``fused_recurrent_rwkv7`` for T < 64 and ``chunk_rwkv7`` otherwise,
  dispatched at wkvm/models/rwkv7.py:108-111), implemented by treating the
  ``[N, H, K, V]`` state tensor as a slot pool with ids ``0..N-1``.

Error behaviour mirrors the reference: invalid arguments raise ``ValueError``
(wkvm/runner/runner.py:34-35,48-49,78-79 style); a failed launch raises
``WKV7Error``.
"""

from __future__ import annotations

import threading
from collections import OrderedDict
from typing import Iterable, Sequence

import numpy as np
import torch

from . import _lib
from .layout import HEAD_SIZE

_IDS = (list, tuple, range, np.ndarray)


# The current stream's raw handle: torch's own fast accessor when present (a
# launch wrapper pays for torch.cuda.current_stream's Stream object otherwise).
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_ptr(device: torch.device) -> int:
    if _RAW_STREAM is None:
        return torch.cuda.current_stream(device).cuda_stream
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return _RAW_STREAM(idx)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _require_cuda(t: torch.Tensor, what: str) -> None:
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{what} must be a torch.Tensor")
    if not t.is_cuda:
        raise ValueError(f"{what} must be a GPU tensor (the WKV7 ops have no CPU path)")


def _check_pool(pool: torch.Tensor) -> tuple[int, int]:
    _require_cuda(pool, "wkv pool")
    if pool.dtype != torch.float32:
        raise ValueError(f"wkv pool must be float32, got {pool.dtype}")
    if pool.dim() != 4 or pool.shape[2] != HEAD_SIZE or pool.shape[3] != HEAD_SIZE:
        raise ValueError(f"wkv pool must be [rows, H, 64, 64], got {tuple(pool.shape)}")
    if not pool.is_contiguous():
        raise ValueError("wkv pool layer must be contiguous")
    return int(pool.shape[0]), int(pool.shape[1])


def host_ids(ids, rows: int, what: str, distinct: bool) -> list[int]:
    """Validate host-side slot ids: in [0, rows) and (optionally) distinct."""
    if isinstance(ids, torch.Tensor):
        ids = ids.tolist()
    out = [int(i) for i in ids]
    for i in out:
        if i < 0 or i >= rows:
            raise ValueError(f"{what}: slot id {i} out of range [0, {rows})")
    if distinct and len(set(out)) != len(out):
        raise ValueError(f"{what}: duplicate slot ids {out}")
    return out


def device_ids(ids, rows: int, device: torch.device, what: str, distinct: bool = True) -> torch.Tensor:
    """Slot ids as a device int32 tensor.

    Host ids (list / tuple / numpy / CPU tensor) are validated first and raise
    ``ValueError``. A CUDA int32 tensor is taken as already validated: the
    kernels skip out-of-range rows without touching memory, and duplicate ids
    in a write set race.
    """
    if isinstance(ids, torch.Tensor) and ids.is_cuda:
        if ids.dtype != torch.int32 or ids.dim() != 1:
            raise ValueError(f"{what}: device ids must be a 1-D int32 tensor")
        if ids.device != device:
            raise ValueError(f"{what}: ids on {ids.device}, pool on {device}")
        return ids
    lst = host_ids(ids, rows, what, distinct)
    return torch.tensor(lst, dtype=torch.int32, device=device)


def decode_plan(slot_ids, rows: int, device: torch.device) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Device ``(slot_ids, row_order)`` for a decode batch.

    Host ids are validated (in range, distinct) and uploaded together with the
    batch rows sorted by slot id -- the visiting order that keeps the kernel's
    HBM stream local -- in one copy. Device ids pass through with no order.
    """
    if isinstance(slot_ids, torch.Tensor) and slot_ids.is_cuda:
        return device_ids(slot_ids, rows, device, "slot_ids"), None
    lst = host_ids(slot_ids, rows, "slot_ids", distinct=True)
    order = sorted(range(len(lst)), key=lst.__getitem__)
    both = torch.tensor(lst + order, dtype=torch.int32, device=device)
    return both[:len(lst)], both[len(lst):]


def _check_vectors(xs: Sequence[torch.Tensor], shape: tuple[int, ...], device: torch.device,
                   what: str) -> list[torch.Tensor]:
    out = []
    for name, x in zip("rwkvab", xs):
        if not (isinstance(x, torch.Tensor) and x.is_cuda):  # (message built on failure only)
            _require_cuda(x, f"{what}.{name}")
        if x.dtype != torch.bfloat16:
            raise ValueError(f"{what}.{name} must be bfloat16, got {x.dtype}")
        if tuple(x.shape) != shape:
            raise ValueError(f"{what}.{name} must be {shape}, got {tuple(x.shape)}")
        if x.device != device:
            raise ValueError(f"{what}.{name} on {x.device}, pool on {device}")
        x = x.contiguous()
        if x.data_ptr() % 16:
            x = x.clone()  # the kernels read 16-byte vectors
        out.append(x)
    return out


def _y_code(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return _lib.WKV7_Y_BF16
    if dtype == torch.float32:
        return _lib.WKV7_Y_F32
    raise ValueError(f"y dtype must be bfloat16 or float32, got {dtype}")


def _out(out: torch.Tensor | None, shape, dtype, device, what: str) -> torch.Tensor:
    if out is None:
        return torch.empty(shape, dtype=dtype, device=device)
    _require_cuda(out, what)
    if tuple(out.shape) != tuple(shape) or not out.is_contiguous():
        raise ValueError(f"{what} must be a contiguous {tuple(shape)} tensor")
    return out


# -- slot-indexed hot path ---------------------------------------------------------

def wkv7_decode_slots(wkv_layer: torch.Tensor, slot_ids, r, w, k, v, a, b, *,
                      scale: float = 1.0, out: torch.Tensor | None = None,
                      out_dtype: torch.dtype = torch.bfloat16,
                      row_order: torch.Tensor | None = None) -> torch.Tensor:
    """One decode token per slot, in place on ``wkv_layer`` ([rows, H, 64, 64]).

    ``r, w, k, v, a, b``: bf16 ``[B, H, 64]`` (``w`` is log-decay). Returns
    ``y`` ``[B, H, 64]`` in ``out_dtype`` (bf16 or fp32). ``row_order`` (device
    int32, a permutation of the batch rows) only sets the visiting order; for
    host ids the slot-sorted order is computed here.
    """
    rows, H = _check_pool(wkv_layer)
    dev = wkv_layer.device
    ids, order = decode_plan(slot_ids, rows, dev)
    if row_order is not None:
        if not (isinstance(row_order, torch.Tensor) and row_order.is_cuda
                and row_order.dtype == torch.int32 and row_order.shape == ids.shape):
            raise ValueError("row_order must be a device int32 tensor shaped like slot_ids")
        order = row_order
    B = int(ids.shape[0])
    xs = _check_vectors((r, w, k, v, a, b), (B, H, HEAD_SIZE), dev, "decode")
    code = _y_code(out.dtype if out is not None else out_dtype)
    y = _out(out, (B, H, HEAD_SIZE), out_dtype if out is None else out.dtype, dev, "out")
    if B == 0:
        return y
    lib = _lib.load()
    rc = lib.wkv7_decode_slots(wkv_layer.data_ptr(), rows, H, ids.data_ptr(), _ptr(order), B,
                               *[x.data_ptr() for x in xs], y.data_ptr(), code, float(scale),
                               _stream_ptr(dev))
    _lib.check(rc, "wkv7_decode_slots")
    return y


def _state_tensor(t: torch.Tensor | None, H: int, device: torch.device, what: str) -> int:
    """Rows of an optional ``[rows, H, 64, 64]`` fp32 state tensor (0 for None)."""
    if t is None:
        return 0
    rows, heads = _check_pool(t)
    if heads != H:
        raise ValueError(f"{what} has {heads} heads, the inputs {H}")
    if t.device != device:
        raise ValueError(f"{what} on {t.device}, inputs on {device}")
    return rows


def wkv7_decode_into(state_in: torch.Tensor | None, state_out: torch.Tensor | None,
                     r, w, k, v, a, b, *, in_ids=None, out_ids=None, scale: float = 1.0,
                     out: torch.Tensor | None = None, out_dtype: torch.dtype = torch.bfloat16,
                     row_order: torch.Tensor | None = None) -> torch.Tensor:
    """One decode token per row with the state read from ``state_in`` and
    written to ``state_out`` (each ``[rows, H, 64, 64]`` fp32, or None: a zero
    initial state / no state written). Row ``b`` reads ``state_in[in_ids[b]]``
    and writes ``state_out[out_ids[b]]``; ``None`` ids mean row ``b``. This is
    fla's recurrent op at seq_len 1 (initial_state -> final_state) without a
    copy of the state. Returns ``y [B, H, 64]``."""
    _require_cuda(r, "decode.r")
    if r.dim() != 3:
        raise ValueError(f"decode inputs must be [B, H, 64], got {tuple(r.shape)}")
    B, H = int(r.shape[0]), int(r.shape[1])
    dev = r.device
    xs = _check_vectors((r, w, k, v, a, b), (B, H, HEAD_SIZE), dev, "decode")
    in_rows = _state_tensor(state_in, H, dev, "state_in")
    out_rows = _state_tensor(state_out, H, dev, "state_out")
    if in_ids is not None and state_in is None:
        raise ValueError("in_ids without state_in")
    if out_ids is not None and state_out is None:
        raise ValueError("out_ids without state_out")
    for t, ids, n in ((state_in, in_ids, "state_in"), (state_out, out_ids, "state_out")):
        if t is not None and ids is None and t.shape[0] < B:
            raise ValueError(f"{n} has {t.shape[0]} rows for {B} batch rows")
    if state_in is not None and state_out is not None and _overlaps(state_in, state_out):
        # in place row by row, or disjoint row sets; anything else would let a
        # row overwrite a state another row still has to read
        if state_in.data_ptr() != state_out.data_ptr():
            raise ValueError("state_in and state_out overlap at different offsets")
        if not all(isinstance(x, _IDS) or x is None for x in (in_ids, out_ids)):
            raise ValueError("overlapping state tensors need host ids (checked here)")
        src = list(range(B)) if in_ids is None else [int(i) for i in in_ids]
        dst = list(range(B)) if out_ids is None else [int(i) for i in out_ids]
        if src != dst and set(src) & set(dst):
            raise ValueError("a row writes a state row that another row reads")
    d_in = None if in_ids is None else device_ids(in_ids, in_rows, dev, "in_ids", distinct=False)
    d_out = None if out_ids is None else device_ids(out_ids, out_rows, dev, "out_ids",
                                                    distinct=True)
    for ids in (d_in, d_out):
        if ids is not None and int(ids.shape[0]) != B:
            raise ValueError(f"{int(ids.shape[0])} ids for {B} batch rows")
    if row_order is not None and not (isinstance(row_order, torch.Tensor) and row_order.is_cuda
                                      and row_order.dtype == torch.int32
                                      and tuple(row_order.shape) == (B,)):
        raise ValueError("row_order must be a device int32 tensor of B entries")
    code = _y_code(out.dtype if out is not None else out_dtype)
    y = _out(out, (B, H, HEAD_SIZE), out_dtype if out is None else out.dtype, dev, "out")
    if B == 0:
        return y
    rc = _lib.load().wkv7_decode_into(_ptr(state_in), in_rows, _ptr(d_in), _ptr(state_out),
                                      out_rows, _ptr(d_out), H, _ptr(row_order), B,
                                      *[x.data_ptr() for x in xs], y.data_ptr(), code,
                                      float(scale), _stream_ptr(dev))
    _lib.check(rc, "wkv7_decode_into")
    return y


def _host_cu(cu, T: int) -> list[int]:
    if isinstance(cu, torch.Tensor):
        cu = cu.tolist()
    lst = [int(c) for c in cu]
    if not lst or lst[0] != 0 or lst[-1] != T:
        raise ValueError(f"cu_seqlens must start at 0 and end at total tokens {T}, got {lst[:3]}..")
    for i in range(len(lst) - 1):
        if lst[i + 1] < lst[i]:
            raise ValueError("cu_seqlens must be non-decreasing")
    if T >= 2**31:
        raise ValueError("total tokens must fit int32")
    return lst


_PLANS: "OrderedDict[tuple, tuple[torch.Tensor, int]]" = OrderedDict()  # (plan, its stream)
_PLAN_CACHE_SIZE = 256
_PLANS_LOCK = threading.Lock()
# plans a HIP graph captured: a replay reads them, so they are never evicted
_CAPTURED_PLANS: dict[tuple, tuple[torch.Tensor, int]] = {}


def _device_plan(lst: list[int], dev: torch.device) -> torch.Tensor:
    """``cu_seqlens`` followed by the longest-first start order, as one device
    int32 tensor. Cached per (device, offsets): the fla-signature callers
    repeat the same offsets on every call (one request per call in fixed
    prefill_chunk slices, wkvm/runner/runner.py:52-61), and the upload is the
    largest part of such a call's host time. The tensor is complete when it
    is returned (a blocking copy from pageable memory) and only ever read; a
    use on another stream than the one it was made on is recorded on that
    stream, so an entry evicted while such a launch still reads it is not
    reused before the launch ends. A plan used under HIP-graph capture (it
    must be cached before the capture: the upload cannot be captured) stays
    alive for good, since the graph's replays read it. The cache is shared by
    the threads of the process."""
    key = (dev.index, tuple(lst))
    capturing = torch.cuda.is_current_stream_capturing()
    stream = _stream_ptr(dev)
    with _PLANS_LOCK:
        entry = _CAPTURED_PLANS.get(key)
        if entry is None:
            entry = _PLANS.get(key)
            if entry is not None:
                _PLANS.move_to_end(key)
    if entry is None:
        if capturing:
            raise RuntimeError("cu_seqlens given as host offsets under graph capture: run the "
                               "call once before the capture (its device plan is then cached) "
                               "or pass device cu_seqlens and seq_order")
        plan = torch.tensor(lst + longest_first(lst), dtype=torch.int32, device=dev)
        with _PLANS_LOCK:
            entry = _PLANS.setdefault(key, (plan, stream))
            if len(_PLANS) > _PLAN_CACHE_SIZE:
                _PLANS.popitem(last=False)
    plan, made_on = entry
    if capturing:
        with _PLANS_LOCK:
            _CAPTURED_PLANS[key] = entry
    elif stream != made_on:
        plan.record_stream(torch.cuda.current_stream(dev))
    return plan


def longest_first(cu: Sequence[int]) -> list[int]:
    """Sequence order for a ragged prefill launch: longest first (ties in
    index order), which packs the per-(sequence, head) workgroups onto the
    compute units with the smallest idle tail."""
    n = len(cu) - 1
    return sorted(range(n), key=lambda s: cu[s] - cu[s + 1])


def wkv7_prefill_varlen(wkv_layer: torch.Tensor, slot_ids, cu_seqlens, r, w, k, v, a, b, *,
                        zero_init: bool = False, scale: float = 1.0,
                        out: torch.Tensor | None = None,
                        out_dtype: torch.dtype = torch.bfloat16,
                        seq_order: torch.Tensor | None = None) -> torch.Tensor:
    """Ragged prefill: sequence ``s`` runs tokens ``cu_seqlens[s]:cu_seqlens[s+1]``
    of the ``[T, H, 64]`` bf16 inputs from slot ``slot_ids[s]`` (or zero state
    if ``zero_init``) and leaves its final state in that slot. Returns ``y``
    ``[T, H, 64]``. ``seq_order`` (device int32 permutation) only sets the
    order in which sequences are started; for host ``cu_seqlens`` it is
    computed here (longest first).
    """
    rows, H = _check_pool(wkv_layer)
    dev = wkv_layer.device
    ids = device_ids(slot_ids, rows, dev, "slot_ids", distinct=True)
    nseq = int(ids.shape[0])
    _require_cuda(r, "prefill.r")
    T = int(r.shape[0]) if r.dim() == 3 else -1
    xs = _check_vectors((r, w, k, v, a, b), (T, H, HEAD_SIZE), dev, "prefill")
    if isinstance(cu_seqlens, torch.Tensor) and cu_seqlens.is_cuda:
        if cu_seqlens.dtype != torch.int32 or cu_seqlens.shape != (nseq + 1,):
            raise ValueError("device cu_seqlens must be int32 [nseq + 1]")
        cu = cu_seqlens
    else:
        lst = _host_cu(cu_seqlens, T)
        if len(lst) != nseq + 1:
            raise ValueError(f"cu_seqlens has {len(lst)} entries for {nseq} sequences")
        both = _device_plan(lst, dev)
        cu = both[:nseq + 1]
        if seq_order is None:
            seq_order = both[nseq + 1:]
    if seq_order is not None:
        if not (isinstance(seq_order, torch.Tensor) and seq_order.is_cuda
                and seq_order.dtype == torch.int32 and seq_order.shape == (nseq,)):
            raise ValueError("seq_order must be a device int32 tensor of nseq entries")
    code = _y_code(out.dtype if out is not None else out_dtype)
    y = _out(out, (T, H, HEAD_SIZE), out_dtype if out is None else out.dtype, dev, "out")
    if y.data_ptr() % (16 if y.dtype == torch.float32 else 8):
        raise ValueError("out must be 8-byte aligned (bf16) or 16-byte aligned (fp32): the "
                         "kernel stores whole rows as vectors")
    if nseq == 0:
        return y
    rc = _lib.load().wkv7_prefill_varlen(wkv_layer.data_ptr(), rows, H, ids.data_ptr(),
                                         cu.data_ptr(), _ptr(seq_order), nseq, T,
                                         *[x.data_ptr() for x in xs], y.data_ptr(), code,
                                         int(bool(zero_init)), float(scale), _stream_ptr(dev))
    _lib.check(rc, "wkv7_prefill_varlen")
    return y


def wkv7_prefill_into(state_in: torch.Tensor | None, state_out: torch.Tensor | None,
                      cu_seqlens, r, w, k, v, a, b, *, in_ids=None, out_ids=None,
                      scale: float = 1.0, out: torch.Tensor | None = None,
                      out_dtype: torch.dtype = torch.bfloat16,
                      seq_order: torch.Tensor | None = None) -> torch.Tensor:
    """Ragged prefill with the state read from ``state_in`` and written to
    ``state_out`` (each ``[rows, H, 64, 64]`` fp32, or None: a zero initial
    state / no final state written). Sequence ``s`` reads
    ``state_in[in_ids[s]]`` and writes ``state_out[out_ids[s]]``; ``None`` ids
    mean row ``s``. This is fla's ``chunk_rwkv7`` contract (initial_state ->
    a new final_state) without a copy of the state. Returns ``y [T, H, 64]``.
    """
    _require_cuda(r, "prefill.r")
    if r.dim() != 3:
        raise ValueError(f"prefill inputs must be [T, H, 64], got {tuple(r.shape)}")
    T, H = int(r.shape[0]), int(r.shape[1])
    dev = r.device
    xs = _check_vectors((r, w, k, v, a, b), (T, H, HEAD_SIZE), dev, "prefill")
    lst = _host_cu(cu_seqlens, T) if not (isinstance(cu_seqlens, torch.Tensor)
                                          and cu_seqlens.is_cuda) else None
    nseq = len(lst) - 1 if lst is not None else int(cu_seqlens.shape[0]) - 1
    in_rows = _state_tensor(state_in, H, dev, "state_in")
    out_rows = _state_tensor(state_out, H, dev, "state_out")
    if in_ids is not None and state_in is None:
        raise ValueError("in_ids without state_in")
    if out_ids is not None and state_out is None:
        raise ValueError("out_ids without state_out")
    for t, ids, n in ((state_in, in_ids, "state_in"), (state_out, out_ids, "state_out")):
        if t is not None and ids is None and t.shape[0] < nseq:
            raise ValueError(f"{n} has {t.shape[0]} rows for {nseq} sequences")
    if state_in is not None and state_out is not None and _overlaps(state_in, state_out):
        if state_in.data_ptr() != state_out.data_ptr():
            raise ValueError("state_in and state_out overlap at different offsets")
        if not all(isinstance(x, _IDS) or x is None for x in (in_ids, out_ids)):
            raise ValueError("overlapping state tensors need host ids (checked here)")
        src = list(range(nseq)) if in_ids is None else [int(i) for i in in_ids]
        dst = list(range(nseq)) if out_ids is None else [int(i) for i in out_ids]
        if src != dst and set(src) & set(dst):
            raise ValueError("a sequence writes a state row that another sequence reads")
    d_in = None if in_ids is None else device_ids(in_ids, in_rows, dev, "in_ids", distinct=False)
    d_out = None if out_ids is None else device_ids(out_ids, out_rows, dev, "out_ids",
                                                    distinct=True)
    for ids in (d_in, d_out):
        if ids is not None and int(ids.shape[0]) != nseq:
            raise ValueError(f"{int(ids.shape[0])} ids for {nseq} sequences")
    if lst is not None:
        both = _device_plan(lst, dev)
        cu = both[:nseq + 1]
        if seq_order is None:
            seq_order = both[nseq + 1:]
    else:
        if cu_seqlens.dtype != torch.int32:
            raise ValueError("device cu_seqlens must be int32")
        cu = cu_seqlens
    if seq_order is not None and not (isinstance(seq_order, torch.Tensor) and seq_order.is_cuda
                                      and seq_order.dtype == torch.int32
                                      and tuple(seq_order.shape) == (nseq,)):
        raise ValueError("seq_order must be a device int32 tensor of nseq entries")
    code = _y_code(out.dtype if out is not None else out_dtype)
    y = _out(out, (T, H, HEAD_SIZE), out_dtype if out is None else out.dtype, dev, "out")
    if y.data_ptr() % (16 if y.dtype == torch.float32 else 8):
        raise ValueError("out must be 8-byte aligned (bf16) or 16-byte aligned (fp32): the "
                         "kernel stores whole rows as vectors")
    if nseq == 0:
        return y
    rc = _lib.load().wkv7_prefill_into(_ptr(state_in), in_rows, _ptr(d_in), _ptr(state_out),
                                       out_rows, _ptr(d_out), H, cu.data_ptr(), _ptr(seq_order),
                                       nseq, T, *[x.data_ptr() for x in xs], y.data_ptr(), code,
                                       float(scale), _stream_ptr(dev))
    _lib.check(rc, "wkv7_prefill_into")
    return y


def segment_cuts(length: int, segments: int) -> list[int]:
    """Cut points ``0 = c_0 < ... < c_G = length`` of one sequence into at most
    ``segments`` pieces, each a multiple of 16 tokens except the last."""
    if length <= 0:
        return [0]
    G = max(1, min(int(segments), (length + 15) // 16))
    step = ((length + G - 1) // G + 15) // 16 * 16
    return list(range(0, length, step)) + [length]


def wkv7_prefill_segments(wkv_layer: torch.Tensor, slot_ids, cu_seqlens, r, w, k, v, a, b, *,
                          segments: int, zero_init: bool = False, scale: float = 1.0,
                          out: torch.Tensor | None = None,
                          out_dtype: torch.dtype = torch.bfloat16,
                          state_in: torch.Tensor | None = None) -> torch.Tensor:
    """``wkv7_prefill_varlen`` with each sequence cut into up to ``segments``
    pieces that run side by side, for batches of few, long sequences (one
    sequence of H heads keeps only H compute units busy).

    The scan is linear in its initial state. One ``wkv7_prefill_runs`` launch
    holds, per sequence, segment 0 from the slot state (or zero) and, for every
    later segment g, a run from zero state (y0_g, final state H0_g) and a run
    from the identity with k = v = 0 (its transition Phi_g as the final state,
    q_g = (scale r)^T Phi_t as y). ``wkv7_segment_chain`` then walks the
    segments in order (H_out = H0_g + Phi_g H_in, ending in the slot) and
    ``wkv7_segment_correct`` writes y = y0 + q H_in for every token, in fp32,
    rounded once to ``out_dtype``. Results match the one-pass scan to fp32
    rounding. ``slot_ids`` and ``cu_seqlens`` are host sequences; the plan is
    one upload, the scratch four tensors from the caching allocator. With
    ``state_in`` (``[nseq, H, 64, 64]`` fp32) sequence ``s`` starts from
    ``state_in[s]`` instead of its slot row; the final state still goes to
    the slot."""
    rows, H = _check_pool(wkv_layer)
    dev = wkv_layer.device
    if segments < 1:
        raise ValueError("segments must be >= 1")
    ids = host_ids(slot_ids, rows, "slot_ids", distinct=True)
    nseq = len(ids)
    _require_cuda(r, "prefill.r")
    T = int(r.shape[0]) if r.dim() == 3 else -1
    xs = _check_vectors((r, w, k, v, a, b), (T, H, HEAD_SIZE), dev, "prefill")
    cu = _host_cu(cu_seqlens, T)
    if len(cu) != nseq + 1:
        raise ValueError(f"cu_seqlens has {len(cu)} entries for {nseq} sequences")
    in_rows = _state_tensor(state_in, H, dev, "state_in")
    if state_in is not None and (zero_init or in_rows < nseq):
        raise ValueError("state_in needs zero_init False and a row per sequence")
    dtype = out.dtype if out is not None else out_dtype
    code = _y_code(dtype)
    y = _out(out, (T, H, HEAD_SIZE), dtype, dev, "out")
    empty = [s for s in range(nseq) if cu[s] == cu[s + 1]]
    if zero_init and empty:
        slot_zero(wkv_layer, [ids[s] for s in empty], slot_dim=0)
    if state_in is not None and empty:
        # an empty sequence's final state is its initial state
        slot_copy(wkv_layer, [ids[s] for s in empty], state_in, empty, slot_dim=0)
    if T == 0:
        return y
    L = _lib
    run_slot, run_flags, prim_cu, run_src = [], [], [0], []
    alt_slot, alt_flags, alt_pairs = [], [], []
    seq_tab, seg_tab, blk = [], [], []
    n_alt = nsegs = 0

    def blocks(b_, e_, seg):
        for t in range(b_, e_, 64):
            blk.extend((t, min(64, e_ - t), seg))

    for s in range(nseq):
        beg, end = cu[s], cu[s + 1]
        if beg == end:
            continue
        cuts = segment_cuts(end - beg, segments)
        run_slot.append(ids[s])
        run_src.append(s)
        run_flags.append(L.WKV7_RUN_INIT_ZERO if zero_init else 0)
        prim_cu.append(beg + cuts[1])
        blocks(beg, beg + cuts[1], -1)
        first = nsegs
        for g in range(1, len(cuts) - 1):
            b_, e_ = beg + cuts[g], beg + cuts[g + 1]
            run_slot.append(n_alt)
            run_src.append(0)  # zero start: state_in is not read
            run_flags.append(L.WKV7_RUN_INIT_ZERO | L.WKV7_RUN_STATE_ALT)
            prim_cu.append(e_)
            alt_slot.append(n_alt + 1)
            alt_flags.append(L.WKV7_RUN_INIT_IDENTITY | L.WKV7_RUN_KV_ZERO | L.WKV7_RUN_Y_ALT
                             | L.WKV7_RUN_STATE_ALT)
            alt_pairs += [b_, e_]
            seg_tab += [n_alt, n_alt + 1]
            blocks(b_, e_, nsegs)
            n_alt += 2
            nsegs += 1
        if nsegs > first:
            seq_tab += [ids[s], first, nsegs - first]
    n_primary = len(run_slot)
    nruns = n_primary + len(alt_slot)
    lens = [prim_cu[i + 1] - prim_cu[i] for i in range(n_primary)]
    lens += [alt_pairs[2 * i + 1] - alt_pairs[2 * i] for i in range(len(alt_slot))]
    order = sorted(range(nruns), key=lambda i: -lens[i])
    parts = [run_slot + alt_slot, run_flags + alt_flags, prim_cu, alt_pairs or [0, 0], order,
             seq_tab or [0, 0, 0], seg_tab or [0, 0], blk, run_src + [0] * len(alt_slot)]
    plan = torch.tensor([x for p in parts for x in p], dtype=torch.int32, device=dev)
    views, at = [], 0
    for p in parts:
        views.append(plan[at:at + len(p)])
        at += len(p)
    v_ids, v_flags, v_cu, v_pairs, v_order, v_seq, v_seg, v_blk, v_src = views
    y0 = torch.empty((T, H, HEAD_SIZE), dtype=torch.float32, device=dev)
    q = torch.empty_like(y0) if nsegs else y0
    alt = torch.empty((max(n_alt, 1), H, HEAD_SIZE, HEAD_SIZE), dtype=torch.float32, device=dev)
    hin = torch.empty((max(nsegs, 1), H, HEAD_SIZE, HEAD_SIZE), dtype=torch.float32, device=dev)
    lib = _lib.load()
    stream = _stream_ptr(dev)
    rc = lib.wkv7_prefill_runs(wkv_layer.data_ptr(), rows, H, v_ids.data_ptr(), v_cu.data_ptr(),
                               v_order.data_ptr(), nruns, T, *[x.data_ptr() for x in xs],
                               y0.data_ptr(), _lib.WKV7_Y_F32, 0, float(scale),
                               v_flags.data_ptr(), v_pairs.data_ptr(), n_primary,
                               alt.data_ptr(), n_alt, q.data_ptr(), _ptr(state_in), in_rows,
                               v_src.data_ptr() if state_in is not None else None, stream)
    _lib.check(rc, "wkv7_prefill_runs")
    if nsegs:
        rc = lib.wkv7_segment_chain(wkv_layer.data_ptr(), rows, H, alt.data_ptr(), n_alt,
                                    v_seq.data_ptr(), len(seq_tab) // 3, v_seg.data_ptr(), nsegs,
                                    hin.data_ptr(), stream)
        _lib.check(rc, "wkv7_segment_chain")
    rc = lib.wkv7_segment_correct(T, H, y0.data_ptr(), q.data_ptr(), v_blk.data_ptr(),
                                  len(blk) // 3, hin.data_ptr(), nsegs, y.data_ptr(), code,
                                  stream)
    _lib.check(rc, "wkv7_segment_correct")
    return y


# -- slot row copies -----------------------------------------------------------------

def slot_view(t: torch.Tensor, slot_dim: int) -> tuple[int, int, int, int, int]:
    """Describe ``t`` as ``outer`` blocks of slot rows along ``slot_dim``.

    Returns ``(outer, outer_stride_B, slot_stride_B, rows, row_bytes)``. The
    dims after ``slot_dim`` must be contiguous and the dims before it must
    collapse into a single stride.
    """
    if slot_dim < 0:
        slot_dim += t.dim()
    if not 0 <= slot_dim < t.dim():
        raise ValueError("slot_dim out of range")
    es = t.element_size()
    row_elems = 1
    expect = 1
    for d in range(t.dim() - 1, slot_dim, -1):
        if t.shape[d] != 1 and t.stride(d) != expect:
            raise ValueError("dims after the slot dim must be contiguous")
        expect *= t.shape[d]
        row_elems *= t.shape[d]
    rows = int(t.shape[slot_dim])
    slot_stride = t.stride(slot_dim) * es
    outer = 1
    outer_stride = 0
    for d in range(slot_dim - 1, -1, -1):
        if t.shape[d] == 1:
            continue
        if outer == 1:
            outer_stride = t.stride(d) * es
        elif t.stride(d) * es != outer_stride * outer:
            raise ValueError("dims before the slot dim must collapse to one stride")
        outer *= int(t.shape[d])
    return outer, outer_stride, slot_stride, rows, row_elems * es


def slot_copy(dst: torch.Tensor, dst_ids, src: torch.Tensor, src_ids, slot_dim: int) -> None:
    """Bit-exact ``dst[..., dst_ids[p], ...] = src[..., src_ids[p], ...]`` along
    ``slot_dim`` for every pair p. ``None`` ids mean ``0..n-1`` (dense staging
    side of a gather or scatter). Within one tensor, destination rows must be
    distinct and disjoint from the source rows (fork into fresh slots)."""
    _require_cuda(dst, "dst")
    _require_cuda(src, "src")
    if dst.dtype != src.dtype or dst.device != src.device:
        raise ValueError("dst and src must share dtype and device")
    d_outer, d_os, d_ss, d_rows, d_rb = slot_view(dst, slot_dim)
    s_outer, s_os, s_ss, s_rows, s_rb = slot_view(src, slot_dim)
    if d_outer != s_outer or d_rb != s_rb:
        raise ValueError("dst and src slot rows differ in shape")
    dev = dst.device
    if dst_ids is None and src_ids is None:
        raise ValueError("at least one of dst_ids / src_ids is required")
    n = None
    if dst_ids is not None and not (isinstance(dst_ids, torch.Tensor) and dst_ids.is_cuda):
        dst_ids = host_ids(dst_ids, d_rows, "dst_ids", distinct=True)
        n = len(dst_ids)
    if src_ids is not None and not (isinstance(src_ids, torch.Tensor) and src_ids.is_cuda):
        src_ids = host_ids(src_ids, s_rows, "src_ids", distinct=False)
        if n is not None and len(src_ids) != n:
            raise ValueError("dst_ids and src_ids differ in length")
        n = len(src_ids)
    if isinstance(dst_ids, list) and isinstance(src_ids, list) and _overlaps(dst, src):
        if set(dst_ids) & set(src_ids):
            raise ValueError("fork destination rows overlap source rows")
    d_t = device_ids(dst_ids, d_rows, dev, "dst_ids") if dst_ids is not None else None
    s_t = device_ids(src_ids, s_rows, dev, "src_ids", distinct=False) if src_ids is not None else None
    if n is None:
        n = int((d_t if d_t is not None else s_t).shape[0])
    if d_t is None and n > d_rows:
        raise ValueError(f"dense dst has {d_rows} rows for {n} copies")
    if s_t is None and n > s_rows:
        raise ValueError(f"dense src has {s_rows} rows for {n} copies")
    if n == 0:
        return
    rc = _lib.load().wkv7_slot_copy(dst.data_ptr(), d_os, d_ss, d_rows, _ptr(d_t),
                                    src.data_ptr(), s_os, s_ss, s_rows, _ptr(s_t),
                                    d_outer, d_rb, n, _stream_ptr(dev))
    _lib.check(rc, "wkv7_slot_copy")


def slot_gather_dense(t: torch.Tensor, slot: int, slot_dim: int, out: torch.Tensor) -> None:
    """Bit-exact ``out = t.select(slot_dim, slot)`` into a dense device tensor
    with one ``wkv7_slot_copy`` launch (no id upload: the slot's rows are
    addressed directly)."""
    _require_cuda(t, "slot tensor")
    outer, outer_stride, slot_stride, rows, row_bytes = slot_view(t, slot_dim)
    if not 0 <= int(slot) < rows:
        raise ValueError(f"slot {slot} out of range [0, {rows})")
    if out.device != t.device or not out.is_contiguous() or out.dtype != t.dtype:
        raise ValueError("out must be a contiguous tensor of t's dtype on t's device")
    if out.numel() * out.element_size() != outer * row_bytes:
        raise ValueError(f"out holds {out.numel() * out.element_size()} B, the slot's rows are "
                         f"{outer * row_bytes} B")
    rc = _lib.load().wkv7_slot_copy(out.data_ptr(), row_bytes, 0, 1, None,
                                    t.data_ptr() + int(slot) * slot_stride, outer_stride, 0, 1,
                                    None, outer, row_bytes, 1, _stream_ptr(t.device))
    _lib.check(rc, "wkv7_slot_copy")


def _slot_transfer(direction: int, t: torch.Tensor, slot: int, slot_dim: int,
                   host: torch.Tensor, staging: torch.Tensor | None) -> None:
    _require_cuda(t, "slot tensor")
    outer, outer_stride, slot_stride, rows, row_bytes = slot_view(t, slot_dim)
    if not 0 <= int(slot) < rows:
        raise ValueError(f"slot {slot} out of range [0, {rows})")
    if host.is_cuda or not host.is_contiguous() or host.dtype != t.dtype:
        raise ValueError("host buffer must be a contiguous CPU tensor of the slot tensor's dtype")
    if host.numel() * host.element_size() != outer * row_bytes:
        raise ValueError(f"host buffer holds {host.numel() * host.element_size()} B, "
                         f"the slot's rows are {outer * row_bytes} B")
    if not host.is_pinned():
        raise ValueError("host buffer must be pinned (pin_memory) for the DMA copy")
    st_ptr, st_bytes = None, 0
    if staging is not None:
        if staging.device != t.device or not staging.is_contiguous():
            raise ValueError("staging must be a contiguous tensor on the slot tensor's device")
        st_bytes = staging.numel() * staging.element_size()
        if st_bytes < outer * row_bytes:
            raise ValueError(f"staging holds {st_bytes} B, the slot's rows are "
                             f"{outer * row_bytes} B")
        st_ptr = staging.data_ptr()
    rc = _lib.load().wkv7_slot_transfer(direction, host.data_ptr(), t.data_ptr(), outer_stride,
                                        slot_stride, rows, int(slot), outer, row_bytes,
                                        st_ptr, st_bytes, _stream_ptr(t.device))
    _lib.check(rc, "wkv7_slot_transfer")


def slot_to_host(t: torch.Tensor, slot: int, slot_dim: int, host: torch.Tensor | None = None,
                 staging: torch.Tensor | None = None) -> torch.Tensor:
    """Asynchronous copy of one slot's rows of ``t`` (every outer block) into a
    dense pinned host tensor shaped like ``t.select(slot_dim, slot)``; the
    caller synchronises before reading it. With ``staging`` (a device tensor
    of at least the slot's bytes) the rows are gathered on the device first
    and cross the host link as one contiguous DMA; without it the DMA itself
    is strided."""
    _require_cuda(t, "slot tensor")
    shape = t.shape[:slot_dim] + t.shape[slot_dim + 1:]
    if host is None:
        host = torch.empty(shape, dtype=t.dtype, pin_memory=True)
    _slot_transfer(_lib.WKV7_TO_HOST, t, slot, slot_dim, host, staging)
    return host


def slot_from_host(t: torch.Tensor, slot: int, slot_dim: int, host: torch.Tensor,
                   staging: torch.Tensor | None = None) -> None:
    """Asynchronous copy of a dense pinned host tensor (shaped like
    ``t.select(slot_dim, slot)``) into one slot's rows of ``t``; ``staging``
    as for ``slot_to_host``."""
    _slot_transfer(_lib.WKV7_FROM_HOST, t, slot, slot_dim, host, staging)


def _overlaps(x: torch.Tensor, y: torch.Tensor) -> bool:
    return x.untyped_storage().data_ptr() == y.untyped_storage().data_ptr()


def slot_zero(t: torch.Tensor, ids, slot_dim: int) -> None:
    """Zero slot rows ``ids`` of ``t`` along ``slot_dim`` with a fill kernel."""
    _require_cuda(t, "tensor")
    outer, os_, ss, rows, rb = slot_view(t, slot_dim)
    ids_t = device_ids(ids, rows, t.device, "ids", distinct=False)
    n = int(ids_t.shape[0])
    if n == 0:
        return
    rc = _lib.load().wkv7_slot_zero(t.data_ptr(), os_, ss, rows, ids_t.data_ptr(), outer, rb, n,
                                    _stream_ptr(t.device))
    _lib.check(rc, "wkv7_slot_zero")


# -- time-mix stages around the WKV op ------------------------------------------------

def _bf16_2d(t: torch.Tensor, what: str, shape: tuple[int, ...] | None = None) -> torch.Tensor:
    _require_cuda(t, what)
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{what} must be bfloat16, got {t.dtype}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{what} must be {tuple(shape)}, got {tuple(t.shape)}")
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def seq_plan(slot_ids, cu_seqlens, rows: int, T: int,
             device: torch.device) -> tuple[torch.Tensor, torch.Tensor, int]:
    """Device ``(slot_ids, cu_seqlens, nseq)`` for a ragged token batch.
    ``cu_seqlens=None`` is a decode batch (one token per slot). Host inputs
    are validated and uploaded in one copy; device tensors pass through."""
    if isinstance(slot_ids, torch.Tensor) and slot_ids.is_cuda:
        ids = device_ids(slot_ids, rows, device, "slot_ids")
        nseq = int(ids.shape[0])
        if cu_seqlens is None:
            if nseq != T:
                raise ValueError(f"{nseq} slots for {T} decode tokens")
            cu = torch.arange(nseq + 1, dtype=torch.int32, device=device)
        elif isinstance(cu_seqlens, torch.Tensor) and cu_seqlens.is_cuda:
            if cu_seqlens.dtype != torch.int32 or cu_seqlens.shape != (nseq + 1,):
                raise ValueError("device cu_seqlens must be int32 [nseq + 1]")
            cu = cu_seqlens
        else:
            lst = _host_cu(cu_seqlens, T)
            if len(lst) != nseq + 1:
                raise ValueError(f"cu_seqlens has {len(lst)} entries for {nseq} sequences")
            cu = torch.tensor(lst, dtype=torch.int32, device=device)
        return ids, cu, nseq
    lst = host_ids(slot_ids, rows, "slot_ids", distinct=True)
    nseq = len(lst)
    if cu_seqlens is None:
        if nseq != T:
            raise ValueError(f"{nseq} slots for {T} decode tokens")
        cu_l = list(range(nseq + 1))
    else:
        cu_l = _host_cu(cu_seqlens, T)
        if len(cu_l) != nseq + 1:
            raise ValueError(f"cu_seqlens has {len(cu_l)} entries for {nseq} sequences")
    both = torch.tensor(lst + cu_l, dtype=torch.int32, device=device)
    return both[:nseq], both[nseq:], nseq


def token_shift_mix(x: torch.Tensor, shift_rows: torch.Tensor, slot_ids, mix: torch.Tensor,
                    cu_seqlens=None, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """Token shift of one state family fused with its lerp mixes.

    ``x [T, D]`` bf16 (the mixer's input), ``shift_rows [rows, D]`` bf16 (one
    layer and family of ``bank.shift``, e.g. ``bank.shift[l, 0]``), ``mix
    [M, D]`` bf16. ``cu_seqlens=None`` means one token per slot (decode; the
    kernel then gets no offsets). Returns ``out [M, T, D]``:
    ``bf16(x + bf16(prev - x) * mix[m])`` with prev the previous token, or the
    slot's row for a sequence's first token; each sequence's last row of ``x``
    becomes its slot's row (in place)."""
    _require_cuda(shift_rows, "shift_rows")
    if shift_rows.dtype != torch.bfloat16 or shift_rows.dim() != 2 or shift_rows.stride(1) != 1:
        raise ValueError("shift_rows must be a bf16 [rows, D] view with unit channel stride")
    rows, D = int(shift_rows.shape[0]), int(shift_rows.shape[1])
    if x.dim() != 2 or int(x.shape[1]) != D:
        raise ValueError(f"x must be [T, {D}], got {tuple(x.shape)}")
    x = _bf16_2d(x, "x")
    T = int(x.shape[0])
    if mix.dim() != 2 or int(mix.shape[1]) != D:
        raise ValueError(f"mix must be [M, {D}], got {tuple(mix.shape)}")
    mix = _bf16_2d(mix, "mix")
    M = int(mix.shape[0])
    dev = x.device
    if shift_rows.device != dev or mix.device != dev:
        raise ValueError("x, shift_rows and mix must share a device")
    if D % 8 or shift_rows.stride(0) % 8 or shift_rows.data_ptr() % 16:
        raise ValueError("D and the shift row stride must be multiples of 8 (16-byte rows)")
    if cu_seqlens is None:  # decode: sequence t is token t, no offsets
        ids = device_ids(slot_ids, rows, dev, "slot_ids")
        nseq, cu = int(ids.shape[0]), None
        if nseq != T:
            raise ValueError(f"{nseq} slots for {T} decode tokens")
    else:
        ids, cu, nseq = seq_plan(slot_ids, cu_seqlens, rows, T, dev)
    y = _out(out, (M, T, D), torch.bfloat16, dev, "out")
    if y.dtype != torch.bfloat16 or y.data_ptr() % 16:
        raise ValueError("out must be a 16-byte aligned bf16 tensor")
    if T == 0 or nseq == 0:
        return y
    rc = _lib.load().wkv7_token_shift_mix(x.data_ptr(), T, D, shift_rows.data_ptr(), rows,
                                          int(shift_rows.stride(0)), ids.data_ptr(),
                                          _ptr(cu), nseq, mix.data_ptr(), M, y.data_ptr(),
                                          T * D, _stream_ptr(dev))
    _lib.check(rc, "wkv7_token_shift_mix")
    return y


def time_mix_inputs(H: int, k, v, w_lora, a_lora, k_k, k_a, v_lora=None, v_first=None):
    """WKV op inputs from the time-mix projections, all ``[T, H*64]`` bf16
    (``k_k``, ``k_a`` ``[H*64]``). ``v_lora``/``v_first`` are given together
    (layers after the first). Returns ``(w, k, v, a, b)`` ``[T, H*64]`` bf16
    with w the log-decay."""
    D = int(H) * HEAD_SIZE
    T = int(k.shape[0]) if k.dim() == 2 else -1
    shape = (T, D)
    k = _bf16_2d(k, "k", shape)
    dev = k.device
    v, w_lora, a_lora = (_bf16_2d(t, n, shape) for t, n in
                         ((v, "v"), (w_lora, "w_lora"), (a_lora, "a_lora")))
    k_k = _bf16_2d(k_k.reshape(-1), "k_k", (D,))
    k_a = _bf16_2d(k_a.reshape(-1), "k_a", (D,))
    if (v_lora is None) != (v_first is None):
        raise ValueError("v_lora and v_first go together")
    if v_lora is not None:
        v_lora = _bf16_2d(v_lora, "v_lora", shape)
        v_first = _bf16_2d(v_first, "v_first", shape)
    for t in (v, w_lora, a_lora, k_k, k_a) + (() if v_lora is None else (v_lora, v_first)):
        if t.device != dev:
            raise ValueError("time-mix inputs must share a device")
    outs = torch.empty((5, T, D), dtype=torch.bfloat16, device=dev)
    if T == 0:
        return tuple(outs)
    rc = _lib.load().wkv7_time_mix_inputs(T, int(H), k.data_ptr(), v.data_ptr(),
                                          w_lora.data_ptr(), a_lora.data_ptr(), _ptr(v_lora),
                                          _ptr(v_first), k_k.data_ptr(), k_a.data_ptr(),
                                          *[o.data_ptr() for o in outs], _stream_ptr(dev))
    _lib.check(rc, "wkv7_time_mix_inputs")
    return tuple(outs)


def time_mix_output(H: int, y, r, k, v, g, r_k, ln_w, ln_b, eps: float,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """Per-head GroupNorm of the WKV output ``y [T, H, 64]`` (bf16 or fp32)
    plus the bonus term ``(sum r k r_k) v``, times the gate ``g``; every other
    tensor ``[T, H*64]`` bf16, ``r_k``/``ln_w``/``ln_b`` ``[H*64]``. Returns
    the output projection's input ``[T, H*64]`` bf16."""
    D = int(H) * HEAD_SIZE
    _require_cuda(y, "y")
    T = int(y.shape[0])
    if tuple(y.shape) not in ((T, int(H), HEAD_SIZE), (T, D)):
        raise ValueError(f"y must be [T, {H}, 64], got {tuple(y.shape)}")
    code = _y_code(y.dtype)
    y = y.contiguous()
    if y.data_ptr() % 16:
        y = y.clone()
    dev = y.device
    r, k, v, g = (_bf16_2d(t, n, (T, D)) for t, n in ((r, "r"), (k, "k"), (v, "v"), (g, "g")))
    r_k, ln_w, ln_b = (_bf16_2d(t.reshape(-1), n, (D,)) for t, n in
                       ((r_k, "r_k"), (ln_w, "ln_w"), (ln_b, "ln_b")))
    for t in (r, k, v, g, r_k, ln_w, ln_b):
        if t.device != dev:
            raise ValueError("time-mix output tensors must share a device")
    o = _out(out, (T, D), torch.bfloat16, dev, "out")
    if T == 0:
        return o
    rc = _lib.load().wkv7_time_mix_output(T, int(H), y.data_ptr(), code, r.data_ptr(),
                                          k.data_ptr(), v.data_ptr(), g.data_ptr(),
                                          r_k.data_ptr(), ln_w.data_ptr(), ln_b.data_ptr(),
                                          float(eps), o.data_ptr(), _stream_ptr(dev))
    _lib.check(rc, "wkv7_time_mix_output")
    return o


def wkv7_decode_block(wkv_layer: torch.Tensor, slot_ids, H: int, r, k, v, w_lora, a_lora, g,
                      k_k, k_a, r_k, ln_w, ln_b, eps: float, *, v_lora=None, v_first=None,
                      row_order=None, scale: float = 1.0, want_v: bool = False,
                      out: torch.Tensor | None = None):
    """The time-mix decode of one token per slot in one launch
    (``wkv7_decode_block``): ``time_mix_inputs`` -> in-place WKV decode of
    ``wkv_layer`` (bf16 y) -> ``time_mix_output``, bit-identical to those three
    calls. Row vectors ``[B, H*64]`` bf16, parameters ``[H*64]``. Returns
    ``out [B, H*64]`` (the output projection's input), and with ``want_v``
    also the WKV op's v (the first layer's is v_first for the others)."""
    rows, pool_heads = _check_pool(wkv_layer)
    if pool_heads != int(H):
        raise ValueError(f"pool has {pool_heads} heads, H = {H}")
    dev = wkv_layer.device
    ids = device_ids(slot_ids, rows, dev, "slot_ids")
    B, D = int(ids.shape[0]), int(H) * HEAD_SIZE
    if (v_lora is None) != (v_first is None):
        raise ValueError("v_lora and v_first go together (both None for the first layer)")
    vecs = [_bf16_2d(t, n, (B, D)) for t, n in ((r, "r"), (k, "k"), (v, "v"), (w_lora, "w_lora"),
                                                 (a_lora, "a_lora"), (g, "g"))]
    lora = [None, None] if v_lora is None else [_bf16_2d(v_lora, "v_lora", (B, D)),
                                                 _bf16_2d(v_first, "v_first", (B, D))]
    params = [_bf16_2d(t.reshape(-1), n, (D,)) for t, n in ((k_k, "k_k"), (k_a, "k_a"),
                                                            (r_k, "r_k"), (ln_w, "ln_w"),
                                                            (ln_b, "ln_b"))]
    for t in vecs + params + [x for x in lora if x is not None]:
        if t.device != dev:
            raise ValueError("decode block tensors must share the pool's device")
    o = _out(out, (B, D), torch.bfloat16, dev, "out")
    v_out = torch.empty((B, D), dtype=torch.bfloat16, device=dev) if want_v else None
    order = None
    if row_order is not None:
        order = device_ids(row_order, B, dev, "row_order")
    if B:
        rc = _lib.load().wkv7_decode_block(
            wkv_layer.data_ptr(), rows, int(H), ids.data_ptr(), _ptr(order), B,
            *(t.data_ptr() for t in vecs[:5]), _ptr(lora[0]), _ptr(lora[1]), vecs[5].data_ptr(),
            *(t.data_ptr() for t in params), float(eps), float(scale), o.data_ptr(),
            _ptr(v_out), _stream_ptr(dev))
        _lib.check(rc, "wkv7_decode_block")
    return (o, v_out) if want_v else o


ACTIVATIONS = {None: _lib.WKV7_ACT_NONE, "tanh": _lib.WKV7_ACT_TANH,
               "sigmoid": _lib.WKV7_ACT_SIGMOID}


def proj_grouped(products: Sequence[tuple], outs: Sequence[torch.Tensor | None] | None = None,
                 ) -> list[torch.Tensor]:
    """Independent projections ``act(x @ w.T + bias)`` in one launch
    (``wkv7_proj_grouped``): ``products`` holds up to 8 tuples ``(x, w)``,
    ``(x, w, bias)`` or ``(x, w, bias, act)`` with ``x [M, k]`` (row stride
    a multiple of 8, unit column stride), ``w [n, k]`` bf16 (nn.Linear's
    [out, in]), ``bias [n]`` or None and ``act`` None, ``"tanh"`` or
    ``"sigmoid"``; every ``x`` has the same M. Returns the ``[M, n]`` bf16
    outputs (written into ``outs[i]`` where given, which may be strided
    row views)."""
    if not 1 <= len(products) <= _lib.WKV7_PROJ_MAX_GROUPS:
        raise ValueError(f"1..{_lib.WKV7_PROJ_MAX_GROUPS} products per launch, got {len(products)}")
    groups = (_lib.ProjGroup * len(products))()
    ys, keep = [], []
    M = None
    for i, prod in enumerate(products):
        x, w = prod[0], prod[1]
        bias = prod[2] if len(prod) > 2 else None
        act = prod[3] if len(prod) > 3 else None
        if act not in ACTIVATIONS:
            raise ValueError(f"act must be one of {list(ACTIVATIONS)}, got {act!r}")
        for t, n in ((x, "x"), (w, "w")):
            _require_cuda(t, n)
            if t.dtype != torch.bfloat16 or t.dim() != 2:
                raise ValueError(f"{n} must be a 2-D bfloat16 tensor")
        if x.stride(1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
            x = x.clone(memory_format=torch.contiguous_format)
        w = _bf16_2d(w, "w")
        m, k = int(x.shape[0]), int(x.shape[1])
        n = int(w.shape[0])
        if M is None:
            M = m
        if m != M:
            raise ValueError("every product needs the same row count")
        if int(w.shape[1]) != k:
            raise ValueError(f"w must be [n, {k}], got {tuple(w.shape)}")
        if k < 32 or k % 32:
            raise ValueError(f"k must be a positive multiple of 32, got {k}")
        if bias is not None:
            bias = _bf16_2d(bias.reshape(-1), "bias", (n,))
        y = outs[i] if outs is not None and i < len(outs) else None
        if y is None:
            y = torch.empty((M, n), dtype=torch.bfloat16, device=x.device)
        else:
            _require_cuda(y, "out")
            if y.dtype != torch.bfloat16 or tuple(y.shape) != (M, n) or y.stride(1) != 1:
                raise ValueError(f"out must be a bf16 [{M}, {n}] tensor with unit column stride")
        for t in (w, y) + ((bias,) if bias is not None else ()):
            if t.device != x.device:
                raise ValueError("projection tensors must share a device")
        groups[i] = _lib.ProjGroup(x.data_ptr(), w.data_ptr(), _ptr(bias), y.data_ptr(),
                                   x.stride(0), w.stride(0), y.stride(0), n, k,
                                   ACTIVATIONS[act], 0)
        keep += [x, w, bias]
        ys.append(y)
    if M:
        lib = _lib.load()
        n = len(products)
        ws_bytes = int(lib.wkv7_proj_workspace_bytes(M, groups, n))
        ws = (torch.empty(ws_bytes, dtype=torch.uint8, device=ys[0].device) if ws_bytes
              else None)
        rc = lib.wkv7_proj_grouped(M, groups, n, _ptr(ws), ws_bytes,
                                   _stream_ptr(ys[0].device))
        _lib.check(rc, "wkv7_proj_grouped")
    return ys


# -- fla wkv-op signatures --------------------------------------------------------------

def auto_segments(H: int, lens: Sequence[int], device: torch.device) -> int:
    """Segments per sequence for ``wkv7_prefill_segments`` when a one-pass
    launch would leave most compute units idle: the busy (sequence, head)
    workgroups fill at most a quarter of the GPU and the longest sequence has
    at least 2,048 tokens (below that the split does not pay). G segments
    take 2G - 1 workgroups per (sequence, head)."""
    busy = sum(1 for n in lens if n > 0) * H
    if busy == 0 or max(lens) < 2048:
        return 1
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    if 4 * busy > cus:
        return 1
    return max(1, min(4, (cus // busy + 1) // 2))


def _fla_state(initial_state, nseq: int, H: int, dev: torch.device) -> torch.Tensor | None:
    if initial_state is None:
        return None
    if tuple(initial_state.shape) != (nseq, H, HEAD_SIZE, HEAD_SIZE):
        raise ValueError(f"initial_state must be {(nseq, H, HEAD_SIZE, HEAD_SIZE)}, "
                         f"got {tuple(initial_state.shape)}")
    return initial_state.to(device=dev, dtype=torch.float32).contiguous()


def _seq_op(r, w, k, v, a, b, scale, initial_state, output_final_state, cu_seqlens, head_first):
    """fla's wkv-op contract: ``[B, T, H, 64]`` inputs (or ``[1, T_total, H,
    64]`` packed by ``cu_seqlens``), ``initial_state`` read, a new
    ``final_state`` returned. One token per sequence runs the decode kernel
    and longer sequences the chunked scan, both out of place (initial_state ->
    final_state, no copy of the state)."""
    if head_first:
        r, w, k, v, a, b = (x.transpose(1, 2) for x in (r, w, k, v, a, b))
    _require_cuda(r, "r")
    if r.dim() != 4:
        raise ValueError("inputs must be [B, T, H, K]")
    B, T, H, K = (int(d) for d in r.shape)
    if K != HEAD_SIZE:
        raise ValueError(f"head size must be {HEAD_SIZE}, got {K}")
    if r.dtype != torch.bfloat16:
        raise ValueError("the gfx950 WKV7 kernels take bfloat16 inputs")
    if cu_seqlens is None:
        nseq = B
        host_cu = [i * T for i in range(B + 1)]
        flat = [x.reshape(B * T, H, K) for x in (r, w, k, v, a, b)]
    else:
        if B != 1:
            raise ValueError("cu_seqlens requires batch size 1 (packed sequences)")
        # fla passes a device LongTensor; the offsets are validated on the host
        host_cu = _host_cu(cu_seqlens, T)
        nseq = len(host_cu) - 1
        flat = [x[0] for x in (r, w, k, v, a, b)]
    dev = r.device
    state = _fla_state(initial_state, nseq, H, dev)
    lens = [host_cu[i + 1] - host_cu[i] for i in range(nseq)]
    if nseq and all(n == 1 for n in lens):  # decode: one token per sequence
        final = (torch.empty((nseq, H, K, K), dtype=torch.float32, device=dev)
                 if output_final_state else None)
        y = wkv7_decode_into(state, final, *flat, scale=scale, out_dtype=r.dtype)
        o = y.reshape(B, T, H, K)
        return (o.transpose(1, 2) if head_first else o), final
    G = auto_segments(H, lens, dev)
    if G > 1:  # few long sequences: run their segments side by side
        # the segment chain needs the final states in a pool of its own
        pool = torch.empty((nseq, H, K, K), dtype=torch.float32, device=dev)
        y = wkv7_prefill_segments(pool, list(range(nseq)), host_cu, *flat, segments=G,
                                  zero_init=state is None, scale=scale, out_dtype=r.dtype,
                                  state_in=state)
        final = pool if output_final_state else None
    else:
        # state read from initial_state, written to a new final_state: no copy
        final = (torch.empty((nseq, H, K, K), dtype=torch.float32, device=dev)
                 if output_final_state else None)
        y = wkv7_prefill_into(state, final, host_cu, *flat, scale=scale, out_dtype=r.dtype)
    o = y.reshape(B, T, H, K)
    if head_first:
        o = o.transpose(1, 2)
    return o, final


def fused_recurrent_rwkv7(r, w, k, v, a, b, scale: float = 1.0, initial_state=None,
                          output_final_state: bool = True, cu_seqlens=None,
                          head_first: bool = False):
    """fla-signature recurrent WKV7 (the reference's decode / T < 64 path,
    wkvm/models/rwkv7.py:108-111).

    Tensors ``[B, T, H, 64]`` bf16 (``w`` log-decay); ``initial_state``
    ``[N, H, 64, 64]`` fp32 with N = B, or the number of packed sequences when
    ``cu_seqlens`` is given (a host sequence or a device tensor of any integer
    dtype). Returns ``(o, final_state)``; ``initial_state`` is not modified.
    One token per sequence runs ``wkv7_decode_into``: the state is read from
    ``initial_state`` and written to a new ``final_state`` (or not at all when
    ``output_final_state`` is False), with no copy.
    """
    return _seq_op(r, w, k, v, a, b, scale, initial_state, output_final_state, cu_seqlens,
                   head_first)


def chunk_rwkv7(r, w, k, v, a, b, scale: float = 1.0, initial_state=None,
                output_final_state: bool = True, cu_seqlens=None, head_first: bool = False):
    """fla-signature chunked WKV7 (the reference's prefill path, T >= 64).
    Same arguments and results as ``fused_recurrent_rwkv7``. Few long
    sequences (``auto_segments``) run segmented, to fp32 rounding of the
    one-pass result."""
    return _seq_op(r, w, k, v, a, b, scale, initial_state, output_final_state, cu_seqlens,
                   head_first)


def ids_list(slot_batch: Iterable[dict], family: str) -> list[int]:
    """Slot ids of one family from a list of arena slot dicts (wkvm/core/arena.py:55-67)."""
    return [int(s[family]) for s in slot_batch]
