"""CPU oracle for the WKV7 slot-pool recurrence.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg, never by the product package
``wkvm_amd``. See ``wkv7_oracle.c`` for the restated recurrence and the
reference files it follows.

Contents:

* ``scan_f64`` / ``scan_bf16`` / ``decode_slots_f64`` / ``prefill_f64`` --
  float64 stepwise scan (C, OpenMP) over ragged sequences; the parity checker
  (``scan_bf16`` takes the bf16 bit patterns and fp32 pool rows directly).
* ``chunked_scan_f64`` -- an independent numpy restatement in chunked (WY)
  form, the algebra the HIP prefill kernel implements; cross-checked against
  the stepwise scan.
* ``transition_product_f64`` -- the recurrence as an explicit product of
  transition matrices M_t = diag(w_t) + a_t b_t^T (numpy matmul), used to pin
  the stepwise scan on small inputs and to produce the golden vectors.
* ``slot_copy_np`` / ``slot_gather_np`` / ``slot_scatter_np`` -- the byte
  semantics of the reference's slot views (``index_select``/``index_copy_`` in
  wkvm/runner/state.py:63-97, slice copies in wkvm/store.py:130-131,151-152).
* ``port_*_f32`` -- float32 C restatements with the product's interface, timed
  as the CPU baseline only.

Parity status: every function here is pinned by tests/test_oracle.py (closed
forms, invariants, the product form and golden vectors); none is "unpinned".
"""

from __future__ import annotations

import ctypes
import os
import subprocess
import threading

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libwkv7_oracle.so")
_lib = None
_lock = threading.Lock()

_i64p = ctypes.POINTER(ctypes.c_int64)
_i32p = ctypes.POINTER(ctypes.c_int32)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_f64p = ctypes.POINTER(ctypes.c_double)
_f32p = ctypes.POINTER(ctypes.c_float)


def build(force: bool = False) -> str:
    """Compile the C oracle with gcc (oracle/Makefile) and return its path."""
    src = os.path.join(_HERE, "wkv7_oracle.c")
    stale = (not os.path.exists(_LIB_PATH)) or os.path.getmtime(_LIB_PATH) < os.path.getmtime(src)
    if force or stale:
        args = ["make", "-s", "-C", _HERE] + (["-B"] if force else [])
        subprocess.run(args,
                       check=True, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    return _LIB_PATH


def _load():
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        lib.wkv7_oracle_scan_f64.restype = ctypes.c_int
        lib.wkv7_oracle_scan_f64.argtypes = [
            ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _i64p, _f64p,
            _f64p, _f64p, _f64p, _f64p, _f64p, _f64p, ctypes.c_double, _f64p, _f64p]
        lib.wkv7_oracle_scan_bf16.restype = ctypes.c_int
        lib.wkv7_oracle_scan_bf16.argtypes = [
            ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _i64p, _f32p, ctypes.c_int64, _i32p,
            _u16p, _u16p, _u16p, _u16p, _u16p, _u16p, ctypes.c_double, _f64p, _f64p]
        lib.wkv7_port_decode_slots_f32.restype = ctypes.c_int
        lib.wkv7_port_decode_slots_f32.argtypes = [
            _f32p, ctypes.c_int64, ctypes.c_int64, _i32p, ctypes.c_int64,
            _u16p, _u16p, _u16p, _u16p, _u16p, _u16p, ctypes.c_float, _u16p]
        lib.wkv7_port_prefill_f32.restype = ctypes.c_int
        lib.wkv7_port_prefill_f32.argtypes = [
            _f32p, ctypes.c_int64, ctypes.c_int64, _i32p, _i64p, ctypes.c_int64,
            _u16p, _u16p, _u16p, _u16p, _u16p, _u16p, ctypes.c_int, ctypes.c_float, _u16p]
        lib.wkv7_oracle_set_threads.argtypes = [ctypes.c_int]
        lib.wkv7_oracle_max_threads.restype = ctypes.c_int
        lib.wkv7_oracle_bf16_to_double.argtypes = [ctypes.c_uint16]
        lib.wkv7_oracle_bf16_to_double.restype = ctypes.c_double
        lib.wkv7_oracle_float_to_bf16.argtypes = [ctypes.c_float]
        lib.wkv7_oracle_float_to_bf16.restype = ctypes.c_uint16
        _lib = lib
        return lib


def set_threads(n: int) -> None:
    _load().wkv7_oracle_set_threads(int(n))


def max_threads() -> int:
    return int(_load().wkv7_oracle_max_threads())


# -- bf16 helpers (numpy has no bfloat16; bf16 tensors travel as uint16 bits) --

def bf16_bits_to_f64(bits: np.ndarray) -> np.ndarray:
    """Exact widening of bf16 bit patterns (uint16) to float64."""
    u = np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16
    return u.view(np.float32).astype(np.float64)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bit patterns (uint16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    quiet = ((u >> 16) | 0x40).astype(np.uint16)
    return np.where(nan, quiet, rounded)


def round_f64_to_bf16(x: np.ndarray) -> np.ndarray:
    """float64 -> nearest bf16 value (via float32, as a bf16 output store does
    when the kernel accumulates in fp32), returned as float64."""
    return bf16_bits_to_f64(f32_to_bf16_bits(np.asarray(x, dtype=np.float32)))


def _ptr(a: np.ndarray, p):
    return a.ctypes.data_as(p)


# -- float64 stepwise scan ------------------------------------------------------

def scan_f64(cu_seqlens, r, w, k, v, a, b, h0=None, scale: float = 1.0):
    """Stepwise float64 scan over ragged sequences.

    ``r, w, k, v, a, b``: ``[T, H, N]`` (any float dtype; ``w`` is log-decay).
    ``cu_seqlens``: ``[nseq+1]`` token offsets. ``h0``: ``[nseq, H, N, N]`` in the
    bank orientation ``h[j(key), i(value)]``, or None for zero state.
    Returns ``(y [T,H,N], hT [nseq,H,N,N])`` as float64.
    """
    lib = _load()
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int64)
    nseq = cu.shape[0] - 1
    ins = [np.ascontiguousarray(x, dtype=np.float64) for x in (r, w, k, v, a, b)]
    T, H, N = ins[0].shape
    for x in ins:
        if x.shape != (T, H, N):
            raise ValueError("inputs must share one [T, H, N] shape")
    if nseq < 0 or cu[0] != 0 or cu[-1] != T:
        raise ValueError("cu_seqlens must start at 0 and end at T")
    y = np.zeros((T, H, N), dtype=np.float64)
    hT = np.zeros((max(nseq, 0), H, N, N), dtype=np.float64)
    h0p = None
    if h0 is not None:
        h0c = np.ascontiguousarray(h0, dtype=np.float64)
        if h0c.shape != (nseq, H, N, N):
            raise ValueError("h0 must be [nseq, H, N, N]")
        h0p = _ptr(h0c, _f64p)
    rc = lib.wkv7_oracle_scan_f64(nseq, H, N, _ptr(cu, _i64p), h0p,
                                  *[_ptr(x, _f64p) for x in ins], float(scale),
                                  _ptr(y, _f64p), _ptr(hT, _f64p))
    if rc != 0:
        raise RuntimeError(f"wkv7_oracle_scan_f64 failed: {rc}")
    return y, hT


def scan_bf16(cu_seqlens, r, w, k, v, a, b, pool=None, slot_ids=None, scale: float = 1.0):
    """``scan_f64`` for bf16 inputs given as uint16 bit patterns ``[T, H, N]``.

    The initial state of sequence s is ``pool[slot_ids[s]]`` (float32 numpy
    ``[rows, H, N, N]``), or zero when ``pool`` is None. Inputs are widened
    exactly to float64 inside the C loop, so full-size cases need no float64
    copies. Returns ``(y [T,H,N], hT [nseq,H,N,N])`` float64.
    """
    lib = _load()
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int64)
    nseq = cu.shape[0] - 1
    ins = [np.ascontiguousarray(x, dtype=np.uint16) for x in (r, w, k, v, a, b)]
    T, H, N = ins[0].shape
    for x in ins:
        if x.shape != (T, H, N):
            raise ValueError("inputs must share one [T, H, N] shape")
    if nseq < 0 or cu[0] != 0 or cu[-1] != T:
        raise ValueError("cu_seqlens must start at 0 and end at T")
    y = np.zeros((T, H, N), dtype=np.float64)
    hT = np.zeros((max(nseq, 0), H, N, N), dtype=np.float64)
    pool_p, ids_p, rows = None, None, 0
    if pool is not None:
        poolc = np.ascontiguousarray(pool, dtype=np.float32)
        if poolc.shape[1:] != (H, N, N):
            raise ValueError("pool must be [rows, H, N, N]")
        ids = np.ascontiguousarray(slot_ids, dtype=np.int32)
        if ids.shape != (nseq,):
            raise ValueError("slot_ids must have one id per sequence")
        pool_p, ids_p, rows = _ptr(poolc, _f32p), _ptr(ids, _i32p), poolc.shape[0]
    rc = lib.wkv7_oracle_scan_bf16(nseq, H, N, _ptr(cu, _i64p), pool_p, rows, ids_p,
                                   *[_ptr(x, _u16p) for x in ins], float(scale),
                                   _ptr(y, _f64p), _ptr(hT, _f64p))
    if rc != 0:
        raise RuntimeError(f"wkv7_oracle_scan_bf16 failed: {rc}")
    return y, hT


def decode_slots_f64(pool, slot_ids, r, w, k, v, a, b, scale: float = 1.0):
    """One decode step for a slot batch against a float32 pool.

    ``pool``: ``[rows, H, N, N]`` (one layer of the bank); ``slot_ids``: ``[B]``;
    inputs ``[B, H, N]``. Returns ``(y [B,H,N], new_state [B,H,N,N])`` float64;
    the pool is not modified.
    """
    ids = np.asarray(slot_ids, dtype=np.int64)
    h0 = np.asarray(pool, dtype=np.float64)[ids]
    cu = np.arange(ids.shape[0] + 1, dtype=np.int64)
    return scan_f64(cu, r, w, k, v, a, b, h0=h0, scale=scale)


def prefill_f64(pool, slot_ids, cu_seqlens, r, w, k, v, a, b, zero_init: bool, scale: float = 1.0):
    """Varlen prefill from slot states (or zero). Returns ``(y, final_states)``."""
    ids = np.asarray(slot_ids, dtype=np.int64)
    h0 = None if zero_init else np.asarray(pool, dtype=np.float64)[ids]
    return scan_f64(cu_seqlens, r, w, k, v, a, b, h0=h0, scale=scale)


# -- explicit transition-matrix product (small N brute force) --------------------

def transition_product_f64(r, w, k, v, a, b, h0=None, scale: float = 1.0):
    """Single sequence, written in the value-by-key orientation of the
    mathematical definition: ``S_t = S_{t-1} M_t + v_t k_t^T`` with
    ``M_t = diag(exp(w_t)) + a_t b_t^T`` and ``y_t = scale * S_t r_t``.

    Inputs ``[T, H, N]``; ``h0`` ``[H, N, N]`` in bank orientation (``h = S^T``).
    Returns ``(y [T,H,N], hT [H,N,N])`` in bank orientation. Computed with
    explicit dense matrix products, independently of the stepwise loop.
    """
    r, w, k, v, a, b = (np.asarray(x, dtype=np.float64) for x in (r, w, k, v, a, b))
    T, H, N = r.shape
    S = np.zeros((H, N, N)) if h0 is None else np.swapaxes(np.asarray(h0, np.float64), -1, -2).copy()
    ys = np.zeros((T, H, N))
    for t in range(T):
        M = np.zeros((H, N, N))
        idx = np.arange(N)
        M[:, idx, idx] = np.exp(w[t])
        M += a[t][:, :, None] * b[t][:, None, :]
        S = S @ M + v[t][:, :, None] * k[t][:, None, :]
        ys[t] = scale * (S @ r[t][:, :, None])[..., 0]
    return ys, np.swapaxes(S, -1, -2).copy()


# -- chunked (WY) restatement ------------------------------------------------------

def _chunk_step(h, r, w, k, v, a, b, scale, mm):
    """One chunk of c <= C tokens for one head, float64.

    h [K, V]; r..b [c, N]. Within the chunk, with G_t = sum_{s<=t} w_s
    (log-decay, inclusive) and G_0 = 0:
        A_hat[t] = a_t * exp(G_{t-1})        R_hat[t] = r_t * exp(G_t)
        B_til[s] = b_s * exp(-G_s)           K_til[s] = k_s * exp(-G_s)
        L_ab = tril(A_hat B_til^T, -1)       L_ak = tril(A_hat K_til^T, -1)
        M_rb = tril(R_hat B_til^T,  0)       M_rk = tril(R_hat K_til^T,  0)
        P    = (I - L_ab)^{-1} (A_hat h + L_ak V)      (p_t = a_t^T h_{t-1})
        Y    = R_hat h + M_rb P + M_rk V
        h'   = diag(exp(G_c)) h + B_bar^T P + K_bar^T V,
               B_bar[s] = b_s exp(G_c - G_s), K_bar[s] = k_s exp(G_c - G_s)
    ``mm(x, y)`` is the matrix product (lets callers model operand rounding).
    """
    c = r.shape[0]
    G = np.cumsum(w, axis=0)
    Gx = np.vstack([np.zeros((1, w.shape[1])), G[:-1]])
    A_hat = a * np.exp(Gx)
    R_hat = r * np.exp(G)
    B_til = b * np.exp(-G)
    K_til = k * np.exp(-G)
    lower = np.tril(np.ones((c, c), dtype=bool), -1)
    lower_eq = np.tril(np.ones((c, c), dtype=bool), 0)
    L_ab = np.where(lower, mm(A_hat, B_til.T), 0.0)
    L_ak = np.where(lower, mm(A_hat, K_til.T), 0.0)
    M_rb = np.where(lower_eq, mm(R_hat, B_til.T), 0.0)
    M_rk = np.where(lower_eq, mm(R_hat, K_til.T), 0.0)
    rhs = mm(A_hat, h) + mm(L_ak, v)
    P = np.linalg.solve(np.eye(c) - L_ab, rhs)
    Y = mm(R_hat, h) + mm(M_rb, P) + mm(M_rk, v)
    decay_end = np.exp(G[-1] - G)
    h_new = np.exp(G[-1])[:, None] * h + mm((b * decay_end).T, P) + mm((k * decay_end).T, v)
    return scale * Y, h_new


def chunked_scan_f64(cu_seqlens, r, w, k, v, a, b, h0=None, scale: float = 1.0,
                     chunk: int = 64, mm=None):
    """Chunked-form restatement of ``scan_f64`` (same arguments/returns).

    Sequences are cut into ``chunk``-token pieces from their first token; the
    last piece may be shorter. Independent of the stepwise C loop, so agreement
    between the two pins the chunk algebra the prefill kernel uses.
    """
    mm = mm or (lambda x, y: x @ y)
    r, w, k, v, a, b = (np.asarray(x, dtype=np.float64) for x in (r, w, k, v, a, b))
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    T, H, N = r.shape
    nseq = cu.shape[0] - 1
    y = np.zeros((T, H, N))
    hT = np.zeros((nseq, H, N, N))
    for s in range(nseq):
        for hd in range(H):
            h = np.zeros((N, N)) if h0 is None else np.array(h0[s, hd], dtype=np.float64)
            for t0 in range(int(cu[s]), int(cu[s + 1]), chunk):
                t1 = min(t0 + chunk, int(cu[s + 1]))
                sl = slice(t0, t1)
                y[sl, hd], h = _chunk_step(h, r[sl, hd], w[sl, hd], k[sl, hd], v[sl, hd],
                                           a[sl, hd], b[sl, hd], scale, mm)
            hT[s, hd] = h
    return y, hT


# -- slot byte semantics -------------------------------------------------------------

def slot_copy_np(t: np.ndarray, slot_dim: int, src, dst) -> np.ndarray:
    """``t[..., dst, ...] = t[..., src, ...]`` along ``slot_dim`` (reference
    fork/snapshot bytes: wkvm/store.py:130-131 then :151-152). Sources are
    read before any destination is written. Returns a new array."""
    out = np.array(t, copy=True)
    src = np.asarray(src, dtype=np.int64)
    dst = np.asarray(dst, dtype=np.int64)
    vals = np.take(t, src, axis=slot_dim)
    idx = [slice(None)] * t.ndim
    idx[slot_dim] = dst
    out[tuple(idx)] = vals
    return out


def slot_gather_np(t: np.ndarray, slot_dim: int, ids) -> np.ndarray:
    """``index_select(slot_dim, ids)`` (wkvm/runner/state.py:77-79)."""
    return np.take(t, np.asarray(ids, dtype=np.int64), axis=slot_dim)


def slot_scatter_np(t: np.ndarray, slot_dim: int, ids, rows: np.ndarray) -> np.ndarray:
    """``index_copy_(slot_dim, ids, rows)`` (wkvm/runner/state.py:91-97)."""
    out = np.array(t, copy=True)
    idx = [slice(None)] * t.ndim
    idx[slot_dim] = np.asarray(ids, dtype=np.int64)
    out[tuple(idx)] = rows
    return out


# -- float32 ports (CPU baseline only) ------------------------------------------------

def port_decode_slots_f32(pool: np.ndarray, slot_ids, r, w, k, v, a, b, scale: float = 1.0):
    """In-place fp32 decode on a numpy ``[rows, H, 64, 64]`` float32 pool with
    bf16-bit (uint16) inputs ``[B, H, 64]``; returns y as bf16 bits."""
    lib = _load()
    ids = np.ascontiguousarray(slot_ids, dtype=np.int32)
    ins = [np.ascontiguousarray(x, dtype=np.uint16) for x in (r, w, k, v, a, b)]
    B, H, N = ins[0].shape
    if N != 64 or pool.dtype != np.float32 or not pool.flags.c_contiguous:
        raise ValueError("port expects N=64 and a contiguous float32 pool")
    y = np.zeros((B, H, N), dtype=np.uint16)
    rc = lib.wkv7_port_decode_slots_f32(_ptr(pool, _f32p), pool.shape[0], H, _ptr(ids, _i32p), B,
                                        *[_ptr(x, _u16p) for x in ins], float(scale), _ptr(y, _u16p))
    if rc != 0:
        raise ValueError("bad slot ids")
    return y


def port_prefill_f32(pool: np.ndarray, slot_ids, cu_seqlens, r, w, k, v, a, b,
                     zero_init: bool, scale: float = 1.0):
    """In-place fp32 varlen prefill on a numpy pool; returns y as bf16 bits."""
    lib = _load()
    ids = np.ascontiguousarray(slot_ids, dtype=np.int32)
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int64)
    ins = [np.ascontiguousarray(x, dtype=np.uint16) for x in (r, w, k, v, a, b)]
    T, H, N = ins[0].shape
    y = np.zeros((T, H, N), dtype=np.uint16)
    rc = lib.wkv7_port_prefill_f32(_ptr(pool, _f32p), pool.shape[0], H, _ptr(ids, _i32p),
                                   _ptr(cu, _i64p), ids.shape[0], *[_ptr(x, _u16p) for x in ins],
                                   int(bool(zero_init)), float(scale), _ptr(y, _u16p))
    if rc != 0:
        raise ValueError("bad prefill arguments")
    return y
