"""ctypes binding of libwkv7.so (declarations in include/wkv7.h).

There is no fallback: if the library is missing, or no GPU is visible when a
compute entry point is called, this module raises. Loading works without a GPU
(the symbol table is what the CPU tests check).
"""

from __future__ import annotations

import ctypes
import os
import re
import threading

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG_DIR, "libwkv7.so")
HEADER_PATH = os.path.join(os.path.dirname(_PKG_DIR), "include", "wkv7.h")

# The ABI this binding is written for (WKV7_ABI_VERSION of include/wkv7.h);
# a library built from other sources is refused at load.
WKV7_ABI_VERSION = 10

WKV7_OK = 0
WKV7_ERR_ARG = -1
WKV7_ERR_SHAPE = -2
WKV7_ERR_WORKSPACE = -3
WKV7_Y_BF16 = 0
WKV7_Y_F32 = 1
WKV7_RUN_INIT_ZERO = 1
WKV7_RUN_INIT_IDENTITY = 2
WKV7_RUN_KV_ZERO = 4
WKV7_RUN_Y_ALT = 8
WKV7_RUN_STATE_ALT = 16
WKV7_TO_HOST = 0
WKV7_FROM_HOST = 1
WKV7_PROJ_MAX_GROUPS = 8
WKV7_PROJ_STATIC_SCRATCH_BYTES = 8 * 1024 * 1024
WKV7_ACT_NONE = 0
WKV7_ACT_TANH = 1
WKV7_ACT_SIGMOID = 2

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_sz = ctypes.c_size_t



class ProjGroup(ctypes.Structure):
    """struct wkv7_proj_group of include/wkv7.h."""
    _fields_ = [("x", _vp), ("w", _vp), ("bias", _vp), ("y", _vp), ("ldx", _i64),
                ("ldw", _i64), ("ldy", _i64), ("n", _i32), ("k", _i32), ("act", _i32),
                ("reserved", _i32)]


# name -> (restype, argtypes); must match include/wkv7.h.
SIGNATURES = {
    "wkv7_abi_version": (ctypes.c_int, []),
    "wkv7_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "wkv7_decode_slots": (ctypes.c_int, [
        _vp, _i64, _i32, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _f32, _vp]),
    "wkv7_decode_into": (ctypes.c_int, [
        _vp, _i64, _vp, _vp, _i64, _vp, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
        _i32, _f32, _vp]),
    "wkv7_prefill_varlen": (ctypes.c_int, [
        _vp, _i64, _i32, _vp, _vp, _vp, _i32, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32,
        _i32, _f32, _vp]),
    "wkv7_prefill_runs": (ctypes.c_int, [
        _vp, _i64, _i32, _vp, _vp, _vp, _i32, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32,
        _i32, _f32, _vp, _vp, _i32, _vp, _i64, _vp, _vp, _i64, _vp, _vp]),
    "wkv7_prefill_into": (ctypes.c_int, [
        _vp, _i64, _vp, _vp, _i64, _vp, _i32, _vp, _vp, _i32, _i64, _vp, _vp, _vp, _vp, _vp,
        _vp, _vp, _i32, _f32, _vp]),
    "wkv7_segment_chain": (ctypes.c_int, [
        _vp, _i64, _i32, _vp, _i64, _vp, _i32, _vp, _i32, _vp, _vp]),
    "wkv7_segment_correct": (ctypes.c_int, [
        _i64, _i32, _vp, _vp, _vp, _i32, _vp, _i32, _vp, _i32, _vp]),
    "wkv7_slot_copy": (ctypes.c_int, [
        _vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i32, _vp]),
    "wkv7_slot_zero": (ctypes.c_int, [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _i32, _vp]),
    "wkv7_slot_transfer": (ctypes.c_int, [_i32, _vp, _vp, _i64, _i64, _i64, _i32, _i64, _i64,
                                         _vp, _sz, _vp]),
    "wkv7_token_shift_mix": (ctypes.c_int, [
        _vp, _i64, _i32, _vp, _i64, _i64, _vp, _vp, _i32, _vp, _i32, _vp, _i64, _vp]),
    "wkv7_time_mix_inputs": (ctypes.c_int, [
        _i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "wkv7_time_mix_output": (ctypes.c_int, [
        _i64, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _f32, _vp, _vp]),
    "wkv7_proj_grouped": (ctypes.c_int, [_i64, ctypes.POINTER(ProjGroup), _i32, _vp, _sz, _vp]),
    "wkv7_proj_workspace_bytes": (_sz, [_i64, ctypes.POINTER(ProjGroup), _i32]),
    "wkv7_proj_grouped_noalloc": (ctypes.c_int, [_i64, ctypes.POINTER(ProjGroup), _i32, _vp]),
    "wkv7_decode_block": (ctypes.c_int, [
        _vp, _i64, _i32, _vp, _vp, _i32] + [_vp] * 13 + [_f32, _f32, _vp, _vp, _vp]),
}

_lib = None
_lock = threading.Lock()


class WKV7Error(RuntimeError):
    """A launch or runtime failure reported by libwkv7 (positive hipError_t)."""


def header_symbols(path: str = HEADER_PATH) -> list[str]:
    """Function names declared in include/wkv7.h."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(wkv7_[a-z_0-9]+)\s*\(", text, flags=re.M)


def load():
    """Load libwkv7.so (once) and attach the C signatures."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m wkvm_amd.build` "
                "(or __graft_entry__.build()) first -- there is no CPU fallback")
        lib = ctypes.CDLL(LIB_PATH)
        lib.wkv7_abi_version.restype = ctypes.c_int
        lib.wkv7_abi_version.argtypes = []
        found = int(lib.wkv7_abi_version())
        if found != WKV7_ABI_VERSION:
            raise RuntimeError(
                f"{LIB_PATH} has ABI version {found}, this package needs {WKV7_ABI_VERSION}; "
                "the library is stale -- rebuild it with `python -m wkvm_amd.build`")
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def strerror(code: int) -> str:
    return load().wkv7_strerror(int(code)).decode()


def check(code: int, what: str) -> None:
    """Raise for a nonzero return code (ValueError for rejected arguments)."""
    if code == WKV7_OK:
        return
    msg = f"{what}: {strerror(code)} (code {code})"
    if code < 0:
        raise ValueError(msg)
    raise WKV7Error(msg)
