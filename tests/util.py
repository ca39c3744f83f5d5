"""Comparison helpers shared by the GPU parity tests."""

from __future__ import annotations

import numpy as np
import torch

import oracle as O


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor (any device) -> numpy uint16 bit patterns."""
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().double().cpu().numpy()


def normwise_max(x: np.ndarray, ref: np.ndarray, tile_dims: int = 2) -> float:
    """max over tiles of max|x - ref| / max|ref|, tiles = the last
    ``tile_dims`` dims (e.g. one 64x64 head state, or one head's y vector)."""
    d = np.abs(x - ref).reshape(-1, *ref.shape[-tile_dims:])
    m = np.abs(ref).reshape(-1, *ref.shape[-tile_dims:])
    axes = tuple(range(1, tile_dims + 1))
    return float(np.max(d.max(axis=axes) / np.maximum(m.max(axis=axes), 1e-30)))


def rel_l2(x: np.ndarray, ref: np.ndarray) -> float:
    return float(np.linalg.norm(x - ref) / max(np.linalg.norm(ref), 1e-300))


def bf16_ulp_distance(y_bits: np.ndarray, ref: np.ndarray) -> np.ndarray:
    """Distance in bf16 ulps between kernel output bits and the float64
    reference rounded to bf16 (same-sign values; sign flips count large)."""
    rb = O.f32_to_bf16_bits(np.asarray(ref, dtype=np.float32)).astype(np.int64)
    yb = y_bits.astype(np.int64)

    def ordered(b):  # map sign-magnitude bits to a monotone integer line
        return np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)

    return np.abs(ordered(yb) - ordered(rb))


def vec_bits(vecs: dict[str, torch.Tensor]) -> list[np.ndarray]:
    return [bits(vecs[n]) for n in "rwkvab"]


def bf16_y_excess(y_bits: np.ndarray, ref: np.ndarray, tol: float = 1e-5) -> float:
    """How far a bf16 output exceeds its bar, as a multiple of the bar (<= 1
    passes). The bar per element is the fp32 contract plus the output's own
    rounding: tol * max|ref| over the (row, head) vector (the last dim) plus
    one bf16 ulp of ref. One ulp alone would be stricter than the fp32
    contract for outputs near zero, where the summands cancel."""
    y = O.bf16_bits_to_f64(y_bits).reshape(ref.shape)
    tile = np.abs(ref).max(axis=-1, keepdims=True)
    ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64) * 65536.0
    bar = tol * tile + ulp
    return float(np.max(np.abs(y - ref) / bar))
