"""CPU oracle for the RWKV-7 time-mix stages around the WKV7 op.

TEST INFRASTRUCTURE ONLY (like the rest of ``oracle/``): imported by
``tests/`` and never by the product package ``wkvm_amd``.

The reference delegates these stages to the third-party ``fla`` package
(RWKV7Attention; wkvm/models/rwkv7.py:108-113 loads it, the runner calls it
through the model forward, wkvm/runner/runner.py:80-88). ``fla`` is not
vendored, not version-pinned and not installed, so its exact bf16 rounding
sequence cannot be reproduced here. What the reference itself fixes, and this
oracle follows, is the token-shift state contract:

* ``conv_state`` / ``ffn_state`` are one ``[hidden]`` row per slot and layer,
  model dtype, in ``bank.shift[:, 0]`` / ``bank.shift[:, 1]``
  (wkvm/runner/state.py:40-46, wkvm/models/rwkv7.py:17-20);
* a zero row is the zero shift-in at position 0 of a fresh sequence
  (wkvm/models/rwkv7.py:25-27);
* the row carried to the next chunk or step is the last token's mixer input,
  so chunked prefill equals one pass (wkvm/runner/runner.py:12-14).

The arithmetic of each stage is restated from the RWKV-7 time-mix definition
with the rounding contract of ``include/wkv7.h`` (fp32 arithmetic, one bf16
rounding per output; ``delta`` rounded to bf16 as the shift's own output).
Parity status: ``token_shift_mix`` is bit-exact by construction of that
contract and pinned by the invariants in tests/test_timemix_oracle.py;
``time_mix_inputs`` / ``time_mix_output`` are pinned by invariants and closed
forms: unit-norm kk, kk of a one-hot and a two-channel ``k_k`` (which fixes
where ``k_k`` enters), the gate limits, the GroupNorm moments under any
per-channel ``ln_w`` / ``ln_b`` (which fixes the affine ``n ln_w + ln_b``) and
the bonus term of a one-hot ``r_k``; the tests also plant a dropped ``k_k``
and a swapped affine in copies of these functions and see the pins fail.
Agreement with fla's own bf16 intermediate roundings is "parity unpinned".
"""

from __future__ import annotations

import numpy as np

from . import bf16_bits_to_f64, f32_to_bf16_bits

DECAY_SCALE = 0.6065306597126334  # exp(-0.5): w = -DECAY_SCALE * sigmoid(.)
HEAD = 64


def _f32(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float64).astype(np.float32)


def token_shift_mix(x_bits, shift_bits, slot_ids, cu_seqlens, mix_bits):
    """Token shift of one state family fused with its lerp mixes.

    x_bits [T, D], shift_bits [rows, D], mix_bits [M, D] (bf16 bit patterns).
    Returns ``(out_bits [M, T, D], new_shift_bits [rows, D])``. For token t of
    sequence s: prev = x[t-1], or shift[slot_ids[s]] for the sequence's first
    token; delta = bf16(f32(prev - x)); out = bf16(f32(x + delta * mix)). The
    sequence's last x row becomes the slot's row."""
    x = bf16_bits_to_f64(x_bits)
    mix = bf16_bits_to_f64(mix_bits)
    T, D = x.shape
    M = mix.shape[0]
    new_shift = np.array(shift_bits, dtype=np.uint16, copy=True)
    prev = np.zeros_like(x)
    cu = [int(c) for c in cu_seqlens]
    for s in range(len(cu) - 1):
        b, e = cu[s], cu[s + 1]
        if e <= b:
            continue
        prev[b] = bf16_bits_to_f64(shift_bits[slot_ids[s]])
        prev[b + 1:e] = x[b:e - 1]
        new_shift[slot_ids[s]] = x_bits[e - 1]
    delta = bf16_bits_to_f64(f32_to_bf16_bits(_f32(prev - x)))
    out = np.empty((M, T, D), dtype=np.uint16)
    for m in range(M):
        # delta * mix is exact in float64 (two 8-bit significands) and so is
        # the sum with x for operands of comparable magnitude; one float32
        # rounding then matches a fused multiply-add.
        out[m] = f32_to_bf16_bits(_f32(x + delta * mix[m]))
    return out, new_shift


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def time_mix_inputs(H, k, v, w_lora, a_lora, k_k, k_a, v_lora=None, v_first=None):
    """The WKV op's inputs from the time-mix projections (float64 values of
    bf16 inputs in, float64 out, unrounded). Shapes [T, H*64]; k_k, k_a [H*64].
    Returns dict w, k, v, a, b."""
    T = k.shape[0]
    a = _sigmoid(a_lora)
    kk = (k * k_k).reshape(T, H, HEAD)
    norm = np.sqrt(np.sum(kk * kk, axis=-1, keepdims=True))
    kk = (kk / np.maximum(norm, 1e-12)).reshape(T, H * HEAD)
    out = {
        "w": -DECAY_SCALE * _sigmoid(w_lora),
        "k": k * (1.0 + (a - 1.0) * k_a),
        "v": v if v_lora is None else v + (v_first - v) * _sigmoid(v_lora),
        "a": -kk,
        "b": kk * a,
    }
    return out


def time_mix_output(H, y, r, k, v, g, r_k, ln_w, ln_b, eps):
    """Per-head GroupNorm of y [T, H, 64] (biased variance), plus the bonus
    term (sum_c r k r_k) v, times the gate g. Inputs float64, [T, H*64];
    r_k, ln_w, ln_b [H*64]. Returns ``(out, scale)`` float64 [T, H*64], where
    ``scale`` = (|normed| + |bonus v|) |g| bounds the rounding error of an
    fp32 evaluation (for tolerances)."""
    T = y.shape[0]
    yh = y.reshape(T, H, HEAD)
    mean = yh.mean(axis=-1, keepdims=True)
    var = ((yh - mean) ** 2).mean(axis=-1, keepdims=True)
    n = ((yh - mean) / np.sqrt(var + eps)).reshape(T, H * HEAD) * ln_w + ln_b
    bonus = np.sum((r * k * r_k).reshape(T, H, HEAD), axis=-1, keepdims=True)
    bv = (bonus * v.reshape(T, H, HEAD)).reshape(T, H * HEAD)
    return (n + bv) * g, (np.abs(n) + np.abs(bv)) * np.abs(g)
