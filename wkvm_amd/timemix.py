"""RWKV-7 time-mix (attention) block over the slot pool.

The reference runs this block inside the third-party ``fla`` package
(RWKV7Attention, reached through the model forward at
wkvm/runner/runner.py:80-88 with the state staged through a Cache,
wkvm/runner/state.py:63-97). Here every state access is slot-indexed and in
place, and every element-wise stage is one of this library's kernels:

  x (mixer input, [T, D] bf16)
    -> token_shift_mix      bank.shift[l, 0] (conv_state) read and updated
                            in place; the six lerp mixes xr..xg
    -> projections          r, k, v, o [D, D] and the LoRAs (w: tanh, a, v:
                            linear, g: sigmoid inside) -- plain GEMMs on the
                            vendor BLAS through torch.mm / torch.addmm
    -> time_mix_inputs      log-decay w, k, v (v_first lerp), a = -kk, b = kk*a
    -> WKV7                 wkv7_decode_slots (one token per slot) or
                            wkv7_prefill_varlen (ragged), bank.wkv[l] in place
    -> time_mix_output      per-head GroupNorm, bonus, gate
    -> o_proj

The LoRA inner activations act on the small [T, rank] tensors between two
GEMMs and stay in torch. Weights are stored [in, out] so each projection is
``x @ W``. Parameter names follow fla's RWKV7Attention (x_r .. x_g, k_k, k_a,
r_k, w0/w1/w2, a0/a1/a2, v0/v1/v2, g1/g2, g_norm). The GroupNorm epsilon is
head_dim * 1e-5.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import ops
from .layout import HEAD_SIZE, RWKV7StateLayout
from .state import RWKV7StateBank

MIX_NAMES = ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g")


def lora_dims(hidden: int) -> dict[str, int]:
    """LoRA ranks of an RWKV-7 layer of width ``hidden`` (the RWKV-7 sizing
    rule, rounded to multiples of 32): 1.5B (2048) -> w 96, a 96, v 64, g 256."""
    def r32(x: float) -> int:
        return max(32, int(round(x / 32)) * 32)
    return {"w": r32(1.8 * hidden ** 0.5), "a": r32(1.8 * hidden ** 0.5),
            "v": r32(1.3 * hidden ** 0.5), "g": r32(0.6 * hidden ** 0.8)}


@dataclass
class TokenBatch:
    """Device plan of one token batch: slot ids, ragged offsets, visiting order.

    ``decode``: one token per slot (``cu_seqlens`` = 0..B); otherwise ragged
    prefill rows, sequence s owning tokens cu_seqlens[s]:cu_seqlens[s+1]."""

    slot_ids: torch.Tensor
    cu_seqlens: torch.Tensor
    order: torch.Tensor | None
    nseq: int
    tokens: int
    decode: bool

    @classmethod
    def plan(cls, bank: RWKV7StateBank, slot_ids, cu_seqlens=None) -> TokenBatch:
        rows, dev = bank.num_slots + 1, bank.device
        if cu_seqlens is None:
            ids, order = ops.decode_plan(slot_ids, rows, dev)
            n = int(ids.shape[0])
            return cls(ids, torch.arange(n + 1, dtype=torch.int32, device=dev), order, n, n, True)
        cu = cu_seqlens.tolist() if isinstance(cu_seqlens, torch.Tensor) else list(cu_seqlens)
        T = int(cu[-1]) if cu else 0
        ids, cu_t, n = ops.seq_plan(slot_ids, cu, rows, T, dev)
        order = torch.tensor(ops.longest_first([int(c) for c in cu]), dtype=torch.int32,
                             device=dev)
        return cls(ids, cu_t, order, n, T, False)


class RWKV7TimeMix:
    """One layer's time-mix block. ``weights`` maps fla's parameter names to
    bf16 tensors: ``mix`` [6, D] (x_r..x_g), ``r``, ``k``, ``v``, ``o``
    [D, D], ``w1`` [D, rw], ``w2`` [rw, D], ``w0`` [D], likewise ``a*``,
    ``v*`` (layers after the first), ``g1`` [D, rg], ``g2`` [rg, D], and
    ``k_k``, ``k_a``, ``r_k``, ``ln_w``, ``ln_b`` [D]."""

    def __init__(self, layout: RWKV7StateLayout, layer_idx: int,
                 weights: dict[str, torch.Tensor]) -> None:
        self.layout = layout
        self.layer_idx = layer_idx
        self.w = weights
        self.eps = HEAD_SIZE * 1e-5

    @classmethod
    def random(cls, layout: RWKV7StateLayout, layer_idx: int, device, seed: int = 0,
               ) -> RWKV7TimeMix:
        """Random-init weights of the real shapes, scaled so activations stay
        O(1) (synthetic benchmarks; there are no checkpoints offline)."""
        D = layout.hidden_size
        ranks = lora_dims(D)
        g = torch.Generator(device=torch.device(device))
        g.manual_seed(int(seed) * 1000 + layer_idx)

        def n(shape, std):
            return (torch.randn(shape, generator=g, device=device) * std).to(torch.bfloat16)

        def u(shape, lo, hi):
            return (torch.rand(shape, generator=g, device=device) * (hi - lo) + lo).to(
                torch.bfloat16)

        w = {"mix": u((6, D), 0.0, 1.0)}
        for name in ("r", "k", "v", "o"):
            w[name] = n((D, D), 1.0 / math.sqrt(D))
        for lo in ("w", "a", "v"):
            if lo == "v" and layer_idx == 0:
                continue
            w[lo + "1"] = n((D, ranks[lo]), 1.0 / math.sqrt(D))
            w[lo + "2"] = n((ranks[lo], D), 1.0 / math.sqrt(ranks[lo]))
            w[lo + "0"] = n((D,), 0.5)
        w["g1"] = n((D, ranks["g"]), 1.0 / math.sqrt(D))
        w["g2"] = n((ranks["g"], D), 1.0 / math.sqrt(ranks["g"]))
        w["k_k"] = u((D,), 0.5, 1.5)
        w["k_a"] = u((D,), 0.0, 1.0)
        w["r_k"] = n((D,), 0.1)
        w["ln_w"] = u((D,), 0.8, 1.2)
        w["ln_b"] = n((D,), 0.05)
        return cls(layout, layer_idx, w)

    def forward(self, bank: RWKV7StateBank, x: torch.Tensor, batch: TokenBatch,
                v_first: torch.Tensor | None = None, *, zero_init: bool = False,
                ) -> tuple[torch.Tensor, torch.Tensor]:
        """``x [T, D]`` bf16 -> ``(o [T, D] bf16, v_first)``; the slots' shift
        row ``bank.shift[l, 0]`` and wkv state ``bank.wkv[l]`` advance in
        place. ``zero_init`` starts prefill sequences from zero wkv state."""
        W, l, H = self.w, self.layer_idx, self.layout.num_heads
        if l > 0 and v_first is None:
            raise ValueError("layers after the first need v_first")
        xr, xw, xk, xv, xa, xg = ops.token_shift_mix(x, bank.shift[l, 0], batch.slot_ids,
                                                     W["mix"], batch.cu_seqlens)
        r = xr @ W["r"]
        k = xk @ W["k"]
        v = xv @ W["v"]
        w_l = torch.addmm(W["w0"], torch.tanh(xw @ W["w1"]), W["w2"])
        a_l = torch.addmm(W["a0"], xa @ W["a1"], W["a2"])
        v_l = torch.addmm(W["v0"], xv @ W["v1"], W["v2"]) if l > 0 else None
        g = torch.sigmoid(xg @ W["g1"]) @ W["g2"]
        w, k2, v2, a, b = ops.time_mix_inputs(H, k, v, w_l, a_l, W["k_k"], W["k_a"], v_l,
                                              v_first if l > 0 else None)
        if l == 0:
            v_first = v2
        T = batch.tokens
        vec = [t.view(T, H, HEAD_SIZE) for t in (r, w, k2, v2, a, b)]
        if batch.decode:
            y = bank.decode_wkv(l, batch.slot_ids, *vec, row_order=batch.order)
        else:
            y = ops.wkv7_prefill_varlen(bank.wkv[l], batch.slot_ids, batch.cu_seqlens, *vec,
                                        zero_init=zero_init, seq_order=batch.order)
        o_in = ops.time_mix_output(H, y, r, k2, v2, g, W["r_k"], W["ln_w"], W["ln_b"], self.eps)
        return o_in @ W["o"], v_first
