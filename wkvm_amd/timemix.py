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
                            linear, g: sigmoid inside): for up to
                            PROJ_MAX_ROWS tokens two grouped launches of
                            wkv7_proj_grouped (all first stages, then all
                            second stages with their biases) and one for o;
                            above that the vendor BLAS through torch's linear
    -> time_mix_inputs      log-decay w, k, v (v_first lerp), a = -kk, b = kk*a
    -> WKV7                 wkv7_prefill_varlen (ragged), bank.wkv[l] in place;
                            for one token per slot, wkv7_decode_block runs
                            time_mix_inputs, the in-place decode and
                            time_mix_output as one launch
    -> time_mix_output      per-head GroupNorm, bonus, gate
    -> o_proj

Weights are stored [out, in] as nn.Linear holds them (each projection is
``linear(x, W)``), the layout both the grouped kernel and the vendor BLAS
read best. At decode sizes each library GEMM is a separate 4-13 us launch;
the grouped kernel runs the seven first-stage products of a 256-token
batch in ~23 us and the four second stages in ~6 us (MI355X, inside a HIP
graph), with the LoRA activations fused into the first stage. Large token
counts (prefill) stay on the vendor BLAS, which reaches ~55 % of the bf16
matrix peak there. Parameter names follow fla's
RWKV7Attention (x_r .. x_g, k_k, k_a, r_k, w0/w1/w2, a0/a1/a2, v0/v1/v2,
g1/g2, g_norm). The GroupNorm epsilon is head_dim * 1e-5.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

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
    bf16 tensors, matrices [out, in]: ``mix`` [6, D] (x_r..x_g), ``r``,
    ``k``, ``v``, ``o`` [D, D], ``w1`` [rw, D], ``w2`` [D, rw], ``w0`` [D],
    likewise ``a*``, ``v*`` (layers after the first), ``g1`` [rg, D], ``g2``
    [D, rg], and ``k_k``, ``k_a``, ``r_k``, ``ln_w``, ``ln_b`` [D]."""

    # Token counts up to this run their projections through wkv7_proj_grouped.
    PROJ_MAX_ROWS = 512

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
            w[lo + "1"] = n((ranks[lo], D), 1.0 / math.sqrt(D))
            w[lo + "2"] = n((D, ranks[lo]), 1.0 / math.sqrt(ranks[lo]))
            w[lo + "0"] = n((D,), 0.5)
        w["g1"] = n((ranks["g"], D), 1.0 / math.sqrt(D))
        w["g2"] = n((D, ranks["g"]), 1.0 / math.sqrt(ranks["g"]))
        w["k_k"] = u((D,), 0.5, 1.5)
        w["k_a"] = u((D,), 0.0, 1.0)
        w["r_k"] = n((D,), 0.1)
        w["ln_w"] = u((D,), 0.8, 1.2)
        w["ln_b"] = n((D,), 0.05)
        return cls(layout, layer_idx, w)

    def forward(self, bank: RWKV7StateBank, x: torch.Tensor, batch: TokenBatch,
                v_first: torch.Tensor | None = None, *, zero_init: bool = False,
                streams: list[torch.cuda.Stream] | None = None,
                ) -> tuple[torch.Tensor, torch.Tensor]:
        """``x [T, D]`` bf16 -> ``(o [T, D] bf16, v_first)``; the slots' shift
        row ``bank.shift[l, 0]`` and wkv state ``bank.wkv[l]`` advance in
        place. ``zero_init`` starts prefill sequences from zero wkv state.

        ``streams`` (side streams of default priority; used above
        ``PROJ_MAX_ROWS`` tokens, where the projections run on the vendor
        BLAS): the projection and LoRA chains are independent of one
        another, so they are forked onto these streams after the token shift
        and joined before the WKV inputs; the results are the same bytes
        either way."""
        W, l, H = self.w, self.layer_idx, self.layout.num_heads
        if l > 0 and v_first is None:
            raise ValueError("layers after the first need v_first")
        xr, xw, xk, xv, xa, xg = ops.token_shift_mix(
            x, bank.shift[l, 0], batch.slot_ids, W["mix"],
            None if batch.decode else batch.cu_seqlens)
        if batch.tokens <= self.PROJ_MAX_ROWS:
            return self._forward_grouped(bank, batch, v_first, zero_init,
                                         (xr, xw, xk, xv, xa, xg))

        # the independent chains between the token shift and the WKV inputs
        chains = {
            "r": lambda: F.linear(xr, W["r"]),
            "k": lambda: F.linear(xk, W["k"]),
            "v": lambda: F.linear(xv, W["v"]),
            "w_l": lambda: F.linear(torch.tanh(F.linear(xw, W["w1"])), W["w2"], W["w0"]),
            "a_l": lambda: F.linear(F.linear(xa, W["a1"]), W["a2"], W["a0"]),
            "g": lambda: F.linear(torch.sigmoid(F.linear(xg, W["g1"])), W["g2"]),
        }
        if l > 0:
            chains["v_l"] = lambda: F.linear(F.linear(xv, W["v1"]), W["v2"], W["v0"])
        res: dict[str, torch.Tensor] = {}
        if streams:
            main = torch.cuda.current_stream(x.device)
            lanes = [main] + list(streams)
            for s in streams:
                s.wait_stream(main)
            for i, (name, fn) in enumerate(chains.items()):
                with torch.cuda.stream(lanes[i % len(lanes)]):
                    res[name] = fn()
            for s in streams:
                main.wait_stream(s)
            if not torch.cuda.is_current_stream_capturing():
                # made on the side streams, used and freed on this one
                for t in res.values():
                    t.record_stream(main)
        else:
            for name, fn in chains.items():
                res[name] = fn()
        r, k, v, w_l, a_l, g = (res[n] for n in ("r", "k", "v", "w_l", "a_l", "g"))
        o_in, v_first = self._wkv_stage(bank, batch, v_first, zero_init, r, k, v, w_l, a_l,
                                        res.get("v_l"), g)
        return F.linear(o_in, W["o"]), v_first

    def _forward_grouped(self, bank, batch, v_first, zero_init, mixes):
        """The block with its projections on wkv7_proj_grouped: one launch
        for the seven first-stage products (r, k, v and the LoRA
        down-projections, tanh / sigmoid fused), one for the four LoRA
        up-projections with their biases, one for o."""
        W, l = self.w, self.layer_idx
        xr, xw, xk, xv, xa, xg = mixes
        first = [(xr, W["r"]), (xk, W["k"]), (xv, W["v"]), (xw, W["w1"], None, "tanh"),
                 (xa, W["a1"]), (xg, W["g1"], None, "sigmoid")]
        if l > 0:
            first.append((xv, W["v1"]))
        r, k, v, hw, ha, hg, *hv = ops.proj_grouped(first)
        second = [(hw, W["w2"], W["w0"]), (ha, W["a2"], W["a0"]), (hg, W["g2"])]
        if l > 0:
            second.append((hv[0], W["v2"], W["v0"]))
        w_l, a_l, g, *v_l = ops.proj_grouped(second)
        o_in, v_first = self._wkv_stage(bank, batch, v_first, zero_init, r, k, v, w_l, a_l,
                                        v_l[0] if v_l else None, g)
        return ops.proj_grouped([(o_in, W["o"])])[0], v_first

    def _wkv_stage(self, bank, batch, v_first, zero_init, r, k, v, w_l, a_l, v_l, g):
        """time_mix_inputs -> in-place WKV7 -> time_mix_output (one fused
        launch for decode batches); returns the output projection's input and
        v_first."""
        W, l, H = self.w, self.layer_idx, self.layout.num_heads
        if batch.decode:
            res = ops.wkv7_decode_block(
                bank.wkv[l], batch.slot_ids, H, r, k, v, w_l, a_l, g, W["k_k"], W["k_a"],
                W["r_k"], W["ln_w"], W["ln_b"], self.eps, v_lora=v_l,
                v_first=v_first if l > 0 else None, row_order=batch.order, want_v=(l == 0))
            return res if l == 0 else (res, v_first)
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
        return o_in, v_first


class TimeMixDecodeGraph:
    """One decode step of every layer's time-mix block as one HIP graph.

    The graph holds, per layer, the token shift over ``bank.shift[l, 0]``, the
    projection GEMMs, the input/output kernels and the in-place WKV decode
    over ``bank.wkv[l]``; ``v_first`` flows from layer 0 inside the graph.
    Static buffers: ``x [L, B, D]`` (each layer's mixer input, filled by the
    caller) and ``o``, the list of the L block outputs ``[B, D]`` (tensors of
    the graph's own memory pool, rewritten by every replay). The batch's slot ids,
    their slot-sorted visiting order and the one-token-per-slot offsets live
    in one device buffer refreshed by ``set_slots``. A graph is bound to a
    batch size and to the bank's tensors (the reference's per-bucket graphs,
    experiments/m2_engine_bench.py:44-131)."""

    def __init__(self, bank: RWKV7StateBank, layers: list[RWKV7TimeMix], batch_size: int,
                 side_streams: int | None = None):
        if batch_size < 1:
            raise ValueError("batch_size must be >= 1")
        if len(layers) < 1 or any(l.layer_idx != i for i, l in enumerate(layers)):
            raise ValueError("layers must be the blocks 0 .. L-1 in order")
        B, D, dev = batch_size, bank.layout.hidden_size, bank.device
        self.bank, self.layers, self.batch_size = bank, layers, batch_size
        # [0, B) slot ids (distinct placeholders until set_slots), [B, 2B) order,
        # [2B, 3B] offsets 0..B
        self.plan = torch.cat([torch.arange(1, B + 1), torch.arange(B),
                               torch.arange(B + 1)]).to(torch.int32).to(dev)
        self.x = torch.zeros((len(layers), B, D), dtype=torch.bfloat16, device=dev)
        self.o: list[torch.Tensor] = []
        batch = TokenBatch(self.plan[:B], self.plan[2 * B:], self.plan[B:2 * B], B, B, True)
        # side streams (default priority) for the block's independent GEMM
        # chains when they run on the vendor BLAS (batches above
        # PROJ_MAX_ROWS; default 2 there, none below); the graph keeps their
        # fork/join as parallel branches
        if side_streams is None:
            side_streams = 2 if batch_size > RWKV7TimeMix.PROJ_MAX_ROWS else 0
        self.streams = [torch.cuda.Stream(dev) for _ in range(side_streams)]
        # initialise the BLAS handles and workspaces of every stream before
        # capture (GEMMs only: the bank is not touched until the first replay)
        main = torch.cuda.current_stream(dev)
        for st in [main] + self.streams:
            st.wait_stream(main)
            with torch.cuda.stream(st):
                for layer in layers:
                    for name in ("r", "k", "v", "o"):
                        _ = F.linear(self.x[0], layer.w[name])
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            v_first = None
            for l, layer in enumerate(layers):
                out, v_first = layer.forward(bank, self.x[l], batch, v_first,
                                             streams=self.streams or None)
                self.o.append(out)

    def set_slots(self, slot_ids) -> None:
        """Validate the batch's slot ids (ints) and upload them with their
        slot-sorted visiting order."""
        lst = ops.host_ids(slot_ids, self.bank.num_slots + 1, "slot_ids", distinct=True)
        if len(lst) != self.batch_size:
            raise ValueError(f"batch of {len(lst)} slots for a graph of batch size "
                             f"{self.batch_size}")
        order = sorted(range(len(lst)), key=lst.__getitem__)
        self.plan[:2 * self.batch_size].copy_(torch.tensor(lst + order, dtype=torch.int32))

    def replay(self) -> list[torch.Tensor]:
        """Run the captured step; returns the static outputs ``o`` (L x [B, D])."""
        self.graph.replay()
        return self.o
