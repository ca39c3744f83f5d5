"""WKV7Runner: the runner's prefill / decode control flow at the WKV-op level.

Mirrors RWKV7Runner (wkvm/runner/runner.py:23-89) with the model forward
reduced to its WKV7 op: callers hand in the per-layer projected vectors
(r, w, k, v, a, b) that the RWKV-7 time-mix produces, instead of token ids.
The control flow is the reference's:

* ``prefill`` walks the prompt in ``prefill_chunk`` slices and, inside each
  slice, every layer; the state round-trips through the slot between slices
  exactly as a preempted request's would (runner.py:12-14, 52-62);
* ``decode_step`` advances a batch of slots by one token through every layer
  (runner.py:65-89);
* ``mixed_step`` is one scheduler step with decode rows and ragged prefill
  rows together, one decode launch plus one varlen prefill launch per layer
  (the split Engine._execute makes, wkvm/engine.py:142-160, laid out with
  MixedBatchMetadata-style offsets, wkvm/core/mixed_batch.py:213-270).

Errors mirror the reference: ``ValueError`` for ``prefill_chunk < 1``, an
empty prompt and a batch / input length mismatch.
"""

from __future__ import annotations

from contextlib import nullcontext as _nullcontext
from typing import Sequence

import torch

from . import ops
from .state import RWKV7StateBank

LayerInputs = Sequence[torch.Tensor]  # (r, w, k, v, a, b)


class WKV7Runner:
    # Chunks at least this long run segmented when ``prefill_segments`` is set
    # (the segmented form is faster from about 2k tokens of one sequence).
    SEGMENT_MIN_TOKENS = 2048

    def __init__(self, bank: RWKV7StateBank, prefill_chunk: int = 512,
                 prefill_segments: int | str | None = None) -> None:
        """``prefill_segments``: cut each prefill chunk of at least
        ``SEGMENT_MIN_TOKENS`` tokens into that many segments that run side by
        side (``ops.wkv7_prefill_segments``); ``"auto"`` picks the count from
        the compute units one chunk leaves idle (``ops.auto_segments``);
        ``None`` runs every chunk in one pass. Results agree to fp32 rounding."""
        if prefill_chunk < 1:
            raise ValueError("prefill_chunk must be >= 1")
        if prefill_segments is not None and prefill_segments != "auto" and (
                not isinstance(prefill_segments, int) or prefill_segments < 1):
            raise ValueError("prefill_segments must be >= 1, 'auto' or None")
        self.bank = bank
        self.prefill_chunk = prefill_chunk
        self.prefill_segments = prefill_segments
        self.device = bank.device

    def _check_layers(self, layer_inputs: Sequence[LayerInputs]) -> None:
        if len(layer_inputs) != self.bank.layout.n_layer:
            raise ValueError(f"expected inputs for {self.bank.layout.n_layer} layers, "
                             f"got {len(layer_inputs)}")

    @torch.inference_mode()
    def prefill(self, layer_inputs: Sequence[LayerInputs], slots: dict[str, int],
                out_dtype: torch.dtype = torch.bfloat16) -> list[torch.Tensor]:
        """Run a prompt's ``[T, H, 64]`` vectors through every layer in chunks,
        leaving the final state in ``slots``; returns per-layer ``y [T, H, 64]``."""
        self._check_layers(layer_inputs)
        T = int(layer_inputs[0][0].shape[0])
        if T == 0:
            raise ValueError("empty prompt")
        H = self.bank.layout.num_heads
        ys = [torch.empty((T, H, 64), dtype=out_dtype, device=self.device)
              for _ in layer_inputs]
        ids = ops.device_ids([slots["wkv"]], self.bank.num_slots + 1, self.device, "slots")
        # device plans (offsets 0, n and the one-sequence order), uploaded once
        # per chunk length rather than once per layer
        plans: dict[int, torch.Tensor] = {}
        for start in range(0, T, self.prefill_chunk):
            n = min(self.prefill_chunk, T - start)
            if n not in plans:
                plans[n] = torch.tensor([0, n, 0], dtype=torch.int32, device=self.device)
            plan = plans[n]
            G = self._segments(n, H)
            for layer, xs in enumerate(layer_inputs):
                chunk = [x[start:start + n] for x in xs]
                if G > 1:
                    ops.wkv7_prefill_segments(self.bank.wkv[layer], [slots["wkv"]], [0, n],
                                              *chunk, segments=G,
                                              out=ys[layer][start:start + n])
                else:
                    self.bank.prefill_wkv(layer, ids, plan[:2], *chunk,
                                          out=ys[layer][start:start + n], seq_order=plan[2:])
        return ys

    def _segments(self, n: int, H: int) -> int:
        if self.prefill_segments is None or n < self.SEGMENT_MIN_TOKENS:
            return 1
        if self.prefill_segments == "auto":
            return ops.auto_segments(H, [n], self.device)
        return self.prefill_segments

    @torch.inference_mode()
    def decode_step(self, slot_batch: list[dict[str, int]],
                    layer_inputs: Sequence[LayerInputs],
                    out_dtype: torch.dtype = torch.bfloat16) -> list[torch.Tensor]:
        """Advance every slot in ``slot_batch`` by one token through every
        layer; ``layer_inputs[l]`` holds ``[B, H, 64]`` vectors. Returns
        per-layer ``y [B, H, 64]``."""
        self._check_layers(layer_inputs)
        if any(int(x.shape[0]) != len(slot_batch) for xs in layer_inputs for x in xs):
            raise ValueError("slot_batch and last_tokens length mismatch")
        ids, order = ops.decode_plan(ops.ids_list(slot_batch, "wkv"), self.bank.num_slots + 1,
                                     self.device)
        return [self.bank.decode_wkv(layer, ids, *xs, out_dtype=out_dtype, row_order=order)
                for layer, xs in enumerate(layer_inputs)]

    @torch.inference_mode()
    def mixed_step(self, decode_batch: list[dict[str, int]],
                   decode_inputs: Sequence[LayerInputs],
                   prefill_batch: list[dict[str, int]], prefill_lens: Sequence[int],
                   prefill_inputs: Sequence[LayerInputs], *, zero_init: bool = False,
                   out_dtype: torch.dtype = torch.bfloat16, concurrent: bool = True):
        """One scheduler step over decode rows (one token each) and ragged
        prefill rows (``prefill_lens`` tokens each, packed along dim 0).
        Returns ``(decode_ys, prefill_ys)`` per layer.

        With ``concurrent`` the decode launches go to a side stream, forked
        from and joined back into the current stream, so the HBM-bound decode
        kernels can run on the compute units the prefill's ragged tail leaves
        idle. A prefill workgroup now fills its compute unit's registers, so
        on config 4 this equals one stream (17.72 ms against 17.72-17.76 ms
        for either serial order, medians of 16 interleaved steps). The two
        touch disjoint slots, so results are identical either way."""
        self._check_layers(decode_inputs)
        self._check_layers(prefill_inputs)
        if len(prefill_lens) != len(prefill_batch):
            raise ValueError("prefill_batch and prefill_lens length mismatch")
        if any(int(n) < 1 for n in prefill_lens):
            raise ValueError("prefill rows need at least one token")
        cu = [0]
        for n in prefill_lens:
            cu.append(cu[-1] + int(n))
        if prefill_batch and any(int(x.shape[0]) != cu[-1] for xs in prefill_inputs for x in xs):
            raise ValueError("prefill inputs do not hold sum(prefill_lens) tokens")
        rows = self.bank.num_slots + 1
        dec_ids, dec_order = ops.decode_plan(ops.ids_list(decode_batch, "wkv"), rows, self.device)
        pre_ids = ops.device_ids(ops.ids_list(prefill_batch, "wkv"), rows, self.device, "prefill")
        if set(ops.ids_list(decode_batch, "wkv")) & set(ops.ids_list(prefill_batch, "wkv")):
            raise ValueError("a slot cannot decode and prefill in the same step")
        # offsets and the longest-first start order in one upload
        nseq = len(prefill_batch)
        plan = torch.tensor(cu + ops.longest_first(cu), dtype=torch.int32, device=self.device)
        cu_t, pre_order = plan[:nseq + 1], plan[nseq + 1:]
        L = self.bank.layout.n_layer
        side = None
        if concurrent and decode_batch and prefill_batch:
            main = torch.cuda.current_stream(self.device)
            side = self._side_stream()
            side.wait_stream(main)
        dec_ys, pre_ys = [None] * L, [None] * L
        for layer in range(L):
            # the layer's prefill first, so its workgroups take the compute units
            # and the decode launch fills in behind them
            if prefill_batch:
                pre_ys[layer] = self.bank.prefill_wkv(layer, pre_ids, cu_t,
                                                      *prefill_inputs[layer],
                                                      zero_init=zero_init, out_dtype=out_dtype,
                                                      seq_order=pre_order)
            if decode_batch:
                with torch.cuda.stream(side) if side is not None else _nullcontext():
                    dec_ys[layer] = self.bank.decode_wkv(layer, dec_ids, *decode_inputs[layer],
                                                         out_dtype=out_dtype,
                                                         row_order=dec_order)
        if side is not None:
            main.wait_stream(side)
            for t in dec_ys + [dec_ids, dec_order]:
                if t is not None:
                    t.record_stream(side)
        return dec_ys, pre_ys

    def _side_stream(self) -> torch.cuda.Stream:
        if getattr(self, "_side", None) is None:
            self._side = torch.cuda.Stream(self.device)  # default priority
        return self._side
