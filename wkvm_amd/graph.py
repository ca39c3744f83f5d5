"""HIP-graph capture of one decode step's WKV work over the slot pool.

The reference graphs its decode forward per batch size
(experiments/m2_engine_bench.py:44-131, ``GraphedDecode``). It keeps the state
handling eager around every replay: 3 ``index_select`` into static inputs and
3 ``index_copy_`` back per layer (m2_engine_bench.py:105-123). Here the decode
kernels read and write each state at its slot row, so the captured step is
just the ``L`` in-place launches. The batch's slot ids and their slot-sorted
visiting order live in one static device buffer, refreshed by one small copy
before each replay. The per-layer input vectors and outputs are static
buffers as well: the caller fills ``inputs`` (the role of the reference's
static ``ids_in``) and reads ``y``.

A graph is bound to a batch size (the reference's bucket) and to the bank's
tensors; it must be rebuilt if the bank is reallocated.
"""

from __future__ import annotations

from typing import Sequence

import torch

from . import ops
from .layout import HEAD_SIZE
from .state import RWKV7StateBank


class DecodeGraph:
    def __init__(self, bank: RWKV7StateBank, batch_size: int, *,
                 out_dtype: torch.dtype = torch.bfloat16, scale: float = 1.0) -> None:
        if batch_size < 1:
            raise ValueError("batch_size must be >= 1")
        if not bank.wkv.is_cuda:
            raise ValueError("DecodeGraph needs a GPU bank")
        L, H = bank.layout.n_layer, bank.layout.num_heads
        dev = bank.device
        self.bank, self.batch_size = bank, batch_size
        # slot ids in [0, B), visiting order in [B, 2B); the pad row 0 until set
        self.plan = torch.zeros(2 * batch_size, dtype=torch.int32, device=dev)
        self.plan[batch_size:] = torch.arange(batch_size, dtype=torch.int32, device=dev)
        # inputs[l] = (r, w, k, v, a, b), each [B, H, 64] bf16 (w = log-decay)
        self.inputs = torch.zeros((L, 6, batch_size, H, HEAD_SIZE), dtype=torch.bfloat16,
                                  device=dev)
        self.y = torch.empty((L, batch_size, H, HEAD_SIZE), dtype=out_dtype, device=dev)
        ids, order = self.plan[:batch_size], self.plan[batch_size:]
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            for layer in range(L):
                ops.wkv7_decode_slots(bank.wkv[layer], ids, *self.inputs[layer],
                                      out=self.y[layer], row_order=order, scale=scale)

    def set_inputs(self, layer_inputs: Sequence[Sequence[torch.Tensor]]) -> None:
        """Copy per-layer ``(r, w, k, v, a, b)`` into the static input buffers."""
        if len(layer_inputs) != self.inputs.shape[0]:
            raise ValueError(f"expected {self.inputs.shape[0]} layers of inputs, "
                             f"got {len(layer_inputs)}")
        for layer, xs in enumerate(layer_inputs):
            if len(xs) != 6:
                raise ValueError("each layer needs (r, w, k, v, a, b)")
            for i, x in enumerate(xs):
                self.inputs[layer, i].copy_(x)

    def set_slots(self, slot_batch) -> None:
        """Validate the batch's slot ids (list of arena slot dicts or ints) and
        upload them with their slot-sorted visiting order."""
        ids = ops.ids_list(slot_batch, "wkv") if slot_batch and isinstance(slot_batch[0], dict) \
            else list(slot_batch)
        if len(ids) != self.batch_size:
            raise ValueError(f"batch of {len(ids)} slots for a graph of batch size "
                             f"{self.batch_size}")
        lst = ops.host_ids(ids, self.bank.num_slots + 1, "slot_ids", distinct=True)
        order = sorted(range(len(lst)), key=lst.__getitem__)
        self.plan.copy_(torch.tensor(lst + order, dtype=torch.int32))

    def replay(self) -> torch.Tensor:
        """Run the captured step; returns the static ``y`` [L, B, H, 64]."""
        self.graph.replay()
        return self.y

    def step(self, slot_batch, layer_inputs=None) -> torch.Tensor:
        """``set_slots`` (+ ``set_inputs`` if given), then ``replay``."""
        self.set_slots(slot_batch)
        if layer_inputs is not None:
            self.set_inputs(layer_inputs)
        return self.replay()
