"""Per-slot state layout of an RWKV-7 model (drop-in for the reference's).

Mirrors ``RWKV7StateLayout`` (wkvm/models/rwkv7.py:41-99) and the two spec
dataclasses it returns (wkvm/core/config.py:17-57): the same field names,
shapes and byte counts, with the wkv family in fp32
(``WKV_DTYPE``, wkvm/models/rwkv7.py:38) and the token-shift family in the
model dtype.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

WKV_DTYPE = torch.float32
HEAD_SIZE = 64  # the only head size the kernels accept (RWKV-7 uses 64)


@dataclass(frozen=True)
class StateFamilySpec:
    """One family of fixed-size per-request state (wkvm/core/config.py:17-40)."""

    name: str
    bytes_per_slot: int
    layer_ids: tuple[int, ...] = ()

    def __post_init__(self) -> None:
        if self.bytes_per_slot <= 0:
            raise ValueError(f"family {self.name!r}: bytes_per_slot must be > 0")


@dataclass(frozen=True)
class ModelStateSpec:
    """All state families of a model (wkvm/core/config.py:43-57)."""

    families: tuple[StateFamilySpec, ...]

    def __post_init__(self) -> None:
        names = [f.name for f in self.families]
        if len(names) != len(set(names)):
            raise ValueError(f"duplicate family names: {names}")

    @property
    def bytes_per_request(self) -> int:
        return sum(f.bytes_per_slot for f in self.families)


@dataclass(frozen=True)
class RWKV7StateLayout:
    """Shapes/dtypes of the per-slot state (wkvm/models/rwkv7.py:41-99)."""

    n_layer: int
    hidden_size: int
    num_heads: int
    head_dim: int
    head_v_dim: int
    dtype: torch.dtype  # model dtype; used for the shift family

    @classmethod
    def from_config(cls, config, dtype: torch.dtype) -> "RWKV7StateLayout":
        """Same derivation as wkvm/models/rwkv7.py:57-70 from an fla config."""
        value_dims = set(config.value_dim)
        if len(value_dims) != 1:
            raise NotImplementedError(
                f"every layer must share one value width; config.value_dim = {config.value_dim}")
        if config.attn is not None:
            raise NotImplementedError("hybrid attn layers are not supported")
        return cls(
            n_layer=config.num_hidden_layers,
            hidden_size=config.hidden_size,
            num_heads=config.num_heads,
            head_dim=config.head_dim,
            head_v_dim=value_dims.pop() // config.num_heads,
            dtype=dtype,
        )

    @classmethod
    def for_shape(cls, name: str, dtype: torch.dtype = torch.bfloat16) -> "RWKV7StateLayout":
        """The RWKV-7 shapes the benchmarks use: 0.1B, 1.5B, 7B (head size 64)."""
        shapes = {"0.1B": (12, 768), "1.5B": (24, 2048), "7B": (32, 4096)}
        if name not in shapes:
            raise KeyError(f"unknown shape {name!r}; known: {sorted(shapes)}")
        n_layer, hidden = shapes[name]
        heads = hidden // HEAD_SIZE
        return cls(n_layer=n_layer, hidden_size=hidden, num_heads=heads,
                   head_dim=HEAD_SIZE, head_v_dim=HEAD_SIZE, dtype=dtype)

    @property
    def wkv_shape(self) -> tuple[int, ...]:
        return (self.num_heads, self.head_dim, self.head_v_dim)

    @property
    def shift_shape(self) -> tuple[int, ...]:
        # One hidden-size row per family; the bank keeps two families per
        # layer (index 0: the time-mix shift, index 1: the channel-mix shift).
        return (self.hidden_size,)

    def state_spec(self) -> ModelStateSpec:
        wkv_elems = self.n_layer * self.num_heads * self.head_dim * self.head_v_dim
        shift_elems = self.n_layer * 2 * self.hidden_size
        return ModelStateSpec(
            families=(
                StateFamilySpec(name="wkv", bytes_per_slot=wkv_elems * WKV_DTYPE.itemsize,
                                layer_ids=tuple(range(self.n_layer))),
                StateFamilySpec(name="shift", bytes_per_slot=shift_elems * self.dtype.itemsize,
                                layer_ids=tuple(range(self.n_layer))),
            )
        )
