"""Seeded synthetic WKV7 inputs with the benchmark distributions.

Per token and head (N = 64), drawn in this order from one generator:
  r, k, v ~ N(0, 1), cast to bf16;
  k' = k / ||k||_2 over the head (fp32 from the bf16 k), cast to bf16;
  a  = -k';  b = k' * sigmoid(g), g ~ N(0, 1), cast to bf16;
  w  = -0.606531 * sigmoid(u), u ~ N(0, 1), cast to bf16 -- the LOG-decay the
       kernels take; the multiplicative decay exp(w) lies in (0.545, 1).
Initial states are N(0, 0.1^2) fp32 (0.1 taken as the standard deviation).
Active slots are a seeded permutation of 1..S (row 0 is the pad slot).

The same tensors feed the GPU kernels and the CPU oracle.
"""

from __future__ import annotations

import torch

DECAY_SCALE = 0.606531  # RWKV-7: decay = exp(-exp(-0.5) * sigmoid(.))


def make_generator(seed: int, device: torch.device | str = "cpu") -> torch.Generator:
    g = torch.Generator(device=torch.device(device))
    g.manual_seed(int(seed))
    return g


def wkv7_vectors(shape: tuple[int, ...], gen: torch.Generator,
                 device: torch.device | str | None = None) -> dict[str, torch.Tensor]:
    """r, w, k, v, a, b as bf16 tensors of ``shape`` (last dim = head size),
    generated on ``gen``'s device and moved to ``device`` if given."""
    dev = gen.device
    r = torch.randn(shape, generator=gen, device=dev).to(torch.bfloat16)
    k = torch.randn(shape, generator=gen, device=dev).to(torch.bfloat16)
    v = torch.randn(shape, generator=gen, device=dev).to(torch.bfloat16)
    kn = torch.nn.functional.normalize(k.float(), dim=-1)
    kn_bf = kn.to(torch.bfloat16)
    gate = torch.sigmoid(torch.randn(shape, generator=gen, device=dev))
    b = (kn_bf.float() * gate).to(torch.bfloat16)
    a = -kn_bf
    u = torch.randn(shape, generator=gen, device=dev)
    w = (-DECAY_SCALE * torch.sigmoid(u)).to(torch.bfloat16)
    out = {"r": r, "w": w, "k": k, "v": v, "a": a, "b": b}
    if device is not None:
        out = {n: t.to(device) for n, t in out.items()}
    return out


def initial_states(shape: tuple[int, ...], gen: torch.Generator, std: float = 0.1) -> torch.Tensor:
    return torch.randn(shape, generator=gen, device=gen.device) * std


def active_slots(num_slots: int, count: int, gen: torch.Generator) -> list[int]:
    """``count`` distinct slot ids from 1..num_slots (seeded)."""
    if count > num_slots:
        raise ValueError("more active slots than the pool holds")
    perm = torch.randperm(num_slots, generator=gen, device=gen.device)[:count] + 1
    return [int(x) for x in perm.tolist()]


def ragged_lengths(count: int, low: int, high: int, gen: torch.Generator) -> list[int]:
    """``count`` sequence lengths uniform in [low, high] (inclusive)."""
    lens = torch.randint(low, high + 1, (count,), generator=gen, device=gen.device)
    return [int(x) for x in lens.tolist()]


def order(vecs: dict[str, torch.Tensor]) -> tuple[torch.Tensor, ...]:
    """The (r, w, k, v, a, b) argument order of the ops."""
    return tuple(vecs[n] for n in "rwkvab")
