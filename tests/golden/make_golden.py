"""Write tests/golden/wkv7_golden.npz.

The reference publishes no WKV7 vectors (its arithmetic lives in the absent
`fla` package), so these fixtures are computed here with the explicit
transition-matrix product ``S_t = S_{t-1}(diag(exp w_t) + a_t b_t^T) + v_t k_t^T``
(``oracle.transition_product_f64``, dense numpy matmuls). The stepwise C scan
and the HIP kernels are checked against them; they share no code with the
stepwise loop.

Cases:
  tiny_*  N = 8, H = 2, three sequences of lengths 5, 1, 9 with random float64
          inputs and initial states (covers multi-step and a length-1 row).
  cfg0_*  the CPU correctness configuration: RWKV-7 0.1B shape (H = 12,
          N = 64, D = 768), one layer, 4 active slots drawn by seed from a
          16-slot pool whose fp32 states are N(0, 0.1^2); bf16 inputs from
          wkvm_amd.synthetic. The pool itself is regenerated from the seed by
          the test (its SHA-256 is stored here to catch generator drift); the
          expected y is stored in full and the expected state as its product
          with a fixed vector plus one full head.

Run: ``python tests/golden/make_golden.py``.
"""

from __future__ import annotations

import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402
from wkvm_amd import synthetic  # noqa: E402

CFG0_SEED = 1234
CFG0_SLOTS = 16
CFG0_ACTIVE = 4
CFG0_H = 12


def cfg0_inputs(seed: int = CFG0_SEED):
    """Pool [17, 12, 64, 64] fp32, active slot ids, and bf16 vectors [4, 12, 64]."""
    g = synthetic.make_generator(seed)
    pool = torch.zeros((CFG0_SLOTS + 1, CFG0_H, 64, 64), dtype=torch.float32)
    pool[1:] = synthetic.initial_states((CFG0_SLOTS, CFG0_H, 64, 64), g)
    ids = synthetic.active_slots(CFG0_SLOTS, CFG0_ACTIVE, g)
    vecs = synthetic.wkv7_vectors((CFG0_ACTIVE, CFG0_H, 64), g)
    return pool, ids, vecs


def projection_vector(n: int = 64) -> np.ndarray:
    return np.cos(np.arange(n) * 0.37) + 0.1 * np.arange(n) / n


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def main() -> None:
    out = {}
    rng = np.random.default_rng(2024)
    lens = [5, 1, 9]
    T, H, N = sum(lens), 2, 8
    r, k, v = (rng.standard_normal((T, H, N)) for _ in range(3))
    kn = k / np.linalg.norm(k, axis=-1, keepdims=True)
    a = -kn
    b = kn / (1 + np.exp(-rng.standard_normal((T, H, N))))
    w = -0.606531 / (1 + np.exp(-rng.standard_normal((T, H, N))))
    h0 = rng.standard_normal((len(lens), H, N, N))
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    ys = np.zeros((T, H, N))
    hT = np.zeros((len(lens), H, N, N))
    for s in range(len(lens)):
        sl = slice(cu[s], cu[s + 1])
        ys[sl], hT[s] = oracle.transition_product_f64(r[sl], w[sl], k[sl], v[sl], a[sl], b[sl],
                                                      h0=h0[s], scale=0.75)
    out.update(tiny_cu=cu, tiny_r=r, tiny_w=w, tiny_k=k, tiny_v=v, tiny_a=a, tiny_b=b,
               tiny_h0=h0, tiny_scale=np.float64(0.75), tiny_y=ys, tiny_hT=hT)

    pool, ids, vecs = cfg0_inputs()
    f64 = {n: vecs[n].double().numpy() for n in "rwkvab"}
    h0c = pool.double().numpy()[ids]
    y = np.zeros((CFG0_ACTIVE, CFG0_H, 64))
    hs = np.zeros((CFG0_ACTIVE, CFG0_H, 64, 64))
    for i in range(CFG0_ACTIVE):
        yi, hs[i] = oracle.transition_product_f64(*(f64[n][i:i + 1] for n in "rwkvab"), h0=h0c[i])
        y[i] = yi[0]
    u = projection_vector()
    out.update(
        cfg0_seed=np.int64(CFG0_SEED),
        cfg0_pool_sha256=np.frombuffer(hashlib.sha256(pool.numpy().tobytes()).digest(), np.uint8),
        cfg0_ids=np.asarray(ids, np.int64),
        **{f"cfg0_{n}": bits(vecs[n]) for n in "rwkvab"},
        cfg0_y=y,
        cfg0_state_proj=hs @ u,
        cfg0_state_block=hs[0, 0],
    )
    path = os.path.join(HERE, "wkv7_golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
