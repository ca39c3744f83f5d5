"""Pins the CPU oracle (oracle/) before anything is checked against it.

Each check is chosen so that a plausible slip in the restated recurrence fails
it: a dropped term (CF1, CF2, linearity), a transposed state (CF3 delta-rule
retrieval with a non-symmetric S_0), a and b swapped (the x-orthogonal-to-b
invariant), the updated instead of the previous state inside (S a) (product
form), a wrong decay exponent or index (CF2), and chunk-boundary mistakes in
the chunked restatement (ragged lengths against the stepwise scan).
"""

from __future__ import annotations

import hashlib
import os

import numpy as np
import pytest
import torch

import oracle as O
from tests.golden import make_golden as G

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "wkv7_golden.npz")


def _rand(rng, T, H, N):
    r, k, v = (rng.standard_normal((T, H, N)) for _ in range(3))
    kn = k / np.linalg.norm(k, axis=-1, keepdims=True)
    a = -kn
    b = kn / (1 + np.exp(-rng.standard_normal((T, H, N))))
    w = -0.606531 / (1 + np.exp(-rng.standard_normal((T, H, N))))
    return r, w, k, v, a, b


def test_golden_tiny():
    g = np.load(GOLDEN)
    y, hT = O.scan_f64(g["tiny_cu"], g["tiny_r"], g["tiny_w"], g["tiny_k"], g["tiny_v"],
                       g["tiny_a"], g["tiny_b"], h0=g["tiny_h0"], scale=float(g["tiny_scale"]))
    np.testing.assert_allclose(y, g["tiny_y"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(hT, g["tiny_hT"], rtol=1e-12, atol=1e-12)


def test_golden_cfg0():
    g = np.load(GOLDEN)
    pool, ids, vecs = G.cfg0_inputs(int(g["cfg0_seed"]))
    digest = hashlib.sha256(pool.numpy().tobytes()).digest()
    assert digest == g["cfg0_pool_sha256"].tobytes(), "synthetic pool generator drifted"
    assert ids == g["cfg0_ids"].tolist()
    for n in "rwkvab":
        assert np.array_equal(G.bits(vecs[n]), g[f"cfg0_{n}"]), f"input {n} drifted"
    f64 = [O.bf16_bits_to_f64(g[f"cfg0_{n}"]) for n in "rwkvab"]
    y, hs = O.decode_slots_f64(pool.numpy(), ids, *f64)
    np.testing.assert_allclose(y, g["cfg0_y"], rtol=1e-11, atol=1e-11)
    np.testing.assert_allclose(hs @ G.projection_vector(), g["cfg0_state_proj"], rtol=1e-11,
                               atol=1e-11)
    np.testing.assert_allclose(hs[0, 0], g["cfg0_state_block"], rtol=1e-12, atol=1e-12)


def test_cf1_linear_attention_prefix_sum():
    """a = b = 0, decay 1: S_t = S_0 + sum_s v_s k_s^T, y_t = S_t r_t."""
    rng = np.random.default_rng(1)
    T, H, N = 11, 3, 16
    r, _, k, v, _, _ = _rand(rng, T, H, N)
    z = np.zeros((T, H, N))
    h0 = rng.standard_normal((1, H, N, N))
    y, hT = O.scan_f64([0, T], r, z, k, v, z, z, h0=h0)
    S = np.swapaxes(h0[0], -1, -2) + np.cumsum(v[:, :, :, None] * k[:, :, None, :], axis=0)
    np.testing.assert_allclose(np.swapaxes(hT[0], -1, -2), S[-1], rtol=1e-12, atol=1e-12)
    y_ref = np.einsum("thij,thj->thi", S, r)
    np.testing.assert_allclose(y, y_ref, rtol=1e-11, atol=1e-11)


def test_cf2_constant_decay_geometric_sum():
    """a = b = 0, per-channel constant decay omega:
    h_T[j,i] = omega_j^T h_0[j,i] + sum_t omega_j^(T-t) k_t[j] v_t[i]."""
    rng = np.random.default_rng(2)
    T, H, N = 9, 2, 8
    r, _, k, v, _, _ = _rand(rng, T, H, N)
    omega = rng.uniform(0.55, 0.99, size=(H, N))
    w = np.broadcast_to(np.log(omega), (T, H, N)).copy()
    z = np.zeros((T, H, N))
    h0 = rng.standard_normal((1, H, N, N))
    _, hT = O.scan_f64([0, T], r, w, k, v, z, z, h0=h0)
    expect = omega[:, :, None] ** T * h0[0]
    for t in range(T):
        expect = expect + (omega ** (T - 1 - t))[:, :, None] * k[t][:, :, None] * v[t][:, None, :]
    np.testing.assert_allclose(hT[0], expect, rtol=1e-12, atol=1e-12)


def test_cf3_delta_rule_retrieval_orientation():
    """decay 1, a = -k^, b = beta k^, k = k^: S_1 k^ = (1 - beta) S_0 k^ + v.
    With beta = 1 this is S_1 k^ = v. A transposed state fails it for a
    non-symmetric S_0."""
    rng = np.random.default_rng(3)
    H, N = 4, 16
    kh = rng.standard_normal((1, H, N))
    kh /= np.linalg.norm(kh, axis=-1, keepdims=True)
    v = rng.standard_normal((1, H, N))
    r = rng.standard_normal((1, H, N))
    h0 = rng.standard_normal((1, H, N, N))
    assert not np.allclose(h0, np.swapaxes(h0, -1, -2))
    z = np.zeros((1, H, N))
    for beta in (1.0, 0.3):
        _, hT = O.scan_f64([0, 1], r, z, kh, v, -kh, beta * kh, h0=h0)
        S0k = np.einsum("hji,hj->hi", h0[0], kh[0])      # S_0 k^ in value space
        S1k = np.einsum("hji,hj->hi", hT[0], kh[0])
        np.testing.assert_allclose(S1k, (1 - beta) * S0k + v[0], rtol=1e-12, atol=1e-12)


def test_cf4_zero_state_zero_value():
    rng = np.random.default_rng(4)
    T, H, N = 7, 2, 8
    r, w, k, _, a, b = _rand(rng, T, H, N)
    y, hT = O.scan_f64([0, T], r, w, k, np.zeros((T, H, N)), a, b)
    assert np.all(y == 0.0) and np.all(hT == 0.0)


def test_cf5_linearity_in_state_and_value():
    rng = np.random.default_rng(5)
    T, H, N = 6, 2, 8
    r, w, k, v1, a, b = _rand(rng, T, H, N)
    v2 = rng.standard_normal((T, H, N))
    s1 = rng.standard_normal((1, H, N, N))
    s2 = rng.standard_normal((1, H, N, N))
    al, be = 0.7, -1.3
    y1, h1 = O.scan_f64([0, T], r, w, k, v1, a, b, h0=s1)
    y2, h2 = O.scan_f64([0, T], r, w, k, v2, a, b, h0=s2)
    y3, h3 = O.scan_f64([0, T], r, w, k, al * v1 + be * v2, a, b, h0=al * s1 + be * s2)
    np.testing.assert_allclose(y3, al * y1 + be * y2, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(h3, al * h1 + be * h2, rtol=1e-10, atol=1e-10)


def test_a_and_b_act_on_their_own_sides():
    """decay 1, k = 0: S_1 = S_0 (I + a b^T). For x orthogonal to b,
    S_1 x = S_0 x; for x = b, S_1 b = S_0 b + (S_0 a)(b^T b). Swapping a and b
    breaks the first identity."""
    rng = np.random.default_rng(6)
    H, N = 3, 8
    a = rng.standard_normal((1, H, N))
    b = rng.standard_normal((1, H, N))
    x = rng.standard_normal((H, N))
    x -= (np.sum(x * b[0], -1) / np.sum(b[0] * b[0], -1))[:, None] * b[0]
    assert np.max(np.abs(np.sum(x * a[0], -1))) > 1e-3
    h0 = rng.standard_normal((1, H, N, N))
    z = np.zeros((1, H, N))
    _, hT = O.scan_f64([0, 1], z, z, z, z, a, b, h0=h0)

    def S_times(h, vec):  # S vec with S = h^T
        return np.einsum("hji,hj->hi", h, vec)

    np.testing.assert_allclose(S_times(hT[0], x), S_times(h0[0], x), rtol=1e-12, atol=1e-12)
    bb = np.sum(b[0] * b[0], -1)[:, None]
    np.testing.assert_allclose(S_times(hT[0], b[0]),
                               S_times(h0[0], b[0]) + S_times(h0[0], a[0]) * bb,
                               rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("N", [4, 8, 64])
def test_scan_matches_transition_product(N):
    rng = np.random.default_rng(7 + N)
    lens = [3, 1, 6]
    T, H = sum(lens), 2
    xs = _rand(rng, T, H, N)
    h0 = rng.standard_normal((3, H, N, N))
    cu = np.concatenate([[0], np.cumsum(lens)])
    y, hT = O.scan_f64(cu, *xs, h0=h0, scale=1.5)
    for s in range(3):
        sl = slice(cu[s], cu[s + 1])
        ye, he = O.transition_product_f64(*(x[sl] for x in xs), h0=h0[s], scale=1.5)
        np.testing.assert_allclose(y[sl], ye, rtol=1e-11, atol=1e-11)
        np.testing.assert_allclose(hT[s], he, rtol=1e-11, atol=1e-11)


@pytest.mark.parametrize("chunk", [16, 64])
def test_chunked_form_matches_stepwise(chunk):
    rng = np.random.default_rng(8)
    lens = [0, 1, 63, 64, 65, 200]
    T, H, N = sum(lens), 2, 64
    xs = _rand(rng, T, H, N)
    h0 = rng.standard_normal((len(lens), H, N, N)) * 0.1
    cu = np.concatenate([[0], np.cumsum(lens)])
    y1, h1 = O.scan_f64(cu, *xs, h0=h0)
    y2, h2 = O.chunked_scan_f64(cu, *xs, h0=h0, chunk=chunk)
    np.testing.assert_allclose(y2, y1, rtol=1e-9, atol=1e-9)
    np.testing.assert_allclose(h2, h1, rtol=1e-9, atol=1e-9)


def test_port_f32_matches_f64():
    g = torch.Generator().manual_seed(9)
    from wkvm_amd import synthetic as syn
    H, rows = 4, 9
    pool = (torch.randn((rows, H, 64, 64), generator=g) * 0.1).numpy()
    ids = [3, 1, 7]
    vecs = syn.wkv7_vectors((3, H, 64), g)
    bitsd = {n: G.bits(vecs[n]) for n in "rwkvab"}
    f64 = [O.bf16_bits_to_f64(bitsd[n]) for n in "rwkvab"]
    y_ref, h_ref = O.decode_slots_f64(pool, ids, *f64)
    p = pool.copy()
    y = O.port_decode_slots_f32(p, ids, *(bitsd[n] for n in "rwkvab"))
    np.testing.assert_allclose(p[ids], h_ref, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(O.bf16_bits_to_f64(y), O.round_f64_to_bf16(y_ref), rtol=1e-2,
                               atol=1e-2)
    # prefill port
    lens = [5, 70]
    vecs = syn.wkv7_vectors((sum(lens), H, 64), g)
    bitsd = {n: G.bits(vecs[n]) for n in "rwkvab"}
    f64 = [O.bf16_bits_to_f64(bitsd[n]) for n in "rwkvab"]
    cu = [0, 5, 75]
    for zero_init in (True, False):
        p = pool.copy()
        y_ref, h_ref = O.prefill_f64(pool, [2, 8], cu, *f64, zero_init=zero_init)
        y = O.port_prefill_f32(p, [2, 8], cu, *(bitsd[n] for n in "rwkvab"), zero_init=zero_init)
        np.testing.assert_allclose(p[[2, 8]], h_ref, rtol=1e-4, atol=1e-4)
        rel = np.linalg.norm(O.bf16_bits_to_f64(y) - y_ref) / np.linalg.norm(y_ref)
        assert rel < 5e-3


def test_bf16_rounding_matches_torch():
    x = torch.cat([torch.randn(10000) * 3, torch.tensor([0.0, -0.0, 1e-40, 3.4e38, float("inf"),
                                                          -float("inf"), 1.00390625, 1.01171875])])
    ours = O.f32_to_bf16_bits(x.numpy())
    ref = x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)
    back = O.bf16_bits_to_f64(ref)
    assert np.array_equal(back, x.to(torch.bfloat16).double().numpy())


def test_slot_byte_semantics_match_torch_index_ops():
    """The numpy slot semantics equal torch's index_select / index_copy_ /
    slice copies -- the ops the reference uses (state.py:77-97, store.py:130-152)."""
    g = torch.Generator().manual_seed(10)
    t = torch.randn((3, 6, 2, 4), generator=g)
    ids = [4, 1, 2]
    np.testing.assert_array_equal(O.slot_gather_np(t.numpy(), 1, ids),
                                  t.index_select(1, torch.tensor(ids)).numpy())
    rows = torch.randn((3, 3, 2, 4), generator=g)
    ref = t.clone()
    ref.index_copy_(1, torch.tensor(ids), rows)
    np.testing.assert_array_equal(O.slot_scatter_np(t.numpy(), 1, ids, rows.numpy()), ref.numpy())
    ref = t.clone()
    ref[:, 5] = t[:, 3]
    ref[:, 0] = t[:, 3]
    np.testing.assert_array_equal(O.slot_copy_np(t.numpy(), 1, [3, 3], [5, 0]), ref.numpy())


def test_scan_bf16_variant_equals_f64_variant():
    from wkvm_amd import synthetic as syn
    g = torch.Generator().manual_seed(11)
    H, rows = 3, 6
    pool = (torch.randn((rows, H, 64, 64), generator=g) * 0.1).numpy()
    lens = [4, 0, 9]
    cu = np.concatenate([[0], np.cumsum(lens)])
    vecs = syn.wkv7_vectors((sum(lens), H, 64), g)
    bitsd = [G.bits(vecs[n]) for n in "rwkvab"]
    f64 = [O.bf16_bits_to_f64(x) for x in bitsd]
    ids = [5, 2, 1]
    y1, h1 = O.scan_bf16(cu, *bitsd, pool=pool, slot_ids=ids, scale=0.5)
    y2, h2 = O.scan_f64(cu, *f64, h0=pool.astype(np.float64)[ids], scale=0.5)
    assert np.array_equal(y1, y2) and np.array_equal(h1, h2)
    y3, h3 = O.scan_bf16(cu, *bitsd)
    y4, h4 = O.scan_f64(cu, *f64)
    assert np.array_equal(y3, y4) and np.array_equal(h3, h4)


def test_bf16_output_bar_helper():
    """The bf16-output bar of the GPU tests: an exactly rounded output sits at
    half its bar, and two planted ulps on one element fail it."""
    from tests import util as U

    rng = np.random.default_rng(0)
    ref = rng.standard_normal((100, 64)) * 5
    bits = O.f32_to_bf16_bits(ref.astype(np.float32))
    assert U.bf16_y_excess(bits, ref) <= 0.5 + 1e-9
    bad = bits.copy()
    bad[3, 5] += 2
    assert U.bf16_y_excess(bad, ref) > 1
