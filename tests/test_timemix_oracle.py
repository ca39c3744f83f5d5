"""Pins the time-mix oracle (oracle/timemix.py) on the CPU, and checks the
argument errors of the time-mix entry points of the C ABI (no GPU work).

The token shift is pinned by what the reference's state contract fixes: a
zero cached row is the zero shift-in of a fresh sequence and the carried row
is the last token's input, so any split of a sequence into chunks threaded
through the slot row, and a token-by-token decode, equal one pass, bit for
bit (wkvm/models/rwkv7.py:25-27, wkvm/runner/runner.py:12-14). Exact
arithmetic cases (small-integer inputs) pin which row is "prev". The other
stages are pinned by invariants their definitions fix: a unit-norm kk and
its closed form under a one-hot or two-channel k_k, the exact limits of every
sigmoid gate, the GroupNorm moments under a per-channel affine ln_w / ln_b,
and the bonus term of a one-hot r_k. Copies of the oracle with a planted
mistake (k_k dropped; n + ln_w ln_b) must fail those pins."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle as O
from oracle import timemix as TM
from wkvm_amd import _lib

RNG = np.random.default_rng(7)


def bits(x) -> np.ndarray:
    return O.f32_to_bf16_bits(np.asarray(x, dtype=np.float32))


def vals(b) -> np.ndarray:
    return O.bf16_bits_to_f64(b)


def rand_bits(*shape, scale=1.0):
    return bits(RNG.standard_normal(shape) * scale)


# -- token shift ----------------------------------------------------------------

def test_shift_mix_zero_is_identity_and_cache_is_last_row():
    T, D, rows = 9, 16, 5
    x, cache = rand_bits(T, D), rand_bits(rows, D)
    mix = bits(np.zeros((2, D)))
    out, new = TM.token_shift_mix(x, cache, [3, 1], [0, 4, 9], mix)
    assert np.array_equal(out[0], x) and np.array_equal(out[1], x)
    assert np.array_equal(new[3], x[3]) and np.array_equal(new[1], x[8])
    for r in (0, 2, 4):
        assert np.array_equal(new[r], cache[r])


def test_shift_mix_one_selects_prev_row():
    # small integers: prev - x and x + delta are exact, so mix = 1 gives prev
    T, D, rows = 7, 8, 4
    x = bits(RNG.integers(-8, 9, size=(T, D)))
    cache = bits(RNG.integers(-8, 9, size=(rows, D)))
    mix = bits(np.ones((1, D)))
    cu = [0, 3, 3, 7]
    slots = [2, 0, 3]
    out, _ = TM.token_shift_mix(x, cache, slots, cu, mix)
    assert np.array_equal(out[0, 0], cache[2])
    assert np.array_equal(out[0, 1:3], x[0:2])
    assert np.array_equal(out[0, 3], cache[3])
    assert np.array_equal(out[0, 4:7], x[3:6])


def test_shift_mix_zero_cache_is_zero_shift_in():
    T, D = 5, 8
    x = bits(RNG.integers(-8, 9, size=(T, D)))
    mix = bits(np.full((1, D), 0.5))
    out, _ = TM.token_shift_mix(x, bits(np.zeros((2, D))), [1], [0, T], mix)
    # x + (0 - x) * 0.5 = x / 2, exact for small integers
    assert np.array_equal(vals(out[0, 0]), vals(x[0]) / 2)


@pytest.mark.parametrize("split", [1, 5, 16, 29])
def test_shift_mix_chunks_through_the_slot_equal_one_pass(split):
    T, D, rows = 30, 24, 6
    x, cache, mix = rand_bits(T, D), rand_bits(rows, D), rand_bits(6, D)
    full, new_full = TM.token_shift_mix(x, cache, [4], [0, T], mix)
    a, c1 = TM.token_shift_mix(x[:split], cache, [4], [0, split], mix)
    b, c2 = TM.token_shift_mix(x[split:], c1, [4], [0, T - split], mix)
    assert np.array_equal(np.concatenate([a, b], axis=1), full)
    assert np.array_equal(c2, new_full)


def test_shift_mix_decode_loop_equals_prefill():
    T, D, rows = 12, 16, 3
    x, cache, mix = rand_bits(T, D), rand_bits(rows, D), rand_bits(3, D)
    full, new_full = TM.token_shift_mix(x, cache, [2], [0, T], mix)
    c = cache
    steps = []
    for t in range(T):
        o, c = TM.token_shift_mix(x[t:t + 1], c, [2], [0, 1], mix)
        steps.append(o)
    assert np.array_equal(np.concatenate(steps, axis=1), full)
    assert np.array_equal(c, new_full)


# -- WKV inputs ------------------------------------------------------------------

def _inputs(T=6, H=3, **kw):
    D = H * 64
    base = dict(k=RNG.standard_normal((T, D)), v=RNG.standard_normal((T, D)),
                w_lora=RNG.standard_normal((T, D)), a_lora=RNG.standard_normal((T, D)),
                k_k=RNG.uniform(0.5, 1.5, D), k_a=RNG.uniform(0, 1, D))
    base.update(kw)
    return H, base


def test_inputs_kk_unit_norm_and_gates():
    H, a = _inputs()
    o = TM.time_mix_inputs(H, **a)
    T = a["k"].shape[0]
    norms = np.linalg.norm(o["a"].reshape(T, H, 64), axis=-1)
    assert np.allclose(norms, 1.0, atol=1e-12)
    gate = o["b"] / -o["a"]
    assert np.allclose(gate, 1 / (1 + np.exp(-a["a_lora"])), atol=1e-12)
    assert np.all((o["w"] < 0) & (o["w"] > -TM.DECAY_SCALE))
    # normalize is scale invariant in k_k
    o2 = TM.time_mix_inputs(H, **{**a, "k_k": 3.0 * a["k_k"]})
    assert np.allclose(o2["a"], o["a"], atol=1e-12)


def test_inputs_limits():
    H, a = _inputs()
    D = H * 64
    big = np.full_like(a["k"], 60.0)
    o = TM.time_mix_inputs(H, **{**a, "k_a": np.zeros(D)})
    assert np.array_equal(o["k"], a["k"])
    o = TM.time_mix_inputs(H, **{**a, "k_a": np.ones(D), "a_lora": big})
    assert np.allclose(o["k"], a["k"], atol=1e-12)
    o = TM.time_mix_inputs(H, **{**a, "w_lora": big})
    assert np.allclose(o["w"], -TM.DECAY_SCALE, atol=1e-12)
    vf = RNG.standard_normal(a["k"].shape)
    o = TM.time_mix_inputs(H, **a, v_lora=big, v_first=vf)
    assert np.allclose(o["v"], vf, atol=1e-12)
    o = TM.time_mix_inputs(H, **a, v_lora=-big, v_first=vf)
    assert np.allclose(o["v"], a["v"], atol=1e-12)
    o = TM.time_mix_inputs(H, **a, v_lora=np.zeros_like(big), v_first=vf)
    assert np.allclose(o["v"], (a["v"] + vf) / 2, atol=1e-12)
    assert np.array_equal(TM.time_mix_inputs(H, **a)["v"], a["v"])


def _check_kk_one_hot(inputs_fn):
    """k_k one-hot on channel c of each head: kk = normalize(k * k_k) is
    sign(k_c) e_c, so a = -sign(k_c) e_c and b = -a sigmoid(a_lora), exactly.
    An oracle that drops k_k normalises all 64 channels of k instead."""
    T, H = 5, 3
    D = H * 64
    chans = [7, 40, 63]
    k_k = np.zeros(D)
    for h, c in enumerate(chans):
        k_k[64 * h + c] = RNG.uniform(0.5, 2.0)
    H, a = _inputs(T=T, H=H, k_k=k_k)
    o = inputs_fn(H, **a)
    expect_a = np.zeros((T, D))
    for h, c in enumerate(chans):
        expect_a[:, 64 * h + c] = -np.sign(a["k"][:, 64 * h + c])
    assert np.array_equal(o["a"], expect_a)
    assert np.allclose(o["b"], -expect_a / (1 + np.exp(-a["a_lora"])), rtol=0, atol=1e-15)


def _check_kk_two_channels(inputs_fn):
    """Two live channels per head: kk is (k_c1 k_k[c1], k_c2 k_k[c2]) over its
    own norm, which a per-channel k_k changes and a dropped k_k does not."""
    T, H = 4, 2
    D = H * 64
    k_k = np.zeros(D)
    k_k[3], k_k[11] = 0.25, 3.0
    k_k[64 + 0], k_k[64 + 50] = 2.0, 0.5
    H, a = _inputs(T=T, H=H, k_k=k_k)
    o = inputs_fn(H, **a)
    for c1, c2 in ((3, 11), (64, 114)):
        x1, x2 = a["k"][:, c1] * k_k[c1], a["k"][:, c2] * k_k[c2]
        n = np.hypot(x1, x2)
        assert np.allclose(o["a"][:, c1], -x1 / n, atol=1e-14)
        assert np.allclose(o["a"][:, c2], -x2 / n, atol=1e-14)


def test_inputs_kk_pins():
    _check_kk_one_hot(TM.time_mix_inputs)
    _check_kk_two_channels(TM.time_mix_inputs)


def _inputs_without_kk(H, k, v, w_lora, a_lora, k_k, k_a, v_lora=None, v_first=None):
    # planted mistake: k_k ignored in the normalisation
    return TM.time_mix_inputs(H, k, v, w_lora, a_lora, np.ones_like(k_k), k_a, v_lora, v_first)


def test_kk_pins_fail_on_an_oracle_without_kk():
    with pytest.raises(AssertionError):
        _check_kk_one_hot(_inputs_without_kk)
    with pytest.raises(AssertionError):
        _check_kk_two_channels(_inputs_without_kk)


# -- WKV output ------------------------------------------------------------------

def test_output_groupnorm_moments():
    T, H = 5, 4
    D = H * 64
    y = RNG.standard_normal((T, H, 64)) * 3 + 1
    z = np.zeros(D)
    args = dict(r=RNG.standard_normal((T, D)), k=RNG.standard_normal((T, D)),
                v=RNG.standard_normal((T, D)), g=np.ones((T, D)), r_k=z, ln_w=np.ones(D),
                ln_b=z, eps=1e-3)
    out, _ = TM.time_mix_output(H, y, **args)
    oh = out.reshape(T, H, 64)
    var = y.var(axis=-1)
    assert np.allclose(oh.mean(axis=-1), 0, atol=1e-12)
    assert np.allclose((oh ** 2).mean(axis=-1), var / (var + 1e-3), atol=1e-12)
    # a constant head normalises to the bias
    yc = np.repeat(RNG.standard_normal((T, H, 1)), 64, axis=-1)
    b = RNG.standard_normal(D)
    out, _ = TM.time_mix_output(H, yc, **{**args, "ln_b": b})
    assert np.allclose(out, np.broadcast_to(b, out.shape), atol=1e-9)


def test_output_bonus_one_hot_and_gate():
    T, H = 4, 2
    D = H * 64
    r, k, v = (RNG.standard_normal((T, D)) for _ in range(3))
    r_k = np.zeros(D)
    r_k[5] = 1.0       # head 0, channel 5
    r_k[64 + 9] = 2.0  # head 1, channel 9
    z = np.zeros(D)
    out, _ = TM.time_mix_output(H, RNG.standard_normal((T, H, 64)), r, k, v, np.ones((T, D)),
                                r_k, z, z, 1e-5)
    assert np.allclose(out[:, :64], (r[:, 5] * k[:, 5])[:, None] * v[:, :64], atol=1e-12)
    assert np.allclose(out[:, 64:], (2 * r[:, 73] * k[:, 73])[:, None] * v[:, 64:], atol=1e-12)
    g = RNG.standard_normal((T, D))
    out_g, _ = TM.time_mix_output(H, RNG.standard_normal((T, H, 64)), r, k, v, g, r_k, z, z,
                                  1e-5)
    assert np.allclose(out_g, out * g, atol=1e-12)


def _check_ln_affine(output_fn):
    """GroupNorm affine per channel: out = n ln_w + ln_b (r_k = 0, g = 1), so
    (out - ln_b) / ln_w has mean 0 and second moment var / (var + eps) per
    head, for any per-channel ln_w and ln_b. An oracle that forms
    n + ln_w ln_b, or drops either parameter, breaks one of the two moments."""
    T, H = 6, 3
    D = H * 64
    eps = 1e-3
    y = RNG.standard_normal((T, H, 64)) * 2 - 0.5
    ln_w = RNG.uniform(0.5, 2.0, D) * RNG.choice([-1.0, 1.0], D)
    ln_b = RNG.standard_normal(D)
    z = np.zeros(D)
    args = dict(r=RNG.standard_normal((T, D)), k=RNG.standard_normal((T, D)),
                v=RNG.standard_normal((T, D)), g=np.ones((T, D)), r_k=z, eps=eps)
    out, _ = output_fn(H, y, ln_w=ln_w, ln_b=ln_b, **args)
    n = ((out - ln_b) / ln_w).reshape(T, H, 64)
    var = y.var(axis=-1)
    assert np.allclose(n.mean(axis=-1), 0, atol=1e-12)
    assert np.allclose((n ** 2).mean(axis=-1), var / (var + eps), atol=1e-12)
    # a constant ln_w = lam scales the moments by lam^2 (ln_b = 0)
    lam = -1.75
    out, _ = output_fn(H, y, ln_w=np.full(D, lam), ln_b=z, **args)
    oh = out.reshape(T, H, 64)
    assert np.allclose((oh ** 2).mean(axis=-1), lam * lam * var / (var + eps), atol=1e-12)


def test_output_ln_affine_pins():
    _check_ln_affine(TM.time_mix_output)


def _output_affine_swapped(H, y, r, k, v, g, r_k, ln_w, ln_b, eps):
    # planted mistake: n + ln_w ln_b in place of n ln_w + ln_b
    D = H * 64
    out, scale = TM.time_mix_output(H, y, r, k, v, g, r_k, np.ones(D), ln_w * ln_b, eps)
    return out, scale


def test_ln_affine_pins_fail_on_a_swapped_affine():
    with pytest.raises(AssertionError):
        _check_ln_affine(_output_affine_swapped)


# -- C ABI argument errors (no launch) -----------------------------------------------

def test_timemix_abi_rejects_bad_arguments():
    lib = _lib.load()
    buf = (ctypes.c_uint8 * 4096)()
    p = ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 16  # 16-byte aligned dummy
    ERR_ARG, ERR_SHAPE = _lib.WKV7_ERR_ARG, _lib.WKV7_ERR_SHAPE
    # token shift: null x, D not a multiple of 8, misaligned x, row stride < D
    assert lib.wkv7_token_shift_mix(None, 4, 64, p, 3, 64, p, p, 1, p, 1, p, 256, None) == ERR_ARG
    assert lib.wkv7_token_shift_mix(p, 4, 60, p, 3, 64, p, p, 1, p, 1, p, 240, None) == ERR_SHAPE
    assert lib.wkv7_token_shift_mix(p + 2, 4, 64, p, 3, 64, p, p, 1, p, 1, p, 256,
                                    None) == ERR_SHAPE
    assert lib.wkv7_token_shift_mix(p, 4, 64, p, 3, 32, p, p, 1, p, 1, p, 256, None) == ERR_ARG
    assert lib.wkv7_token_shift_mix(p, 0, 64, p, 3, 64, p, p, 1, p, 1, p, 0, None) == 0
    # no offsets (one token per sequence) with fewer sequences than tokens
    assert lib.wkv7_token_shift_mix(p, 4, 64, p, 3, 64, p, None, 3, p, 1, p, 256, None) == ERR_ARG
    # inputs: v_lora without v_first, null k, misaligned output
    assert lib.wkv7_time_mix_inputs(2, 1, p, p, p, p, p, None, p, p, p, p, p, p, p,
                                    None) == ERR_ARG
    assert lib.wkv7_time_mix_inputs(2, 1, None, p, p, p, None, None, p, p, p, p, p, p, p,
                                    None) == ERR_ARG
    assert lib.wkv7_time_mix_inputs(2, 1, p, p, p, p, None, None, p, p, p, p, p, p, p + 2,
                                    None) == ERR_SHAPE
    # output: bad y dtype, negative eps, misaligned fp32 y
    assert lib.wkv7_time_mix_output(2, 1, p, 7, p, p, p, p, p, p, p, 1e-5, p, None) == ERR_ARG
    assert lib.wkv7_time_mix_output(2, 1, p, 0, p, p, p, p, p, p, p, -1.0, p, None) == ERR_ARG
    assert lib.wkv7_time_mix_output(2, 1, p + 8, 1, p, p, p, p, p, p, p, 1e-5, p,
                                    None) == ERR_SHAPE
