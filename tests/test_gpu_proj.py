"""Grouped projection GEMMs (wkv7_proj_grouped) against a float64 CPU product.

The kernel accumulates in fp32 and rounds once to bf16, so every output is
within one bf16 ulp of the exact value (fp32 summation error over k <= 2048
is ~2^-12 ulp at these magnitudes). The activations are compared with the
float64 tanh / sigmoid of the exact sum.
"""

import math

import pytest
import torch

from wkvm_amd import ops

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda", 0)


def _rand(shape, gen, dev, std=1.0):
    return (torch.randn(shape, generator=gen) * std).to(torch.bfloat16).to(dev)


def _exact(x, w, bias, act):
    y = x.double().cpu() @ w.double().cpu().T
    if bias is not None:
        y = y + bias.double().cpu()
    if act == "tanh":
        y = torch.tanh(y)
    elif act == "sigmoid":
        y = torch.sigmoid(y)
    return y


def _assert_within_one_ulp(got, exact):
    got = got.double().cpu()
    mag = exact.abs().clamp_min(1e-3 * exact.pow(2).mean().sqrt().item() + 1e-30)
    ulp = torch.exp2(torch.floor(torch.log2(mag)) - 7)
    err = (got - exact).abs()
    worst = (err / ulp).max().item()
    assert worst <= 1.0, f"max error {worst:.3f} bf16 ulp"


@pytest.mark.parametrize("M", [1, 17, 256, 300])
def test_single_projection(dev, M):
    gen = torch.Generator().manual_seed(100 + M)
    x = _rand((M, 2048), gen, dev)
    w = _rand((2048, 2048), gen, dev, 1 / math.sqrt(2048))
    (y,) = ops.proj_grouped([(x, w)])
    _assert_within_one_ulp(y, _exact(x, w, None, None))


def test_time_mix_first_stage_group(dev):
    """The seven first-stage products of a time-mix layer in one launch:
    r, k, v [2048 x 2048] and the LoRA down-projections (tanh for w,
    sigmoid for g), each from its own mixed input."""
    gen = torch.Generator().manual_seed(7)
    M, D = 256, 2048
    xs = [_rand((M, D), gen, dev) for _ in range(7)]
    ns = [D, D, D, 96, 96, 256, 64]
    acts = [None, None, None, "tanh", None, "sigmoid", None]
    ws = [_rand((n, D), gen, dev, 1 / math.sqrt(D)) for n in ns]
    ys = ops.proj_grouped([(x, w, None, a) for x, w, a in zip(xs, ws, acts)])
    for x, w, a, y in zip(xs, ws, acts, ys):
        assert tuple(y.shape) == (M, w.shape[0])
        _assert_within_one_ulp(y, _exact(x, w, None, a))


@pytest.mark.parametrize("M", [3, 256])
def test_lora_second_stage_with_bias_and_k_tail(dev, M):
    """Up-projections with k = 96, 96, 64, 256 (96 leaves a 32-wide k tail)
    and a bias on three of them."""
    gen = torch.Generator().manual_seed(11 + M)
    D = 2048
    ks = [96, 96, 64, 256]
    hs = [_rand((M, k), gen, dev) for k in ks]
    ws = [_rand((D, k), gen, dev, 1 / math.sqrt(k)) for k in ks]
    bs = [_rand((D,), gen, dev, 0.5), _rand((D,), gen, dev, 0.5), _rand((D,), gen, dev, 0.5),
          None]
    ys = ops.proj_grouped(list(zip(hs, ws, bs)))
    for h, w, b, y in zip(hs, ws, bs, ys):
        _assert_within_one_ulp(y, _exact(h, w, b, None))


def test_strided_rows_in_and_out(dev):
    """x and y as column slices of wider row-major buffers (row stride > k, n)."""
    gen = torch.Generator().manual_seed(21)
    M = 40
    xbuf = _rand((M, 3 * 128), gen, dev)
    x = xbuf[:, 128:256]
    w = _rand((160, 128), gen, dev, 1 / math.sqrt(128))
    ybuf = torch.full((M, 400), 7.0, dtype=torch.bfloat16, device=dev)
    y = ybuf[:, 200:360]
    ops.proj_grouped([(x, w, None, "sigmoid")], outs=[y])
    _assert_within_one_ulp(y, _exact(x, w, None, "sigmoid"))
    assert bool((ybuf[:, :200] == 7.0).all()) and bool((ybuf[:, 360:] == 7.0).all())


def test_ragged_n_and_many_tiles(dev):
    """n not a multiple of the tile width, and a large row count."""
    gen = torch.Generator().manual_seed(5)
    M = 1000
    x = _rand((M, 256), gen, dev)
    w = _rand((72, 256), gen, dev, 1 / 16)
    b = _rand((72,), gen, dev)
    (y,) = ops.proj_grouped([(x, w, b, "tanh")])
    _assert_within_one_ulp(y, _exact(x, w, b, "tanh"))


def test_rejected_arguments(dev):
    x = torch.zeros((4, 48), dtype=torch.bfloat16, device=dev)
    w = torch.zeros((8, 48), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="multiple of 32"):
        ops.proj_grouped([(x, w)])
    x = torch.zeros((4, 64), dtype=torch.bfloat16, device=dev)
    w = torch.zeros((8, 64), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="products per launch"):
        ops.proj_grouped([(x, w)] * 9)
    with pytest.raises(ValueError, match="act"):
        ops.proj_grouped([(x, w, None, "relu")])
    with pytest.raises(ValueError, match="same row count"):
        ops.proj_grouped([(x, w), (x[:2], w)])


def test_split_k_partials_and_unsplit_fallback(dev):
    """A long-k product with few rows splits k over several workgroups when
    given the workspace it asks for (the last part holding the 32-wide k
    tail), and runs unsplit without one. Both are within one bf16 ulp of the
    exact product and each repeats bit for bit."""
    from wkvm_amd import _lib

    lib = _lib.load()
    gen = torch.Generator().manual_seed(31)
    M, K, N = 5, 1056, 2048
    x = _rand((M, K), gen, dev)
    w = _rand((N, K), gen, dev, 1 / math.sqrt(K))
    b = _rand((N,), gen, dev)
    exact = _exact(x, w, b, "tanh")
    arr = (_lib.ProjGroup * 1)()
    outs = []
    for use_ws in (True, False, True):
        y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        arr[0] = _lib.ProjGroup(x.data_ptr(), w.data_ptr(), b.data_ptr(), y.data_ptr(), K, K, N,
                                N, K, _lib.WKV7_ACT_TANH, 0)
        ws_bytes = int(lib.wkv7_proj_workspace_bytes(M, arr, 1)) if use_ws else 0
        if use_ws:
            assert ws_bytes > 0, "few rows and long k should ask for a split-k workspace"
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        rc = lib.wkv7_proj_grouped(M, arr, 1, ws.data_ptr() if use_ws else None, ws_bytes,
                                   torch.cuda.current_stream().cuda_stream)
        assert rc == 0
        torch.cuda.synchronize()
        _assert_within_one_ulp(y, exact)
        outs.append(y)
    assert torch.equal(outs[0], outs[2])


def test_split_k_over_several_groups(dev):
    """Several products with few rows split k together (different n, one
    with bias and sigmoid); every output within one bf16 ulp."""
    from wkvm_amd import _lib

    gen = torch.Generator().manual_seed(41)
    M, K = 3, 2048
    x1, x2 = _rand((M, K), gen, dev), _rand((M, K), gen, dev)
    w1 = _rand((2048, K), gen, dev, 1 / math.sqrt(K))
    w2 = _rand((96, K), gen, dev, 1 / math.sqrt(K))
    b2 = _rand((96,), gen, dev)
    ys = [torch.empty((M, w.shape[0]), dtype=torch.bfloat16, device=dev) for w in (w1, w2)]
    arr = (_lib.ProjGroup * 2)()
    for i, (x, w, b, a) in enumerate(((x1, w1, None, None), (x2, w2, b2, "sigmoid"))):
        arr[i] = _lib.ProjGroup(x.data_ptr(), w.data_ptr(), None if b is None else b.data_ptr(),
                                ys[i].data_ptr(), K, K, w.shape[0], w.shape[0], K,
                                ops.ACTIVATIONS[a], 0)
    assert _lib.load().wkv7_proj_workspace_bytes(M, arr, 2) > 0, "expected a split-k plan"
    y1, y2 = ops.proj_grouped([(x1, w1), (x2, w2, b2, "sigmoid")], outs=ys)
    _assert_within_one_ulp(y1, _exact(x1, w1, None, None))
    _assert_within_one_ulp(y2, _exact(x2, w2, b2, "sigmoid"))
