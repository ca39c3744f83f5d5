"""wkv7_proj_grouped_noalloc: the projection entry point that allocates
nothing, its split-k partials in the library's static per-GPU buffer.

Checked through the C ABI against wkv7_proj_grouped given the workspace it
asks for (same plan, so the outputs must be bit-identical) and against the
float64 product (within one bf16 ulp), on two calls in a row whose second
input is smaller, both of which split k. The second call reuses the buffer the
first one left its partials in."""

import math

import numpy as np
import pytest
import torch

from wkvm_amd import _lib

pytestmark = pytest.mark.gpu


def _rand(shape, gen, dev, std=1.0):
    return (torch.randn(shape, generator=gen) * std).to(torch.bfloat16).to(dev)


def _exact(x, w, bias, act):
    y = x.double().cpu() @ w.double().cpu().T
    if bias is not None:
        y = y + bias.double().cpu()
    if act == _lib.WKV7_ACT_TANH:
        y = torch.tanh(y)
    elif act == _lib.WKV7_ACT_SIGMOID:
        y = torch.sigmoid(y)
    return y


def _assert_within_one_ulp(got, exact):
    got = got.double().cpu()
    mag = exact.abs().clamp_min(1e-3 * exact.pow(2).mean().sqrt().item() + 1e-30)
    ulp = torch.exp2(torch.floor(torch.log2(mag)) - 7)
    worst = ((got - exact).abs() / ulp).max().item()
    assert worst <= 1.0, f"max error {worst:.3f} bf16 ulp"


def _groups(products):
    arr = (_lib.ProjGroup * len(products))()
    for i, (x, w, b, y, act) in enumerate(products):
        arr[i] = _lib.ProjGroup(x.data_ptr(), w.data_ptr(), None if b is None else b.data_ptr(),
                                y.data_ptr(), x.shape[1], w.shape[1], y.shape[1], w.shape[0],
                                x.shape[1], act, 0)
    return arr


def _case(gen, dev, M, K, ns, acts):
    prods = []
    for n, act in zip(ns, acts):
        x = _rand((M, K), gen, dev)
        w = _rand((n, K), gen, dev, 1 / math.sqrt(K))
        b = _rand((n,), gen, dev) if act != _lib.WKV7_ACT_NONE else None
        prods.append((x, w, b, act))
    return prods


def test_noalloc_matches_the_workspace_entry_point_on_two_calls(dev):
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    gen = torch.Generator().manual_seed(7001)
    cases = [
        # first call: one long-k product and a LoRA-sized one at 4 rows
        (4, 2048, [2048, 96], [_lib.WKV7_ACT_NONE, _lib.WKV7_ACT_TANH]),
        # second call, smaller: one row, k = 1024, n = 1024
        (1, 1024, [1024], [_lib.WKV7_ACT_SIGMOID]),
    ]
    for M, K, ns, acts in cases:
        prods = _case(gen, dev, M, K, ns, acts)
        ys_ref = [torch.empty((M, w.shape[0]), dtype=torch.bfloat16, device=dev)
                  for _, w, _, _ in prods]
        ys = [torch.full((M, w.shape[0]), 7.0, dtype=torch.bfloat16, device=dev)
              for _, w, _, _ in prods]
        ref_arr = _groups([(x, w, b, y, a) for (x, w, b, a), y in zip(prods, ys_ref)])
        arr = _groups([(x, w, b, y, a) for (x, w, b, a), y in zip(prods, ys)])
        ws_bytes = int(lib.wkv7_proj_workspace_bytes(M, ref_arr, len(prods)))
        assert 0 < ws_bytes <= _lib.WKV7_PROJ_STATIC_SCRATCH_BYTES, \
            "the case must take the split-k path, within the static buffer"
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        assert lib.wkv7_proj_grouped(M, ref_arr, len(prods), ws.data_ptr(), ws_bytes,
                                     stream) == 0
        assert lib.wkv7_proj_grouped_noalloc(M, arr, len(prods), stream) == 0
        torch.cuda.synchronize()
        for (x, w, b, a), y, y_ref in zip(prods, ys, ys_ref):
            assert torch.equal(y, y_ref), f"M={M} K={K}: differs from the workspace entry point"
            _assert_within_one_ulp(y, _exact(x, w, b, a))


def test_noalloc_unsplit_and_rejections(dev):
    """Enough rows for an unsplit plan (no scratch touched), zero rows, and
    argument errors returned before any launch."""
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    gen = torch.Generator().manual_seed(7002)
    (x, w, b, a), = _case(gen, dev, 256, 512, [512], [_lib.WKV7_ACT_NONE])
    y = torch.empty((256, 512), dtype=torch.bfloat16, device=dev)
    arr = _groups([(x, w, b, y, a)])
    assert lib.wkv7_proj_workspace_bytes(256, arr, 1) == 0
    assert lib.wkv7_proj_grouped_noalloc(256, arr, 1, stream) == 0
    torch.cuda.synchronize()
    _assert_within_one_ulp(y, _exact(x, w, b, a))
    assert lib.wkv7_proj_grouped_noalloc(0, arr, 1, stream) == 0
    assert lib.wkv7_proj_grouped_noalloc(-1, arr, 1, stream) == _lib.WKV7_ERR_ARG
    assert lib.wkv7_proj_grouped_noalloc(4, None, 1, stream) == _lib.WKV7_ERR_ARG
    assert np.isfinite(y.float().cpu().numpy()).all()
