#!/usr/bin/env python3
"""WKV7 slot-pool hot path on one MI355X: decode slot-steps/s (headline),
chunked-prefill tokens/s, 7B decode with slot forks, and a ragged mixed step.

Prints ONE JSON line on stdout (progress goes to stderr):
  value     config 1 decode slot-steps/s -- 256 active slots scattered in a
            512-slot pool, RWKV-7 1.5B shape (H=32, 24 layers), one token per
            slot per step through all 24 layers' WKV7 update (24 launches)
  roofline  decode kernel: algorithmic bytes per launch / average launch
            duration (HIP events on the launch stream) against 8 TB/s
  cpu_baseline  the fp32 C port (oracle/, OpenMP) on this host's cores over a
            bounded sample of the same decode workload

Inputs are synthetic (wkvm_amd.synthetic distributions), generated on the GPU
before the timed region; the per-layer input vectors (2.3 % of the bytes) are
drawn from 4 distinct sets per layer and reused across steps, while every step
reads and writes all 24 layers' distinct slot state (3 GiB, far beyond the
256 MB Infinity Cache).
"""

from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
BF16_DENSE_PEAK_TFLOPS = 2500.0

# Algorithmic bytes (one layer, one slot): fp32 state read + write 2 x 16 KiB
# per head, six bf16 input vectors and one bf16 y vector of 128 B per head.
HEAD_STATE_B = 64 * 64 * 4
HEAD_VEC_B = 64 * 2


def slot_layer_bytes(H: int) -> int:
    return H * (2 * HEAD_STATE_B + 7 * HEAD_VEC_B)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--prefill-iters", type=int, default=30)
    ap.add_argument("--no-extra", action="store_true", help="skip configs 3 and 4")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--only", choices=("fla_decode", "fork_decode_7b", "mixed_ragged",
                                       "decode_graph", "state_store", "time_mix", "proj",
                                       "request_prefill"),
                    help="run just this extra section and print its result as JSON (for "
                         "rocprofv3 runs; not the benchmark line)")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="for rocprofv3 --pmc runs: a few config-1 decode steps plus one "
                         "1 GiB slot copy (the counter calibration), then exit")
    return ap.parse_args()


class Launcher:
    """Pre-bound ctypes calls into libwkv7.so (no per-call Python validation;
    every id / shape was validated once at set-up)."""

    def __init__(self, torch, dev):
        from wkvm_amd import _lib

        self.lib = _lib.load()
        self.check = _lib.check
        self.stream = torch.cuda.current_stream(dev).cuda_stream

    def decode(self, pool, rows, H, ids, order, B, xs, y, stream=None):
        rc = self.lib.wkv7_decode_slots(pool, rows, H, ids, order, B, *xs, y, 0, 1.0,
                                        self.stream if stream is None else stream)
        if rc:
            self.check(rc, "wkv7_decode_slots")

    def prefill(self, pool, rows, H, ids, cu, nseq, T, xs, y, zero_init, order=None):
        rc = self.lib.wkv7_prefill_varlen(pool, rows, H, ids, cu, order, nseq, T, *xs, y, 0,
                                          zero_init, 1.0, self.stream)
        if rc:
            self.check(rc, "wkv7_prefill_varlen")

    def copy(self, *args):
        rc = self.lib.wkv7_slot_copy(*args, self.stream)
        if rc:
            self.check(rc, "wkv7_slot_copy")


def ptrs(xs):
    return [x.data_ptr() for x in xs]


def sorted_order(torch, ids, dev):
    """Batch rows sorted by slot id: the decode kernel's visiting order."""
    order = sorted(range(len(ids)), key=ids.__getitem__)
    return torch.tensor(order, dtype=torch.int32, device=dev)


def bench_decode(torch, dev, args, launcher):
    """Config 1: 1.5B decode, 256 of 512 slots, 24 layers."""
    from wkvm_amd import synthetic

    L, H, S, B, NSETS = 24, 32, 512, 256, 4
    gcpu = synthetic.make_generator(args.seed)
    ids = synthetic.active_slots(S, B, gcpu)
    ids_t = torch.tensor(ids, dtype=torch.int32, device=dev)
    order_t = sorted_order(torch, ids, dev)
    gdev = synthetic.make_generator(args.seed + 1, dev)
    wkv = torch.empty((L, S + 1, H, 64, 64), dtype=torch.float32, device=dev)
    wkv.normal_(0.0, 0.1, generator=gdev)
    vec_tensors = []  # kept alive for the whole run; launches use their raw pointers
    for _ in range(L):
        for _ in range(NSETS):
            vec_tensors.append(synthetic.order(synthetic.wkv7_vectors((B, H, 64), gdev)))
    vecs = [[ptrs(vec_tensors[l * NSETS + s]) for s in range(NSETS)] for l in range(L)]
    ys = [torch.empty((B, H, 64), dtype=torch.bfloat16, device=dev) for _ in range(L)]
    pools = [wkv[l].data_ptr() for l in range(L)]
    y_ptrs = [y.data_ptr() for y in ys]
    idp = ids_t.data_ptr()
    odp = order_t.data_ptr()

    def step(i, events=None):
        s = i % NSETS
        for l in range(L):
            if events is not None:
                events[2 * l].record()
            launcher.decode(pools[l], S + 1, H, idp, odp, B, vecs[l][s], y_ptrs[l])
            if events is not None:
                events[2 * l + 1].record()

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # timed region: K steps bracketed by synchronize (one rank, no barrier needed)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record()
    for i in range(args.steps):
        step(i)
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev0.elapsed_time(ev1)
    # second pass of the same K steps with an event pair around every launch
    per = []
    for i in range(args.steps):
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(2 * L)]
        step(i, evs)
        per.append(evs)
    torch.cuda.synchronize()
    durs = [evs[2 * l].elapsed_time(evs[2 * l + 1]) for evs in per for l in range(L)]
    # Launches in the timed region run back to back on one stream, so the
    # region's event time over the launch count is the kernel's average launch
    # duration (it agrees with rocprofv3's per-kernel average); a pair of events
    # around every launch adds a few microseconds of its own to each.
    avg_launch_ms = gpu_ms / (args.steps * L)
    paired_ms = sum(durs) / len(durs)
    bytes_launch = B * slot_layer_bytes(H)
    res = {
        "slot_steps_per_s": B * args.steps / wall,
        "ms_per_step": 1e3 * wall / args.steps,
        "gpu_ms_per_step": gpu_ms / args.steps,
        "hbm_gbps_step": B * args.steps * L * slot_layer_bytes(H) / wall / 1e9,
        "avg_launch_us": 1e3 * avg_launch_ms,
        "avg_launch_us_event_pairs": 1e3 * paired_ms,
        "launch_gbps": bytes_launch / (avg_launch_ms * 1e-3) / 1e9,
        "bytes_per_launch": bytes_launch,
        "bytes_per_slot_step": L * slot_layer_bytes(H),
        "launches": args.steps * L,
    }
    log(f"decode cfg1: {res['slot_steps_per_s']:.0f} slot-steps/s, {res['ms_per_step']:.3f} ms/step, "
        f"launch {res['avg_launch_us']:.1f} us = {res['launch_gbps']:.0f} GB/s")
    del wkv, vec_tensors, ys
    torch.cuda.empty_cache()
    return res


def bench_fla_decode(torch, dev, args):
    """Config 1 through fla's wkv-op signature (the reference model layer's
    decode call, wkvm/models/rwkv7.py:108-111): per layer,
    ``o, final = fused_recurrent_rwkv7(r, w, k, v, a, b, initial_state=state_l,
    output_final_state=True)`` on dense [256, H, 64, 64] states, and the
    caller keeps ``final`` as the layer's next state (as fla's Cache does).
    The call runs the decode kernel out of place: each state is read once
    and written once. Timed with the Python wrapper's per-call validation in
    the loop (events around each 24-layer step) and per kernel launch."""
    from wkvm_amd import ops, synthetic

    L, H, B, NSETS = 24, 32, 256, 4
    gdev = synthetic.make_generator(args.seed + 21, dev)
    states = [torch.empty((B, H, 64, 64), dtype=torch.float32, device=dev).normal_(
        0.0, 0.1, generator=gdev) for _ in range(L)]
    sets = [[synthetic.order(synthetic.wkv7_vectors((B, 1, H, 64), gdev)) for _ in range(NSETS)]
            for _ in range(L)]

    def step(i):
        for l in range(L):
            _, states[l] = ops.fused_recurrent_rwkv7(*sets[l][i % NSETS],
                                                      initial_state=states[l])

    for i in range(3):
        step(i)
    torch.cuda.synchronize()
    steps = max(10, args.steps // 4)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        step(i)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    layer_bytes = B * slot_layer_bytes(H)
    res = {
        "slot_steps_per_s": B / (ms * 1e-3),
        "ms_per_step": ms,
        "hbm_gbps": L * layer_bytes / (ms * 1e-3) / 1e9,
        "hbm_frac": L * layer_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
        "steps": steps,
        "state_bytes_per_layer": 2 * B * H * HEAD_STATE_B,
    }
    log(f"fla decode cfg1: {ms:.3f} ms/step ({res['slot_steps_per_s']:.0f} slot-steps/s), "
        f"{res['hbm_gbps']:.0f} GB/s = {res['hbm_frac']:.3f} of peak")
    del states, sets
    torch.cuda.empty_cache()
    return res


def bench_proj(torch, dev, args):
    """The 1.5B time-mix block's projection launches at decode size (256 rows)
    on wkv7_proj_grouped, timed on their own: stage 1 (r, k, v and the four
    LoRA down-projections, 7 products, 27.3 MB of weights), stage 2 (the four
    LoRA up-projections) and o_proj. Each sweep runs one launch per layer over
    24 layers' distinct weights and inputs (0.9 GB, beyond the 256 MB
    Infinity Cache); algorithmic bytes = weights + the distinct x rows + the
    outputs."""
    from wkvm_amd import _lib
    from wkvm_amd.layout import RWKV7StateLayout
    from wkvm_amd.timemix import RWKV7TimeMix

    L, M = 24, 256
    lay = RWKV7StateLayout.for_shape("1.5B")
    D = lay.hidden_size
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    gdev = torch.Generator(device=dev)
    gdev.manual_seed(args.seed + 31)

    def rows(n):
        return (torch.randn((M, n), generator=gdev, device=dev)).to(torch.bfloat16)

    keep, launches = [], {"stage1": [], "stage2": [], "o_proj": []}
    nbytes = {"stage1": 0, "stage2": 0, "o_proj": 0}

    def group_array(prods):
        arr = (_lib.ProjGroup * len(prods))()
        total = 0
        xs_seen = set()
        for i, (x, w, bias, act) in enumerate(prods):
            y = torch.empty((M, w.shape[0]), dtype=torch.bfloat16, device=dev)
            keep.append(y)
            arr[i] = _lib.ProjGroup(x.data_ptr(), w.data_ptr(),
                                    None if bias is None else bias.data_ptr(), y.data_ptr(),
                                    x.stride(0), w.stride(0), y.stride(0), w.shape[0],
                                    w.shape[1], _lib.WKV7_ACT_NONE if act is None else act, 0)
            total += w.numel() * 2 + y.numel() * 2 + (0 if bias is None else bias.numel() * 2)
            if x.data_ptr() not in xs_seen:
                xs_seen.add(x.data_ptr())
                total += x.numel() * 2
        return arr, total

    for layer in range(L):
        W = RWKV7TimeMix.random(lay, 1, dev, seed=args.seed + layer).w
        keep.append(W)
        xr, xw, xk, xv, xa, xg = (rows(D) for _ in range(6))
        hw, ha, hg, hv = rows(W["w1"].shape[0]), rows(W["a1"].shape[0]), rows(W["g1"].shape[0]), \
            rows(W["v1"].shape[0])
        o_in = rows(D)
        keep.extend([xr, xw, xk, xv, xa, xg, hw, ha, hg, hv, o_in])
        stages = {
            "stage1": [(xr, W["r"], None, None), (xk, W["k"], None, None), (xv, W["v"], None, None),
                       (xw, W["w1"], None, _lib.WKV7_ACT_TANH), (xa, W["a1"], None, None),
                       (xg, W["g1"], None, _lib.WKV7_ACT_SIGMOID), (xv, W["v1"], None, None)],
            "stage2": [(hw, W["w2"], W["w0"], None), (ha, W["a2"], W["a0"], None),
                       (hg, W["g2"], None, None), (hv, W["v2"], W["v0"], None)],
            "o_proj": [(o_in, W["o"], None, None)],
        }
        for name, prods in stages.items():
            arr, total = group_array(prods)
            ws_bytes = int(lib.wkv7_proj_workspace_bytes(M, arr, len(prods)))
            ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
            keep.extend([arr, ws])
            launches[name].append((arr, len(prods), ws.data_ptr() if ws_bytes else None, ws_bytes))
            nbytes[name] = total

    def sweep(name):
        for arr, n, ws, wsb in launches[name]:
            rc = lib.wkv7_proj_grouped(M, arr, n, ws, wsb, stream)
            if rc:
                _lib.check(rc, "wkv7_proj_grouped")

    res = {}
    for name in launches:
        for _ in range(2):
            sweep(name)
        torch.cuda.synchronize()
        reps = max(3, args.steps // 10)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            sweep(name)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * L)
        res[name] = {"us_per_launch": us, "algorithmic_bytes": nbytes[name],
                     "hbm_frac": nbytes[name] / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS}
        log(f"proj {name} at {M} rows: {us:.2f} us per launch, {nbytes[name] / 1e6:.1f} MB "
            f"-> {res[name]['hbm_frac']:.3f} of HBM peak")
    del keep, launches
    torch.cuda.empty_cache()
    return res


def bench_prefill(torch, dev, args, launcher):
    """Config 2: 1.5B shape, 8 sequences x 4096 tokens, zero initial state,
    final states into 8 seeded slots; per-layer launch timing over 3 distinct
    layers' inputs. Under this load the part runs at its power limit and its
    clock settles within about a second, so the launches run ~1 s (at most
    2000 launches) before the timed ones; each timed launch has its own events
    and the reported time is their median (p50), the mean beside it."""
    from wkvm_amd import ops, synthetic

    H, S, nseq, T, NL = 32, 16, 8, 4096, 3
    gcpu = synthetic.make_generator(args.seed + 2)
    ids = synthetic.active_slots(S, nseq, gcpu)
    ids_t = torch.tensor(ids, dtype=torch.int32, device=dev)
    cu_t = torch.arange(nseq + 1, dtype=torch.int32, device=dev) * T
    gdev = synthetic.make_generator(args.seed + 3, dev)
    pools = [torch.zeros((S + 1, H, 64, 64), dtype=torch.float32, device=dev) for _ in range(NL)]
    xs = [synthetic.order(synthetic.wkv7_vectors((nseq * T, H, 64), gdev)) for _ in range(NL)]
    ys = [torch.empty((nseq * T, H, 64), dtype=torch.bfloat16, device=dev) for _ in range(NL)]
    def run(l):
        launcher.prefill(pools[l].data_ptr(), S + 1, H, ids_t.data_ptr(), cu_t.data_ptr(), nseq,
                         nseq * T, ptrs(xs[l]), ys[l].data_ptr(), 1)

    warm, w0 = 0, time.perf_counter()
    while warm < 2000 and (warm < 2 or time.perf_counter() - w0 < 1.0):
        for _ in range(10):
            run(warm % NL)
            warm += 1
        torch.cuda.synchronize()
    durs = []
    t0 = time.perf_counter()
    for i in range(args.prefill_iters):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        run(i % NL)
        e1.record()
        durs.append((e0, e1))
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    times = [a.elapsed_time(b) for a, b in durs]
    ms = statistics.median(times)
    tokens = nseq * T
    bytes_layer = tokens * H * 7 * HEAD_VEC_B + nseq * H * HEAD_STATE_B
    flops_layer = tokens * H * (18 * 64 * 64 + 8 * 64 * 64)
    res = {
        "tokens_per_s_per_layer": tokens / (ms * 1e-3),
        "ms_per_layer": ms,
        "ms_per_layer_mean": sum(times) / len(times),
        "warmup_launches": warm,
        "wall_ms_per_layer": 1e3 * wall / args.prefill_iters,
        "hbm_gbps": bytes_layer / (ms * 1e-3) / 1e9,
        "mfma_util": flops_layer / (ms * 1e-3) / (BF16_DENSE_PEAK_TFLOPS * 1e12),
        "algorithmic_bytes_per_layer": bytes_layer,
        "algorithmic_flops_per_layer": flops_layer,
        "tokens_per_s_24_layers": tokens / (ms * 1e-3) / 24,
    }
    log(f"prefill cfg2: {res['tokens_per_s_per_layer']:.3e} tok/s/layer, {ms:.3f} ms/layer, "
        f"{res['hbm_gbps']:.0f} GB/s, MFMA {100 * res['mfma_util']:.2f} %")
    del pools, xs, ys
    torch.cuda.empty_cache()
    res["one_sequence"] = bench_prefill_one_sequence(torch, dev, args)
    return res


def bench_prefill_one_sequence(torch, dev, args):
    """One long sequence (1.5B heads, 16,384 tokens, from a slot state): the
    one-pass kernel keeps 32 compute units busy; ops.wkv7_prefill_segments
    runs 4 segments side by side. Per-call time including the host side."""
    from wkvm_amd import ops, synthetic

    H, T = 32, 16384
    gdev = synthetic.make_generator(args.seed + 5, dev)
    xs = synthetic.order(synthetic.wkv7_vectors((T, H, 64), gdev))
    pool = torch.zeros((2, H, 64, 64), dtype=torch.float32, device=dev)
    pool.normal_(0.0, 0.1, generator=gdev)
    y = torch.empty((T, H, 64), dtype=torch.bfloat16, device=dev)

    def timed(fn, reps=5):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    one = timed(lambda: ops.wkv7_prefill_varlen(pool, [1], [0, T], *xs, out=y))
    seg = timed(lambda: ops.wkv7_prefill_segments(pool, [1], [0, T], *xs, segments=4, out=y))
    res = {"tokens": T, "one_pass_ms": one, "segments4_ms": seg,
           "segments4_tokens_per_s": T / (seg * 1e-3)}
    log(f"prefill one sequence of {T} tokens (H={H}): one pass {one:.3f} ms, "
        f"4 segments {seg:.3f} ms")
    del xs, pool, y
    torch.cuda.empty_cache()
    return res


def bench_request_prefill(torch, dev, args, launcher):
    """One 4,096-token request at the reference's own call pattern: RWKV7Runner
    prefill in prefill_chunk = 512 slices at batch 1 (wkvm/runner/runner.py:
    52-61, one request per call from wkvm/engine.py:152-153), each slice
    through every one of the 24 layers (1.5B heads, each layer its own
    state). Three ways in, each from the same zero-initialised state:
    * fla: chunk_rwkv7(initial_state=, output_final_state=True) per layer and
      slice, as the model layer calls it (wkvm/models/rwkv7.py:108-113);
    * runner: WKV7Runner.prefill on the slot pool (state in its slot row);
    * launcher: the same 192 launches through pre-bound ctypes calls, i.e. the
      kernels with no per-call Python work (what the GPU side takes).
    Whole-request time from events around it (inputs resident in HBM)."""
    from wkvm_amd import ops, synthetic
    from wkvm_amd.layout import RWKV7StateLayout
    from wkvm_amd.runner import WKV7Runner
    from wkvm_amd.state import RWKV7StateBank

    H, T, L, chunk = 32, 4096, 24, 512
    gdev = synthetic.make_generator(args.seed + 9, dev)
    xs = [synthetic.order(synthetic.wkv7_vectors((T, H, 64), gdev)) for _ in range(L)]
    lay = RWKV7StateLayout(n_layer=L, hidden_size=H * 64, num_heads=H, head_dim=64,
                           head_v_dim=64, dtype=torch.bfloat16)
    bank = RWKV7StateBank(lay, num_slots=1, device=dev)
    run = WKV7Runner(bank, prefill_chunk=chunk)
    # the model layer hands chunk_rwkv7 one slice's [1, chunk, H, 64] tensors
    # (wkvm/models/rwkv7.py:108-113); cut them before the timed region
    fla_x = [[[x.unsqueeze(0)[:, c:c + chunk] for x in layer] for layer in xs]
             for c in range(0, T, chunk)]
    ys = [torch.empty((T, H, 64), dtype=torch.bfloat16, device=dev) for _ in range(L)]
    ids_t = torch.tensor([1], dtype=torch.int32, device=dev)
    cu_t = torch.tensor([0, chunk], dtype=torch.int32, device=dev)
    slot = {"wkv": 1, "shift": 1}

    def fla():
        states = [None] * L
        for sl in fla_x:
            for l in range(L):
                _, states[l] = ops.chunk_rwkv7(*sl[l], initial_state=states[l],
                                               output_final_state=True)
        return states

    def runner():
        bank.zero_slots(slot)
        run.prefill(xs, slot)

    rows = bank.num_slots + 1
    esz = 2 * H * 64  # bytes per token row of one input

    def raw():
        for c in range(0, T, chunk):
            for l in range(L):
                launcher.prefill(bank.wkv[l].data_ptr(), rows, H, ids_t.data_ptr(),
                                 cu_t.data_ptr(), 1, chunk,
                                 [x.data_ptr() + c * esz for x in xs[l]],
                                 ys[l].data_ptr() + c * esz, 1 if c == 0 else 0)

    def timed(fn, reps=5):
        fn()
        torch.cuda.synchronize()
        out = []
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0 = time.perf_counter()
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            out.append((e0.elapsed_time(e1), 1e3 * (time.perf_counter() - t0)))
        return statistics.median(o[0] for o in out), statistics.median(o[1] for o in out)

    res = {"tokens": T, "layers": L, "heads": H, "prefill_chunk": chunk, "launches": L * T // chunk}
    for name, fn in (("fla", fla), ("runner", runner), ("launcher", raw)):
        ms, wall = timed(fn)
        res[f"{name}_ms"] = ms
        res[f"{name}_wall_ms"] = wall
        res[f"{name}_tokens_per_s"] = T / (ms * 1e-3)
        log(f"request prefill ({T} tokens, chunk {chunk}, {L} layers, H={H}) via {name}: "
            f"{ms:.3f} ms ({T / (ms * 1e-3):.3e} tok/s), host wall {wall:.3f} ms")
    del xs, fla_x, ys, bank
    torch.cuda.empty_cache()
    return res


def bench_fork_decode_7b(torch, dev, args, launcher):
    """Config 3: 7B shape (H=64, 32 layers), 1024 active slots, before each of
    10 steps fork 128 seeded live slots into the 128 free slots (wkv + shift),
    then decode every active slot through all 32 layers."""
    from wkvm_amd import ops, synthetic

    L, H, D, S, B, NF, steps = 32, 64, 4096, 1152, 1024, 128, 10
    gcpu = synthetic.make_generator(args.seed + 4)
    live = synthetic.active_slots(1024, B, gcpu)
    free = list(range(1025, S + 1))
    gdev = synthetic.make_generator(args.seed + 5, dev)
    wkv = torch.empty((L, S + 1, H, 64, 64), dtype=torch.float32, device=dev)
    wkv.normal_(0.0, 0.1, generator=gdev)
    shift = torch.zeros((L, 2, S + 1, D), dtype=torch.bfloat16, device=dev)
    ids_t = torch.tensor(live, dtype=torch.int32, device=dev)
    order_t = sorted_order(torch, live, dev)
    xs_keep = [synthetic.order(synthetic.wkv7_vectors((B, H, 64), gdev)) for _ in range(L)]
    xs = [ptrs(x) for x in xs_keep]
    ys = [torch.empty((B, H, 64), dtype=torch.bfloat16, device=dev) for _ in range(L)]
    srcs = []
    for _ in range(steps + 1):
        pick = torch.randperm(B, generator=gcpu)[:NF].tolist()
        srcs.append(torch.tensor([live[i] for i in pick], dtype=torch.int32, device=dev))
    dst_t = torch.tensor(free, dtype=torch.int32, device=dev)
    w_os, w_ss, w_rows, w_rb = ops.slot_view(wkv, 1)[1:]
    s_outer, s_os, s_ss, s_rows, s_rb = ops.slot_view(shift, 2)

    def fork(i):
        launcher.copy(wkv.data_ptr(), w_os, w_ss, w_rows, dst_t.data_ptr(), wkv.data_ptr(), w_os,
                      w_ss, w_rows, srcs[i].data_ptr(), L, w_rb, NF)
        launcher.copy(shift.data_ptr(), s_os, s_ss, s_rows, dst_t.data_ptr(), shift.data_ptr(),
                      s_os, s_ss, s_rows, srcs[i].data_ptr(), s_outer, s_rb, NF)

    def decode():
        for l in range(L):
            launcher.decode(wkv[l].data_ptr(), S + 1, H, ids_t.data_ptr(), order_t.data_ptr(), B, xs[l],
                            ys[l].data_ptr())

    fork(steps)
    decode()
    torch.cuda.synchronize()
    fork_ms, dec_ms = [], []
    t0 = time.perf_counter()
    for i in range(steps):
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        e[0].record()
        fork(i)
        e[1].record()
        decode()
        e[2].record()
        fork_ms.append((e[0], e[1]))
        dec_ms.append((e[1], e[2]))
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    f_ms = sum(a.elapsed_time(b) for a, b in fork_ms) / steps
    d_ms = sum(a.elapsed_time(b) for a, b in dec_ms) / steps
    fork_bytes = 2 * NF * L * (H * HEAD_STATE_B + 2 * D * 2)
    res = {
        "slot_steps_per_s": B / (d_ms * 1e-3),
        "decode_ms_per_step": d_ms,
        "decode_hbm_gbps": B * L * slot_layer_bytes(H) / (d_ms * 1e-3) / 1e9,
        "fork_ms_per_round": f_ms,
        "fork_gbps": fork_bytes / (f_ms * 1e-3) / 1e9,
        "fork_slots_per_s": NF / (f_ms * 1e-3),
        "wall_ms_per_step": 1e3 * wall / steps,
    }
    log(f"7B fork+decode cfg3: decode {d_ms:.2f} ms/step ({res['decode_hbm_gbps']:.0f} GB/s), "
        f"fork {f_ms:.3f} ms/round ({res['fork_gbps']:.0f} GB/s)")
    del wkv, shift, xs_keep, ys
    torch.cuda.empty_cache()
    return res


def bench_mixed(torch, dev, args, launcher):
    """Config 4: 1.5B, 1024-slot pool; 64 rows prefill U[1, 2048] tokens from
    zero state plus 448 rows decode one token; one decode launch and one varlen
    prefill launch per layer, 24 layers = one scheduler step. Timed with the
    decode launches on a side stream (the runner's schedule) and on one stream."""
    from wkvm_amd import ops, synthetic

    L, H, S, NP, ND = 24, 32, 1024, 64, 448
    gcpu = synthetic.make_generator(args.seed + 6)
    slots = synthetic.active_slots(S, NP + ND, gcpu)
    pre, dec = slots[:NP], slots[NP:]
    lens = synthetic.ragged_lengths(NP, 1, 2048, gcpu)
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    T = cu[-1]
    gdev = synthetic.make_generator(args.seed + 7, dev)
    wkv = torch.empty((L, S + 1, H, 64, 64), dtype=torch.float32, device=dev)
    wkv.normal_(0.0, 0.1, generator=gdev)
    pre_t = torch.tensor(pre, dtype=torch.int32, device=dev)
    dec_t = torch.tensor(dec, dtype=torch.int32, device=dev)
    dec_order = sorted_order(torch, dec, dev)
    cu_t = torch.tensor(cu, dtype=torch.int32, device=dev)
    lpt_t = torch.tensor(ops.longest_first(cu), dtype=torch.int32, device=dev)
    dx = [synthetic.order(synthetic.wkv7_vectors((ND, H, 64), gdev)) for _ in range(L)]
    px = [synthetic.order(synthetic.wkv7_vectors((T, H, 64), gdev)) for _ in range(2)]
    dy = torch.empty((ND, H, 64), dtype=torch.bfloat16, device=dev)
    py = torch.empty((T, H, 64), dtype=torch.bfloat16, device=dev)

    side = torch.cuda.Stream(dev)  # default priority
    main = torch.cuda.current_stream(dev)

    def step(order=lpt_t.data_ptr(), decode=True, concurrent=False):
        # concurrent: each layer's prefill on the main stream, then its decode
        # on a side stream forked from and joined into the main stream
        # (WKV7Runner.mixed_step's schedule)
        if decode and concurrent:
            side.wait_stream(main)
        for l in range(L):
            if decode and not concurrent:
                launcher.decode(wkv[l].data_ptr(), S + 1, H, dec_t.data_ptr(),
                                dec_order.data_ptr(), ND, ptrs(dx[l]), dy.data_ptr())
            launcher.prefill(wkv[l].data_ptr(), S + 1, H, pre_t.data_ptr(), cu_t.data_ptr(), NP, T,
                             ptrs(px[l % 2]), py.data_ptr(), 1, order)
            if decode and concurrent:
                launcher.decode(wkv[l].data_ptr(), S + 1, H, dec_t.data_ptr(),
                                dec_order.data_ptr(), ND, ptrs(dx[l]), dy.data_ptr(),
                                stream=side.cuda_stream)
        if decode and concurrent:
            main.wait_stream(side)

    def timed(**kw):
        reps = 3
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            step(**kw)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    step()
    step(concurrent=True)
    torch.cuda.synchronize()
    ms_serial = timed()
    ms = timed(concurrent=True)
    # the ragged prefill alone, longest-first vs index order of the sequences
    pre_lpt, pre_idx = timed(decode=False), timed(decode=False, order=None)
    step_bytes = L * (ND * slot_layer_bytes(H) + T * H * 7 * HEAD_VEC_B + NP * H * HEAD_STATE_B)
    res = {
        "ms_per_step": ms,
        "prefill_tokens": T,
        "hbm_gbps": step_bytes / (ms * 1e-3) / 1e9,
        "tokens_per_s": (T + ND) / (ms * 1e-3),
        "ms_per_step_single_stream": ms_serial,
        "prefill_ms_longest_first": pre_lpt,
        "prefill_ms_index_order": pre_idx,
    }
    log(f"mixed cfg4: {ms:.2f} ms/step over 24 layers (decode on a side stream; "
        f"{ms_serial:.2f} ms on one stream), {T} prefill tokens + {ND} decodes, "
        f"{res['hbm_gbps']:.0f} GB/s; prefill alone {pre_lpt:.2f} ms longest-first, "
        f"{pre_idx:.2f} ms index order")
    del wkv, dx, px, dy, py
    torch.cuda.empty_cache()
    return res


def bench_decode_graph(torch, dev, args):
    """Decode step (1.5B shape, 24 layers, 512-slot pool) as eager launches
    through the Python ops layer vs one replay of the captured HIP graph
    (wkvm_amd.graph.DecodeGraph), per batch size: where launch overhead
    matters (small batches) the graph removes it."""
    from wkvm_amd import ops, synthetic
    from wkvm_amd.graph import DecodeGraph
    from wkvm_amd.layout import RWKV7StateLayout
    from wkvm_amd.state import RWKV7StateBank

    L, H, S = 24, 32, 512
    layout = RWKV7StateLayout.for_shape("1.5B")
    bank = RWKV7StateBank(layout, S, device=dev)
    gdev = synthetic.make_generator(args.seed + 8, dev)
    res = {}
    for B in (1, 8, 64, 256):
        slots = synthetic.active_slots(S, B, synthetic.make_generator(args.seed + 9))
        xs = [synthetic.order(synthetic.wkv7_vectors((B, H, 64), gdev)) for _ in range(L)]
        ids, order = ops.decode_plan(slots, S + 1, dev)
        y = torch.empty((L, B, H, 64), dtype=torch.bfloat16, device=dev)

        def eager():
            for l in range(L):
                ops.wkv7_decode_slots(bank.wkv[l], ids, *xs[l], out=y[l], row_order=order)

        dg = DecodeGraph(bank, B)
        dg.set_slots(slots)
        dg.set_inputs(xs)
        times = {}
        for name, fn in (("eager", eager), ("graph", dg.replay)):
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            n = 50
            t0 = time.perf_counter()
            for _ in range(n):
                fn()
            torch.cuda.synchronize()
            times[name] = 1e6 * (time.perf_counter() - t0) / n
        res[f"B{B}"] = {"eager_us_per_step": times["eager"], "graph_us_per_step": times["graph"]}
        log(f"decode step B={B}: eager {times['eager']:.1f} us, graph {times['graph']:.1f} us")
        del dg, xs, y
    del bank
    torch.cuda.empty_cache()
    return res


def bench_store(torch, dev, args):
    """StateStore HOT <-> WARM transfer of one session's state (every layer's
    wkv and shift rows), vs the reference's Tensor.copy_ of the non-contiguous
    slot views (wkvm/store.py:130-131, 151-152), same pinned host tensors, same
    slots. ``save`` is the StateStore path (both families gathered into a
    device staging buffer by wkv7_slot_copy, then one contiguous DMA each);
    ``save_strided`` is wkv7_slot_transfer's 2-D DMA; ``load`` is
    wkv7_slot_transfer's 2-D DMA, the StateStore load path."""
    from wkvm_amd import ops
    from wkvm_amd.layout import RWKV7StateLayout
    from wkvm_amd.state import RWKV7StateBank

    res = {}
    for shape in ("1.5B", "7B"):
        bank = RWKV7StateBank(RWKV7StateLayout.for_shape(shape), 8, device=dev)
        bank.wkv.normal_()
        slot = 5
        hw = torch.empty(bank.wkv[:, slot].shape, dtype=bank.wkv.dtype, pin_memory=True)
        hs = torch.empty(bank.shift[:, :, slot].shape, dtype=bank.shift.dtype, pin_memory=True)
        wb, sb = hw.numel() * hw.element_size(), hs.numel() * hs.element_size()
        nbytes = wb + sb
        staging = torch.empty(wb + sb, dtype=torch.uint8, device=dev)
        stw = staging[:wb].view(hw.dtype).view(hw.shape)
        sts = staging[wb:].view(hs.dtype).view(hs.shape)

        def save():
            ops.slot_gather_dense(bank.wkv, slot, 1, stw)
            ops.slot_gather_dense(bank.shift, slot, 2, sts)
            hw.copy_(stw, non_blocking=True)
            hs.copy_(sts, non_blocking=True)

        def save_strided():
            ops.slot_to_host(bank.wkv, slot, 1, hw)
            ops.slot_to_host(bank.shift, slot, 2, hs)

        def load():
            ops.slot_from_host(bank.wkv, slot, 1, hw)
            ops.slot_from_host(bank.shift, slot, 2, hs)

        def ref_save():
            hw.copy_(bank.wkv[:, slot], non_blocking=True)
            hs.copy_(bank.shift[:, :, slot], non_blocking=True)

        def ref_load():
            bank.wkv[:, slot].copy_(hw, non_blocking=True)
            bank.shift[:, :, slot].copy_(hs, non_blocking=True)

        out = {"bytes_per_slot": nbytes}
        fns = (("save", save), ("save_strided", save_strided), ("load", load),
               ("ref_save", ref_save), ("ref_load", ref_load))
        # The host link runs slower for the first milliseconds of traffic after
        # GPU-only work, so every variant is warmed up and then timed in
        # interleaved rounds: all of them see the same link state.
        ts = {name: [] for name, _ in fns}
        for i in range(40):
            for name, fn in fns:
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                fn()
                torch.cuda.synchronize()
                if i >= 10:
                    ts[name].append(time.perf_counter() - t0)
        for name, _ in fns:
            med = statistics.median(ts[name])
            out[f"{name}_us"] = 1e6 * med
            out[f"{name}_gbps"] = nbytes / med / 1e9
        res[shape] = out
        log(f"state store {shape}: {nbytes / 2**20:.1f} MiB/slot; save {out['save_us']:.0f} us "
            f"({out['save_gbps']:.1f} GB/s; strided DMA {out['save_strided_us']:.0f} us) vs "
            f"Tensor.copy_ {out['ref_save_us']:.0f} us; load {out['load_us']:.0f} us "
            f"({out['load_gbps']:.1f} GB/s) vs Tensor.copy_ {out['ref_load_us']:.0f} us")
        del bank, hw, hs, staging, stw, sts
        torch.cuda.empty_cache()
    return res


def bench_time_mix(torch, dev, args):
    """The RWKV-7 time-mix stages around the WKV op at the 1.5B width
    (D = 2048, H = 32). Element-wise kernels at the config-2 token count
    (8 x 4096 tokens), each timed alone with HIP events on the launch stream:
      token_shift_mix  per token: x 4 KiB + 6 mixes 24 KiB (the previous row
                       is the neighbour's x, read from cache), per sequence
                       the slot row read + written
      time_mix_inputs  per token: 6 inputs (k, v, w/a/v LoRA, v_first) read,
                       5 outputs written, 4 KiB each
      time_mix_output  per token: y, r, k, v, g read, 1 output written
    and the whole block (shift, GEMMs, kernels, WKV, o_proj) per layer for a
    256-slot decode step and for the 8 x 4096-token prefill."""
    from wkvm_amd import ops
    from wkvm_amd.layout import RWKV7StateLayout
    from wkvm_amd.state import RWKV7StateBank
    from wkvm_amd.timemix import RWKV7TimeMix, TimeMixDecodeGraph, TokenBatch

    layout = RWKV7StateLayout.for_shape("1.5B")
    D, H = layout.hidden_size, layout.num_heads
    nseq, T = 8, 4096
    N = nseq * T
    bank = RWKV7StateBank(layout, 512, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed + 40)

    def rnd(*shape):
        return torch.randn(shape, generator=g, device=dev).to(torch.bfloat16)

    def timed(fn, iters=10):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / iters * 1e3  # us

    slots = list(range(1, nseq + 1))
    cu = [i * T for i in range(nseq + 1)]
    ids_t = torch.tensor(slots, dtype=torch.int32, device=dev)
    cu_t = torch.tensor(cu, dtype=torch.int32, device=dev)
    x = rnd(N, D)
    mix = rnd(6, D)
    shift_out = torch.empty((6, N, D), dtype=torch.bfloat16, device=dev)
    k, v, wl, al, vl, vf = (rnd(N, D) for _ in range(6))
    kk, ka = rnd(D), rnd(D)
    y = rnd(N, H, 64)
    r, gg = rnd(N, D), rnd(N, D)
    rk, lw, lb = rnd(D), rnd(D), rnd(D)
    res = {}
    kern = {
        "token_shift_mix": (lambda: ops.token_shift_mix(x, bank.shift[1, 0], ids_t, mix, cu_t,
                                                        out=shift_out),
                            N * D * 2 * 7 + nseq * D * 2 * 2),
        "time_mix_inputs": (lambda: ops.time_mix_inputs(H, k, v, wl, al, kk, ka, vl, vf),
                            N * D * 2 * 11),
        "time_mix_output": (lambda: ops.time_mix_output(H, y, r, k, v, gg, rk, lw, lb, 64e-5),
                            N * D * 2 * 6),
    }
    for name, (fn, nbytes) in kern.items():
        us = timed(fn)
        res[name] = {"us": us, "bytes": nbytes, "gbps": nbytes / (us * 1e-6) / 1e9,
                     "frac_hbm_peak": nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS}
        log(f"time-mix {name}: {N} tokens x D={D}: {us:.1f} us, "
            f"{res[name]['gbps']:.0f} GB/s ({100 * res[name]['frac_hbm_peak']:.1f} % of peak)")
    del shift_out, k, v, wl, al, vl, vf, y, r, gg
    # whole block, layer 1 (with the v_first lerp)
    layer = RWKV7TimeMix.random(layout, 1, dev, seed=args.seed)
    gen = torch.Generator().manual_seed(args.seed + 41)
    dslots = (torch.randperm(512, generator=gen)[:256] + 1).tolist()
    for mode, xin, batch in (
            ("decode_256", rnd(256, D), TokenBatch.plan(bank, dslots)),
            ("prefill_8x4096", x, TokenBatch.plan(bank, slots, cu))):
        vfirst = rnd(int(xin.shape[0]), D)
        us = timed(lambda: layer.forward(bank, xin, batch, vfirst), iters=5)
        res[f"block_{mode}_us"] = us
        log(f"time-mix block (1.5B layer, {mode}): {us:.1f} us per layer")
    del x
    # the whole 24-layer time-mix decode step for 256 slots: eager vs one graph
    layers = [RWKV7TimeMix.random(layout, l, dev, seed=args.seed) for l in range(layout.n_layer)]
    tg = TimeMixDecodeGraph(bank, layers, 256)
    tg.set_slots(dslots)
    tg.x.copy_(rnd(layout.n_layer, 256, D))
    batch = TokenBatch.plan(bank, dslots)

    def eager_step():
        vf = None
        for l, lay in enumerate(layers):
            _, vf = lay.forward(bank, tg.x[l], batch, vf)

    eager_us = timed(eager_step, iters=5)
    graph_us = timed(tg.replay, iters=10)
    # the same step with the projections on the vendor BLAS (two side streams)
    saved = RWKV7TimeMix.PROJ_MAX_ROWS
    RWKV7TimeMix.PROJ_MAX_ROWS = 0
    try:
        tg_blas = TimeMixDecodeGraph(bank, layers, 256, side_streams=2)
    finally:
        RWKV7TimeMix.PROJ_MAX_ROWS = saved
    tg_blas.set_slots(dslots)
    tg_blas.x.copy_(tg.x)
    blas_us = timed(tg_blas.replay, iters=10)
    res["decode_step_24_layers"] = {"eager_us": eager_us, "graph_us": graph_us,
                                    "slot_steps_per_s_graph": 256 / (graph_us * 1e-6),
                                    "graph_us_vendor_blas": blas_us}
    log(f"time-mix decode step, 24 layers x 256 slots: eager {eager_us:.0f} us, graph "
        f"{graph_us:.0f} us ({256 / (graph_us * 1e-6):.0f} slot-steps/s); projections on "
        f"the vendor BLAS: graph {blas_us:.0f} us")
    del bank, tg, tg_blas, layers
    torch.cuda.empty_cache()
    return res


def cpu_model() -> str | None:
    """The host CPU's model name (/proc/cpuinfo), for the baseline record."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_baseline(args):
    """fp32 C port (oracle/) on this host, OpenMP over every core in this
    process's affinity set: config-1 decode (24 layers x 256 slots of a
    512-slot pool) for as many steps as fit ~10 s, at least one; then config-2
    prefill (one layer, 8 sequences) for ~5 s."""
    import numpy as np
    import torch

    import oracle as O
    from wkvm_amd import synthetic

    affinity = len(os.sched_getaffinity(0))
    threads = affinity  # every core this process may run on
    O.set_threads(threads)
    L, H, S, B = 24, 32, 512, 256
    gen = synthetic.make_generator(args.seed)
    ids = synthetic.active_slots(S, B, gen)
    pool = np.zeros((L, S + 1, H, 64, 64), dtype=np.float32)
    for l in range(L):
        pool[l, ids] = 0.01
    vecs = [synthetic.wkv7_vectors((B, H, 64), gen) for _ in range(L)]
    bits = [[v[n].contiguous().view(torch.int16).numpy().view(np.uint16) for n in "rwkvab"]
            for v in vecs]
    steps, t0 = 0, time.perf_counter()
    while True:
        for l in range(L):
            O.port_decode_slots_f32(pool[l], ids, *bits[l])
        steps += 1
        el = time.perf_counter() - t0
        if el > 10.0 or steps >= 400:
            break
    res = {
        "value": B * steps / el,
        "unit": "slot-steps/s",
        "cores": threads,
        "threads": threads,
        "nproc": os.cpu_count(),
        "affinity_cores": affinity,
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": f"{steps} config-1 decode steps (24 layers x 256 slots, H=32), fp32 C port "
                  f"with OpenMP, {el:.1f} s",
    }
    log(f"cpu baseline: {res['value']:.1f} slot-steps/s on {threads} threads ({steps} steps; "
        f"nproc {res['nproc']}, affinity {affinity}, {res['cpu_model']})")
    del pool
    # config-2 prefill (one layer): 8 sequences from zero state, 512-token
    # slices of the 4096-token rows, repeated for ~5 s
    nseq, Tp = 8, 512
    ppool = np.zeros((nseq + 1, H, 64, 64), dtype=np.float32)
    pv = synthetic.wkv7_vectors((nseq * Tp, H, 64), gen)
    pbits = [pv[n].contiguous().view(torch.int16).numpy().view(np.uint16) for n in "rwkvab"]
    cu = [i * Tp for i in range(nseq + 1)]
    reps, t0 = 0, time.perf_counter()
    while True:
        O.port_prefill_f32(ppool, list(range(1, nseq + 1)), cu, *pbits, zero_init=reps == 0)
        reps += 1
        el = time.perf_counter() - t0
        if el > 5.0 or reps >= 24:
            break
    res["prefill"] = {
        "value": reps * nseq * Tp / el,
        "unit": "tokens/s per layer",
        "sample": f"{reps} x 8 sequences x {Tp} tokens (1.5B heads, H=32), continuing through "
                  f"the slots (up to 8 x {reps * Tp} tokens), fp32 C port with OpenMP, "
                  f"{el:.1f} s",
    }
    log(f"cpu baseline prefill: {res['prefill']['value']:.0f} tokens/s per layer on {threads} "
        f"threads")
    return res


def pmc_probe(torch, dev, args, launcher):
    """Kernels for rocprofv3 --pmc runs: config-1 decode launches (24 layers x
    3 steps after 1 warm-up step), config-2 prefill launches (1 warm-up + 2),
    and one wkv7_slot_copy of exactly 1 GiB read + 1 GiB written, so that
    FETCH_SIZE / WRITE_SIZE per dispatch can be scaled by the copy's counts."""
    from wkvm_amd import synthetic

    L, H, S, B = 24, 32, 512, 256
    gcpu = synthetic.make_generator(args.seed)
    ids = synthetic.active_slots(S, B, gcpu)
    ids_t = torch.tensor(ids, dtype=torch.int32, device=dev)
    order_t = sorted_order(torch, ids, dev)
    gdev = synthetic.make_generator(args.seed + 1, dev)
    wkv = torch.empty((L, S + 1, H, 64, 64), dtype=torch.float32, device=dev)
    wkv.normal_(0.0, 0.1, generator=gdev)
    xs = [synthetic.order(synthetic.wkv7_vectors((B, H, 64), gdev)) for _ in range(L)]
    y = torch.empty((B, H, 64), dtype=torch.bfloat16, device=dev)
    for _ in range(4):
        for l in range(L):
            launcher.decode(wkv[l].data_ptr(), S + 1, H, ids_t.data_ptr(), order_t.data_ptr(), B,
                            ptrs(xs[l]), y.data_ptr())
    torch.cuda.synchronize()
    del wkv, xs, y
    # config 2 prefill
    PS, nseq, T = 16, 8, 4096
    pids = torch.tensor(synthetic.active_slots(PS, nseq, synthetic.make_generator(args.seed + 2)),
                        dtype=torch.int32, device=dev)
    cu_t = torch.arange(nseq + 1, dtype=torch.int32, device=dev) * T
    pool = torch.zeros((PS + 1, H, 64, 64), dtype=torch.float32, device=dev)
    pxs = synthetic.order(synthetic.wkv7_vectors((nseq * T, H, 64),
                                                 synthetic.make_generator(args.seed + 3, dev)))
    py = torch.empty((nseq * T, H, 64), dtype=torch.bfloat16, device=dev)
    for _ in range(3):
        launcher.prefill(pool.data_ptr(), PS + 1, H, pids.data_ptr(), cu_t.data_ptr(), nseq,
                         nseq * T, ptrs(pxs), py.data_ptr(), 1)
    torch.cuda.synchronize()
    del pool, pxs, py
    src = torch.empty((1024, 1 << 20), dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    src.fill_(1)
    torch.cuda.synchronize()
    launcher.copy(dst.data_ptr(), 0, 1 << 20, 1024, None, src.data_ptr(), 0, 1 << 20, 1024, None,
                  1, 1 << 20, 1024)
    torch.cuda.synchronize()
    log("pmc probe done: 96 decode dispatches (first 24 warm-up), 3 prefill dispatches "
        "(first warm-up), 1 GiB calibration copy")


def profile_value(name: str, key: str):
    """A figure from a committed rocprofv3 summary under profiles/ (None if absent)."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    m = re.search(re.escape(key) + r":\s*([0-9.eE+-]+)", open(path).read())
    return float(m.group(1)) if m else None


def pmc_traffic():
    """HBM bytes per decode launch from the committed rocprofv3 PMC summary,
    if present (FETCH_SIZE + WRITE_SIZE, calibrated against a copy kernel)."""
    return profile_value("decode_cfg1_pmc.txt", "traffic_bytes_per_launch")


def main() -> int:
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: the WKV7 slot-pool path shards by slot with no "
              "exchange step, and this build runs on a single MI355X. "
              "Run with --gpus 1.", file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    launcher = Launcher(torch, dev)
    if args.pmc_probe:
        pmc_probe(torch, dev, args, launcher)
        return 0
    if args.only:
        fn = {"fla_decode": lambda: bench_fla_decode(torch, dev, args),
              "proj": lambda: bench_proj(torch, dev, args),
              "fork_decode_7b": lambda: bench_fork_decode_7b(torch, dev, args, launcher),
              "mixed_ragged": lambda: bench_mixed(torch, dev, args, launcher),
              "decode_graph": lambda: bench_decode_graph(torch, dev, args),
              "state_store": lambda: bench_store(torch, dev, args),
              "time_mix": lambda: bench_time_mix(torch, dev, args),
              "request_prefill": lambda: bench_request_prefill(torch, dev, args, launcher)}[args.only]
        print(json.dumps({args.only: fn()}), flush=True)
        return 0
    dec = bench_decode(torch, dev, args, launcher)
    pre = bench_prefill(torch, dev, args, launcher)
    extra = {}
    if not args.no_extra:
        extra["request_prefill"] = bench_request_prefill(torch, dev, args, launcher)
        extra["fla_decode"] = bench_fla_decode(torch, dev, args)
        extra["fork_decode_7b"] = bench_fork_decode_7b(torch, dev, args, launcher)
        extra["mixed_ragged"] = bench_mixed(torch, dev, args, launcher)
        extra["decode_graph"] = bench_decode_graph(torch, dev, args)
        extra["state_store"] = bench_store(torch, dev, args)
        extra["time_mix"] = bench_time_mix(torch, dev, args)
        extra["proj"] = bench_proj(torch, dev, args)
    cpu = None if args.no_cpu_baseline else cpu_baseline(args)
    line = {
        "metric": "WKV7 decode slot-steps/s + achieved HBM GB/s; chunked-prefill tokens/s",
        "value": round(dec["slot_steps_per_s"], 1),
        "unit": "slot-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32 state / bf16 vectors",
        "data": "synthetic (seeded; BASELINE input distributions)",
        "config": {
            "workload": "config 1: WKV7 decode, RWKV-7 1.5B shape (H=32, N=64, 24 layers), "
                        "256 active slots scattered in a 512-slot fp32 pool, 1 token/slot/step",
            "slots": 256, "pool": 512, "layers": 24, "heads": 32, "head_size": 64,
            "parallelism": "single GPU",
        },
        "hbm_gbps": round(dec["hbm_gbps_step"], 1),
        "roofline": {
            "bound": "hbm",
            "achieved": round(dec["launch_gbps"], 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(dec["launch_gbps"] / HBM_PEAK_GBPS, 4),
            "traffic": pmc_traffic(),
            "kernel": "decode_slots_kernel",
            "bytes_per_launch": dec["bytes_per_launch"],
            "avg_launch_us": round(dec["avg_launch_us"], 2),
            "avg_launch_us_event_pairs": round(dec["avg_launch_us_event_pairs"], 2),
            "traffic_source": "profiles/decode_cfg1_pmc.txt (rocprofv3 FETCH_SIZE/WRITE_SIZE, "
                              "copy-calibrated)",
        },
        "decode": {k: (round(v, 4) if isinstance(v, float) else v) for k, v in dec.items()},
        "prefill": {
            **{k: (round(v, 6) if isinstance(v, float) else v) for k, v in pre.items()},
            "pmc": {
                "mfma_busy_frac": profile_value("prefill_cfg2_pmc.txt", "mfma_busy_frac"),
                "mfma_executed_tflops": profile_value("prefill_cfg2_pmc.txt",
                                                      "mfma_executed_tflops"),
                "traffic_bytes": profile_value("prefill_cfg2_pmc.txt", "traffic_bytes_per_launch"),
                "source": "profiles/prefill_cfg2_pmc.txt (rocprofv3 SQ_VALU_MFMA_BUSY_CYCLES, "
                          "SQ_INSTS_VALU_MFMA_MOPS_BF16, FETCH_SIZE/WRITE_SIZE)",
            },
        },
        **{k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
           for k, v in extra.items()},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
