#!/usr/bin/env python3
"""Benchmark of the MI355X quantized linear layer (Kidi's PACKED_LINEAR), one GPU.

Workload of ``value`` (the decode GEMV the headline metric is quoted on): asymmetric int4,
g = 128, fp16 per-group scales, uint4 zero points, M = 1, K = 2048, N = 8192 (up-projection), bf16 activations
~N(0, 1) with 0.1% outliers x20, dynamically quantized to int8 per (row, 128-block). One step = one projection
call through the C ABI (kq_packed_linear: activation quantization + GEMV) on the next of R rotated weights, so the
weight working set (R x 8.7 MB) is larger than the 256 MB Infinity Cache and every step streams its weight from
HBM. Steps are replayed from a HIP graph on one stream, so consecutive projections are serialized as in a decoder.

Also reported (not ``value``): the prefill GEMM of configs[2] (M = 2048, K = 2048, N = 8192, same weight format)
in TOPS against the dense int8 MFMA peak, and the CPU oracle timed on this host's cores (``cpu_baseline``).

    python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
INT8_PEAK_TOPS = 5000.0      # MI355X dense int8 MFMA, TOP/s

# decode up-projection
K_DEC, N_DEC, G_DEC, M_DEC = 2048, 8192, 128, 1
# prefill
M_PRE, K_PRE, N_PRE, G_PRE = 2048, 2048, 8192, 128


def gemv_bytes(M, K, N, g, bits=4, asym=True):
    """Algorithmic HBM bytes of one projection: packed codes + fp16 scales + uint4 zero points + bf16 x + fp32 y."""
    return N * K * bits // 8 + N * (K // g) * 2 + (N * (K // g) // 2 if asym else 0) + M * K * 2 + M * N * 4


def parse():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=6400, help="timed decode projections")
    p.add_argument("--warmup", type=int, default=256, help="untimed decode projections before timing")
    p.add_argument("--rotate", type=int, default=64, help="distinct weights cycled through (>= 32)")
    p.add_argument("--prefill-steps", type=int, default=50)
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample budget (0 = skip)")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--no-extras", action="store_true",
                   help="skip the configs[3]/configs[4] projections and the fused-operator timings")
    p.add_argument("--floor-sweep", action="store_true",
                   help="print the single-launch read floor and empty-launch cost over launch geometries "
                        "(kq_debug_read_floor_shape) as a table and exit")
    p.add_argument("--prefill-workload", choices=("configs2", "qkv"), default=None,
                   help="run one prefill projection ten times, eagerly, and exit (for rocprofv3 --pmc passes): "
                        "configs2 = M=2048 K=2048 N=8192 asym int4 g=128, qkv = M=2048 K=2048 N=2560 sym int4 g=32")
    p.add_argument("--pmc-workload", action="store_true",
                   help="run the HBM-traffic workload for rocprofv3 --pmc passes (a plain 256 MiB copy for calibration, "
                        "then every rotated decode projection twice, one launch each, no graphs) and exit")
    return p.parse_args()


def make_weight(torch, N_, dev, gen, M, K, N, g):
    """Synthetic asymmetric int4 weight in Kidi's layout on the device: uniform bytes (two uniform nibbles, codes
    -8..7), fp16 scales uniform in [0.002, 0.02], uint4 zero points uniform in [0, 15]."""
    values = torch.randint(0, 256, (N, K // 2), dtype=torch.uint8, device=dev, generator=gen)
    scales = (torch.rand((N, K // g), device=dev, generator=gen) * 0.018 + 0.002).to(torch.float16)
    zp = torch.randint(0, 16, (N, K // g), dtype=torch.uint8, device=dev, generator=gen)
    return values, scales, zp


def make_x(torch, dev, gen, M, K):
    x = torch.randn((M, K), device=dev, generator=gen)
    count = max(1, int(round(0.001 * M * K)))
    idx = torch.randperm(M * K, device=dev, generator=gen)[:count]
    x.view(-1)[idx] *= 20.0
    return x.to(torch.bfloat16)


class Projection:
    """One packed weight plus preallocated output and workspace, called through the raw C ABI."""

    def __init__(self, torch, N_, lib, values, scales, zp, K, g, M, x, dev):
        from kidi_amd.ops import DeviceWeight

        self.dw = DeviceWeight(values, scales, 4, g, zp)
        self.lib = lib
        self.y = torch.empty((M, values.shape[0]), dtype=torch.float32, device=dev)
        ws_bytes = lib.kq_linear_workspace_size(self.dw.handle, M)
        self.ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        a = N_.LinearArgs()
        a.x = x.data_ptr()
        a.x_dtype = N_.KQ_BF16
        a.m = M
        a.input_scale = 0.0
        a.output_scale = 0.0
        a.y = self.y.data_ptr()
        a.workspace = self.ws.data_ptr()
        a.workspace_bytes = ws_bytes
        self.args = a
        self.pargs = ctypes.byref(a)

    def __call__(self, stream):
        st = self.lib.kq_packed_linear(self.dw.handle, self.pargs, stream)
        if st != 0:
            raise RuntimeError(f"kq_packed_linear: {self.lib.kq_last_error().decode()}")


def capture(torch, calls, stream_ptr_fn):
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        s = stream_ptr_fn()
        for c in calls:
            c(s)
    return g


class Quiet:
    """Puts the device in a known state before a timed region: one launch that reads a 1 GiB buffer
    (kq_debug_read_floor: reads only, so no dirty lines are left to write back) evicts every weight of the timed steps
    from the 256 MB Infinity Cache, and its ~0.2 ms of device time lets the host enqueue the timed region behind it.
    Host submission latency therefore falls before the start event, and the events bracket device work only."""

    def __init__(self, torch, dev, lib):
        self.torch, self.lib = torch, lib
        self.buf = torch.ones((1 << 30,), dtype=torch.uint8, device=dev)
        self.sink = torch.zeros((1,), dtype=torch.int32, device=dev)

    def __call__(self):
        _ok(self.lib, self.lib.kq_debug_read_floor(self.buf.data_ptr(), self.buf.numel(), self.sink.data_ptr(),
                                                   self.torch.cuda.current_stream().cuda_stream))


def timed(torch, quiet, enqueue):
    """Device milliseconds of the work `enqueue()` issues on the current stream, measured with HIP events that are
    queued behind `quiet` (a read of a buffer four times the Infinity Cache), so the interval holds device work only."""
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    quiet()
    e0.record(stream)
    enqueue()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1)


def mfma_ceiling(torch, lib, dev, quiet, stream_ptr, iters=4096):
    """Sustained int8 MFMA rate of the whole chip (kq_debug_mfma_ceiling: one 8-wave workgroup per CU, two waves per
    SIMD, only v_mfma_i32_32x32x32_i8 in independent chains, ~1 ms per launch): TOP/s, its fraction of the published
    dense figure (2.4 GHz x 1024 SIMDs x 65,536 operations per 32-cycle MFMA), and the shader clock that rate implies
    at 32 cycles per MFMA and SIMD. (The waves' s_memtime counts are not used: that counter does not run at the
    shader clock on gfx950.)"""
    wgs = int(lib.kq_debug_mfma_ceiling_workgroups())
    cycles = torch.zeros((wgs * 8,), dtype=torch.int64, device=dev)
    sink = torch.zeros((wgs * 8,), dtype=torch.int32, device=dev)

    def run():
        _ok(lib, lib.kq_debug_mfma_ceiling(iters, cycles.data_ptr(), sink.data_ptr(), stream_ptr()))

    run()
    torch.cuda.synchronize()
    ms = min(timed(torch, quiet, run) for _ in range(3))
    ops = wgs * 8 * iters * 8 * 65536
    tops = ops / (ms * 1e-3) / 1e12
    return {"tops": round(tops, 1), "frac_of_peak": round(tops / INT8_PEAK_TOPS, 4),
            "implied_clock_ghz": round(tops * 1e12 / (wgs * 4 * 65536 / 32) / 1e9, 3),
            "us_per_launch": round(ms * 1e3, 1),
            "how": f"kq_debug_mfma_ceiling: {wgs} workgroups x 8 waves, {iters} x 8 independent 32x32x32 int8 MFMAs "
                   "per wave, nothing else; best of three launches"}


def run_steps(torch, projs, start, count, graph_full, graph_rem_fn, stream_ptr_fn):
    """Run `count` projections starting at rotation index `start` (a multiple of len(projs)): whole rotations as
    graph replays, the remainder as one graph of the first count % R projections."""
    R = len(projs)
    for _ in range(count // R):
        graph_full.replay()
    rem = count % R
    if rem:
        graph_rem_fn(rem).replay()


def check_decode_parity(torch, proj, values, scales, zp, x, g):
    """Output of the benchmarked projection against the CPU oracle: max|dy| <= 2e-3 max|y_ref|."""
    import numpy as np

    from oracle import kq_ref

    xb = x.float().cpu().numpy()
    y_ref, path = kq_ref.packed_linear(xb, values.cpu().numpy(), scales.cpu().numpy(), 4, g,
                                       zero_points=zp.cpu().numpy(), threads=8)
    y = proj.y.cpu().numpy()
    err = float(np.max(np.abs(y - y_ref)))
    scale = float(np.max(np.abs(y_ref)))
    return {"max_abs_err": err, "max_abs_ref": scale, "ok": bool(err <= 2e-3 * scale and path == kq_ref.PATH_BLOCKWISE)}


def cpu_baseline(torch, values, scales, zp, x, g, budget_s):
    """The oracle (build's C++ restatement of Kidi's CPU BlockwiseLinear path) on this host's cores: repeated
    M=1 projections of the same shape until the time budget is used (at least 3)."""
    import numpy as np

    from oracle import kq_ref

    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    threads = max(1, min(cores, 16))
    v, s, z = values.cpu().numpy(), scales.cpu().numpy(), zp.cpu().numpy()
    xb = x.float().cpu().numpy()
    kq_ref.packed_linear(xb, v, s, 4, g, zero_points=z, threads=threads)  # warm
    n = 0
    t0 = time.perf_counter()
    while True:
        kq_ref.packed_linear(xb, v, s, 4, g, zero_points=z, threads=threads)
        n += 1
        el = time.perf_counter() - t0
        if (el >= budget_s and n >= 3) or n >= 100000:
            break
    per = el / n
    bytes_ = gemv_bytes(M_DEC, K_DEC, N_DEC, g)
    # one thread as well, on a fifth of the budget (the scalar restatement's own rate)
    n1 = 0
    t1 = time.perf_counter()
    while True:
        kq_ref.packed_linear(xb, v, s, 4, g, zero_points=z, threads=1)
        n1 += 1
        el1 = time.perf_counter() - t1
        if (el1 >= budget_s / 5 and n1 >= 2) or n1 >= 100000:
            break
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "")
    except OSError:
        pass
    return {"value": round(bytes_ / per / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{n} projections M=1 K={K_DEC} N={N_DEC} int4 g={g} asym (one weight, cache-warm), "
                      f"{el:.1f} s, {per * 1e3:.2f} ms each, oracle/kq_ref.cpp with {threads} threads",
            "one_thread_value": round(bytes_ / (el1 / n1) / 1e9, 3), "cpu_model": model, "host_cores": cores,
            "label": "build restatement of the reference CPU path (the reference's ynnpack path cannot be built)"}


def floor_sweep(torch, lib, dev, gen, args):
    """Single-launch read floor of the configs[1] decode's bytes over launch geometries: per (threads per workgroup,
    16-byte loads per lane) the device time per launch of kq_debug_read_floor_shape over R rotated buffers, timed as
    `value` is (exactly --steps launches right behind the cache flush, median of five regions), and of an empty kernel
    of the same grid (graph-replayed, per launch)."""
    fb = -(-gemv_bytes(M_DEC, K_DEC, N_DEC, G_DEC) // 16) * 16
    R = args.rotate
    bufs = [torch.randint(0, 256, (fb,), dtype=torch.uint8, device=dev, generator=gen) for _ in range(R)]
    sink = torch.zeros((1,), dtype=torch.int32, device=dev)
    quiet = Quiet(torch, dev, lib)
    stream_ptr = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    print(f"read floor sweep: {fb} bytes per launch, {R} rotated buffers, {args.steps} launches per timed region")
    print("| threads | loads/lane | workgroups | waves | read us/launch | GB/s | % of 8 TB/s | empty us/launch |")
    print("|---|---|---|---|---|---|---|---|")
    for threads in (64, 128, 256, 512, 1024):
        for loads in (1, 2, 4, 8, 16):
            blocks = -(-fb // (16 * threads * loads))
            if blocks < 16:
                continue
            res = {}
            for empty in (0, 1):
                calls = [lambda st, b=b, e=empty: _ok(lib, lib.kq_debug_read_floor_shape(b.data_ptr(), fb, threads, loads, e,
                                                                                         sink.data_ptr(), st))
                         for b in bufs]
                for c in calls:
                    c(stream_ptr())
                torch.cuda.synchronize()
                g = capture(torch, calls, stream_ptr)
                g.replay()
                torch.cuda.synchronize()
                if empty:
                    res[empty] = timed(torch, quiet, lambda: [g.replay() for _ in range(10)]) * 1e3 / (10 * R)
                else:
                    rem = {}

                    def graph_rem(n):
                        if n not in rem:
                            rem[n] = capture(torch, calls[:n], stream_ptr)
                        return rem[n]

                    if args.steps % R:
                        graph_rem(args.steps % R)
                    reps = [timed(torch, quiet, lambda: run_steps(torch, calls, 0, args.steps, g, graph_rem, stream_ptr))
                            for _ in range(5)]
                    res[empty] = sorted(reps)[2] * 1e3 / args.steps
                    del rem
                del g
            gbs = fb / (res[0] * 1e-6) / 1e9
            print(f"| {threads} | {loads} | {blocks} | {blocks * threads // 64} | {res[0]:.3f} | {gbs:.0f} | "
                  f"{100 * gbs / HBM_PEAK_GBS:.1f} | {res[1]:.3f} |", flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: --gpus {args.gpus} is not supported (this build has no multi-GPU "
              "path; the layer shards column- or row-wise with no exchange inside the projection)", file=sys.stderr)
        sys.exit(2)
    if args.rotate < 1 or args.steps < 1 or args.warmup < 0:
        sys.exit("bad --rotate/--steps/--warmup")

    import torch

    from kidi_amd import _native as N_

    lib = N_.load()
    if not torch.cuda.is_available():
        sys.exit("bench.py needs a GPU")
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    stream_ptr = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    if args.floor_sweep:
        floor_sweep(torch, lib, dev, gen, args)
        return
    if args.prefill_workload:
        N = N_PRE if args.prefill_workload == "configs2" else 2560
        g = G_PRE if args.prefill_workload == "configs2" else 32
        values = torch.randint(0, 256, (N, K_PRE // 2), dtype=torch.uint8, device=dev, generator=gen)
        scales = (torch.rand((N, K_PRE // g), device=dev, generator=gen) * 0.018 + 0.002).to(torch.float16)
        zp = torch.randint(0, 16, (N, K_PRE // g), dtype=torch.uint8, device=dev, generator=gen) \
            if args.prefill_workload == "configs2" else None
        proj = Projection(torch, N_, lib, values, scales, zp, K_PRE, g, M_PRE, make_x(torch, dev, gen, M_PRE, K_PRE), dev)
        for _ in range(10):
            proj(stream_ptr())
        torch.cuda.synchronize()
        print(f"prefill workload {args.prefill_workload} done", flush=True)
        return

    if args.pmc_workload:
        src = torch.rand((64 << 20,), device=dev, generator=gen)  # 256 MiB float32
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)  # calibration kernel: reads 256 MiB, writes 256 MiB
        torch.cuda.synchronize()
        del src, dst

    # ---------------- decode GEMV (value) ----------------
    x = make_x(torch, dev, gen, M_DEC, K_DEC)
    projs = []
    first = None
    for r in range(args.rotate):
        values, scales, zp = make_weight(torch, N_, dev, gen, M_DEC, K_DEC, N_DEC, G_DEC)
        projs.append(Projection(torch, N_, lib, values, scales, zp, K_DEC, G_DEC, M_DEC, x, dev))
        if r == 0:
            first = (values, scales, zp)
        else:
            del values, scales, zp
    torch.cuda.synchronize()
    R = len(projs)
    if args.pmc_workload:
        for _ in range(2):
            for p in projs:
                p(stream_ptr())
        torch.cuda.synchronize()
        print("pmc workload done", flush=True)
        return
    graph_full = capture(torch, projs, stream_ptr)
    rem_graphs = {}

    def graph_rem(n):
        if n not in rem_graphs:
            rem_graphs[n] = capture(torch, projs[:n], stream_ptr)
        return rem_graphs[n]

    if args.steps % R:
        graph_rem(args.steps % R)
    if args.warmup % R:
        graph_rem(args.warmup % R)
    # warmup
    run_steps(torch, projs, 0, args.warmup, graph_full, graph_rem, stream_ptr)
    torch.cuda.synchronize()
    parity = check_decode_parity(torch, projs[0], *first, x, G_DEC)

    # the timed region (exactly --steps projections) five times, each behind its own cache flush; the median is
    # reported (BASELINE.md's timing rule: median of >= 5 repetitions)
    quiet = Quiet(torch, dev, lib)
    t0 = time.perf_counter()
    reps_ms = [timed(torch, quiet, lambda: run_steps(torch, projs, 0, args.steps, graph_full, graph_rem, stream_ptr))
               for _ in range(5)]
    wall = (time.perf_counter() - t0) / 5
    dev_ms = sorted(reps_ms)[len(reps_ms) // 2]
    ms_per_step = dev_ms / args.steps
    bytes_step = gemv_bytes(M_DEC, K_DEC, N_DEC, G_DEC)
    value = bytes_step / (ms_per_step * 1e-3) / 1e9
    # The decode step is one kernel launch (kq_packed_linear -> decode_kernel: activation quantization fused), so
    # the per-launch device time over the timed region is the kernel's average launch duration including the gap
    # between back-to-back kernels on the stream.
    traffic = load_traffic()
    roofline = {"bound": "hbm", "achieved": round(value, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(value / HBM_PEAK_GBS, 4),
                "traffic": traffic["traffic_bytes_per_launch"] if traffic else None,
                "kernel": "decode_kernel<4,128> (fused activation quantization + int8 MFMA GEMV)",
                "bytes_per_launch": bytes_step, "us_per_launch": round(ms_per_step * 1e3, 3)}
    if traffic:
        roofline["traffic_source"] = traffic["source"]

    # MALL-resident figure (one weight, repeated): reported separately, never as HBM %
    g1 = capture(torch, [projs[0]] * 64, stream_ptr)
    g1.replay()
    torch.cuda.synchronize()
    g1.replay()  # the one weight back in cache after the flush that precedes the timed region
    mall_ms = timed(torch, lambda: (quiet(), g1.replay()), lambda: [g1.replay() for _ in range(20)]) / (20 * 64)
    del g1

    # Read floor of one launch at this size: kq_debug_read_floor only reads the same number of bytes once (launch
    # shape and argument preloading of the decode kernel), over R rotated buffers, graph-replayed like the decode
    # steps. It bounds what any single-launch kernel of this size can reach (launch, ramp and HBM latency
    # included); reported beside the roofline.
    fb = -(-bytes_step // 16) * 16
    bufs = [torch.randint(0, 256, (fb,), dtype=torch.uint8, device=dev, generator=gen) for _ in range(R)]
    sink = torch.zeros((1,), dtype=torch.int32, device=dev)
    floor_calls = [lambda s, b=b: _ok(lib, lib.kq_debug_read_floor(b.data_ptr(), fb, sink.data_ptr(), s)) for b in bufs]
    for c in floor_calls:
        c(stream_ptr())
    torch.cuda.synchronize()
    gr = capture(torch, floor_calls, stream_ptr)
    for _ in range(3):
        gr.replay()
    torch.cuda.synchronize()
    floor_us = timed(torch, quiet, lambda: [gr.replay() for _ in range(20)]) * 1e3 / (20 * R)
    # ... and timed exactly as `value` is: --steps launches over the rotated buffers right behind the cache flush,
    # median of five regions
    floor_rem = {}

    def floor_graph_rem(n):
        if n not in floor_rem:
            floor_rem[n] = capture(torch, floor_calls[:n], stream_ptr)
        return floor_rem[n]

    if args.steps % R:
        floor_graph_rem(args.steps % R)
    floor_reps = [timed(torch, quiet, lambda: run_steps(torch, floor_calls, 0, args.steps, gr, floor_graph_rem, stream_ptr))
                  for _ in range(5)]
    floor_like_us = sorted(floor_reps)[2] * 1e3 / args.steps
    del gr, floor_rem, bufs, floor_calls

    del graph_full, rem_graphs
    first_cpu = tuple(t.cpu() for t in first)
    x_cpu = x.cpu()
    projs.clear()
    torch.cuda.empty_cache()

    # ---------------- prefill GEMM (reported beside value) ----------------
    vp, sp, zpp = make_weight(torch, N_, dev, gen, M_PRE, K_PRE, N_PRE, G_PRE)
    xp = make_x(torch, dev, gen, M_PRE, K_PRE)
    pre = Projection(torch, N_, lib, vp, sp, zpp, K_PRE, G_PRE, M_PRE, xp, dev)
    # a second weight of the same shape, so back-to-back calls alternate between two weights
    vp2, sp2, zpp2 = make_weight(torch, N_, dev, gen, M_PRE, K_PRE, N_PRE, G_PRE)
    pre2 = Projection(torch, N_, lib, vp2, sp2, zpp2, K_PRE, G_PRE, M_PRE, xp, dev)
    pre(stream_ptr())
    pre2(stream_ptr())
    torch.cuda.synchronize()
    # ten calls per graph (as a captured forward pass issues them), so the per-graph launch gap is amortized
    per_graph = 10
    gp = capture(torch, [pre, pre2] * (per_graph // 2), stream_ptr)
    for _ in range(2):
        gp.replay()
    torch.cuda.synchronize()
    replays = max(1, -(-args.prefill_steps // per_graph))
    pre_ms = timed(torch, quiet, lambda: [gp.replay() for _ in range(replays)]) / (replays * per_graph)
    pre_tops = 2.0 * M_PRE * N_PRE * K_PRE / (pre_ms * 1e-3) / 1e12
    # prefill parity on a sample of rows
    import numpy as np

    from oracle import kq_ref

    rows = np.array([0, 1, 777, M_PRE - 1])
    y_ref, _ = kq_ref.packed_linear(xp[rows].float().cpu().numpy(), vp.cpu().numpy(), sp.cpu().numpy(), 4, G_PRE,
                                    zero_points=zpp.cpu().numpy(), threads=8)
    y_pre = pre.y[torch.from_numpy(rows).to(dev)].cpu().numpy()
    pre_err = float(np.max(np.abs(y_pre - y_ref)))
    pre_ok = pre_err <= 2e-3 * float(np.max(np.abs(y_ref)))
    del gp, pre, pre2

    # ---------------- sustained int8 MFMA rate (the ceiling the prefill figure is read against) ----------------
    ceiling = mfma_ceiling(torch, lib, dev, quiet, stream_ptr)
    ceiling["prefill_vs_ceiling"] = round(pre_tops / ceiling["tops"], 4)

    # ---------------- CPU baseline ----------------
    cpu = None
    if args.cpu_seconds > 0:
        cpu = cpu_baseline(torch, *first_cpu, x_cpu, G_DEC, args.cpu_seconds)

    extras = None if args.no_extras else bench_extras(torch, N_, lib, dev, gen, quiet)

    out = {
        "metric": "int4 GEMV GB/s (% HBM peak) at M=1; prefill GEMM TOPS (% MFMA peak)",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded uniform int4 codes, fp16 scales, uint4 zero points; bf16 N(0,1) x, 0.1% x20)",
        "config": {"workload": "decode GEMV, asymmetric int4 g=128, M=1, K=2048, N=8192 (configs[1] up-proj)",
                   "rotated_weights": R,
                   "distinct_weights_timed": min(R, args.steps),
                   "weight_working_set_MB": round(min(R, args.steps) * projs_bytes(N_DEC, K_DEC, G_DEC) / 1e6, 1),
                   "launch": "HIP graph replay, one stream, queued behind a 1 GiB read that evicts the Infinity Cache"},
        "roofline": roofline,
        "wall_s": round(wall, 4),
        "ms_per_step_repeats": [round(v / args.steps, 6) for v in reps_ms],
        "parity": parity,
        "mall_resident_gbs": round(bytes_step / (mall_ms * 1e-3) / 1e9, 1),
        "read_floor": {"us_per_launch": round(floor_like_us, 3),
                       "gbs": round(bytes_step / (floor_like_us * 1e-6) / 1e9, 1),
                       "frac": round(bytes_step / (floor_like_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                       "how": "kq_debug_read_floor: one launch reading the same bytes once (the fastest geometry of "
                              "bench.py --floor-sweep), rotated buffers, HIP graph, timed exactly as value",
                       "decode_vs_floor": round(floor_like_us / (ms_per_step * 1e3), 4),
                       "steady_rotation_us": round(floor_us, 3)},
        "prefill": {"workload": "GEMM M=2048 K=2048 N=8192 asymmetric int4 g=128 (configs[2])",
                    "calls_per_graph": 10,
                    "ms": round(pre_ms, 5), "tops": round(pre_tops, 2),
                    "mfma_frac": round(pre_tops / INT8_PEAK_TOPS, 4), "parity_ok": bool(pre_ok),
                    "max_abs_err": pre_err},
        "mfma_ceiling": ceiling,
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(out), flush=True)


# ---------------------------------------------------------------------------------------------------------------
# Extras: configs[3] (decoder-layer projections) and configs[4] (mixed 2/4/8-bit stack, int8 output head), and the
# fused operators beside the plain projection. Each figure is the average device time per call over HIP-graph
# replays of R rotated weights whose combined size exceeds the 256 MB Infinity Cache.

def layer_bytes(M, K, N, g, bits, asym, out_cols=None):
    """Algorithmic bytes of one projection call: codes + fp16 scales [+ uint4 zero points] + bf16 x + fp32 y."""
    return N * K * bits // 8 + N * (K // g) * 2 + (N * (K // g) // 2 if asym else 0) + M * K * 2 + M * (out_cols or N) * 4


class Extras:
    def __init__(self, torch, N_, lib, dev, gen, quiet):
        self.torch, self.N_, self.lib, self.dev, self.gen, self.quiet = torch, N_, lib, dev, gen, quiet
        self.stream_ptr = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731

    def weight(self, N, K, bits, g, asym, code_bytes=None):
        from kidi_amd.ops import DeviceWeight

        t, dev, gen = self.torch, self.dev, self.gen
        values = t.randint(0, 256, (N, K * bits // 8), dtype=t.uint8, device=dev, generator=gen)
        scales = (t.rand((N, K // g), device=dev, generator=gen) * 0.018 + 0.002).to(t.float16)
        zp = t.randint(0, 16, (N, K // g), dtype=t.uint8, device=dev, generator=gen) if asym else None
        return DeviceWeight(values, scales, bits, g, zp)

    def weights(self, N, K, bits, g, asym, rotate=None):
        one = layer_bytes(0, K, N, g, bits, asym)
        R = rotate or max(1, min(64, -(-600_000_000 // one)))
        return [self.weight(N, K, bits, g, asym) for _ in range(R)]

    def x(self, M, K):
        return make_x(self.torch, self.dev, self.gen, M, K)

    def args(self, dw, x, M, y, input_scale=0.0, ws_bytes=None):
        t, N_ = self.torch, self.N_
        if ws_bytes is None:
            ws_bytes = self.lib.kq_linear_workspace_size(dw.handle, M)
        ws = t.empty(max(ws_bytes, 1), dtype=t.uint8, device=self.dev)
        a = N_.LinearArgs()
        a.x = x.data_ptr()
        a.x_dtype = N_.KQ_BF16
        a.m = M
        a.input_scale = input_scale
        a.output_scale = 0.0
        a.y = y.data_ptr() if y is not None else None
        a.workspace = ws.data_ptr()
        a.workspace_bytes = ws_bytes
        return a, ws

    def time_calls(self, calls, reps):
        """Average device time (us) per call of `calls`, replayed from one HIP graph `reps` times."""
        t = self.torch
        for c in calls:  # eager once: errors surface here, not inside the capture
            c(self.stream_ptr())
        t.cuda.synchronize()
        g = capture(t, calls, self.stream_ptr)
        g.replay()
        t.cuda.synchronize()
        return timed(t, self.quiet, lambda: [g.replay() for _ in range(reps)]) * 1e3 / (reps * len(calls))

    def linear_calls(self, dws, x, M, out_cols, fn="kq_packed_linear", input_scale=0.0):
        """Calls of `fn` over `dws`, plus `keep`: every tensor and argument block the calls point into. The caller
        must hold `keep` while the calls (or a graph of them) can run: torch.cuda.graph() empties the allocator
        cache on entry, so an output whose tensor was dropped would be unmapped under the replayed kernels."""
        t, lib = self.torch, self.lib
        calls = []
        y = t.empty((M, out_cols), dtype=t.float32, device=self.dev)
        keep = [x, y]
        for dw in dws:
            a, ws = self.args(dw, x, M, y, input_scale)
            keep += [a, ws]
            f = getattr(lib, fn)
            calls.append(lambda s, h=dw.handle, p=ctypes.byref(a), f=f: _ok(lib, f(h, p, s)))
        return calls, keep


def _ok(lib, status):
    if status != 0:
        raise RuntimeError(lib.kq_last_error().decode())


def bench_extras(torch, N_, lib, dev, gen, quiet):
    E = Extras(torch, N_, lib, dev, gen, quiet)
    out = {}
    # configs[0] (symmetric g = 32 up projection) on the GPU, configs[1]'s other decode shapes (M = 4; the down
    # projection K = 8192, N = 2048 at M = 1 and 4) and configs[2]'s M = 512 prefill
    shapes = {}
    for name, K, N, g, asym, M in (("c0_sym_g32_up_M1", 2048, 8192, 32, False, 1),
                                   ("c1_asym_g128_up_M4", 2048, 8192, 128, True, 4),
                                   ("c1_asym_g128_down_M1", 8192, 2048, 128, True, 1),
                                   ("c1_asym_g128_down_M4", 8192, 2048, 128, True, 4),
                                   ("c2_prefill_M512", 2048, 8192, 128, True, 512)):
        dws = E.weights(N, K, 4, g, asym, rotate=2 if M > 16 else None)
        x = E.x(M, K)
        calls, keep = E.linear_calls(dws, x, M, N)
        if M > 16:
            calls = calls * 5  # ten prefill calls per graph
        us = E.time_calls(calls, 20 if M <= 16 else 4)
        b = layer_bytes(M, K, N, g, 4, asym)
        ops = 2 * M * N * K
        shapes[name] = {"us": round(us, 3), "gbs": round(b / us / 1e3, 1), "tops": round(ops / us / 1e6, 1),
                        "rotated": len(dws)}
        del calls, keep, dws
    out["configs0_2_shapes"] = shapes
    torch.cuda.empty_cache()

    H, I, KV = 2048, 8192, 2048 + 256 + 256
    # decoder-layer projections, M = 1 (GB/s) and M = 2048 (TOP/s)
    qkv = E.weights(KV, H, 4, 32, False)
    gate_up = E.weights(2 * I, H, 4, 128, True)
    down = E.weights(H, I, 4, 128, True)
    layer = {}
    for M in (1, 2048):
        xh, xi = E.x(M, H), E.x(M, I)
        rows = {}
        for name, dws, x, K, N, g, asym, fn, cols in (
                ("qkv_g32", qkv, xh, H, KV, 32, False, "kq_packed_linear", KV),
                ("gate_up_gelu_g128", gate_up, xh, H, 2 * I, 128, True, "kq_packed_linear_gelu_gate", I),
                ("down_g128", down, xi, I, H, 128, True, "kq_packed_linear", H)):
            use = dws if M == 1 else dws[:2]
            calls, keep = E.linear_calls(use, x, M, cols, fn)
            if M > 1:
                calls = calls * 5  # ten prefill calls per graph
            us = E.time_calls(calls, 20 if M == 1 else 2)
            b = layer_bytes(M, K, N, g, 4, asym, cols)
            ops = 2 * M * N * K
            rows[name] = {"us": round(us, 3), "gbs": round(b / us / 1e3, 1), "tops": round(ops / us / 1e6, 1),
                          "rotated": len(use)}
            del calls, keep
        # the three projections of one layer back to back (rotating layers)
        if M == 1:
            calls, keep = [], []
            for i in range(len(down)):
                for dws, x, cols, fn in ((qkv, xh, KV, "kq_packed_linear"), (gate_up, xh, I, "kq_packed_linear_gelu_gate"),
                                         (down, xi, H, "kq_packed_linear")):
                    c, k = E.linear_calls([dws[i % len(dws)]], x, M, cols, fn)
                    calls += c
                    keep += k
            rows["layer_us"] = round(E.time_calls(calls, 5) * 3, 3)
            del calls, keep
        layer[f"M{M}"] = rows
    out["configs3_layer"] = layer

    # fused RMS normalization before the projection (kq_packed_linear_rms) against norm + projection, M = 1
    x1, r1 = E.x(1, H), E.x(1, H)
    wn = torch.rand(H, device=dev, generator=gen) + 0.5
    hidden = torch.empty((1, H), dtype=torch.float32, device=dev)
    normed = torch.empty((1, H), dtype=torch.float32, device=dev)
    y = torch.empty((1, I), dtype=torch.float32, device=dev)
    keep = []
    fused, composed = [], []
    for dw in gate_up:
        a, ws = E.args(dw, x1, 1, y, ws_bytes=lib.kq_rms_linear_workspace_size(dw.handle, 1))
        d = N_.NormDesc()
        d.weight, d.epsilon = wn.data_ptr(), 1e-6
        d.residual, d.residual_weight, d.residual_epsilon, d.hidden = r1.data_ptr(), wn.data_ptr(), 1e-6, hidden.data_ptr()
        keep += [a, ws, d]
        fused.append(lambda s, h=dw.handle, p=ctypes.byref(a), q=ctypes.byref(d):
                     _ok(lib, lib.kq_packed_linear_rms(h, p, q, 1, s)))
        ra = N_.RmsArgs()
        ra.x, ra.x_dtype, ra.rows, ra.width = x1.data_ptr(), N_.KQ_BF16, 1, H
        ra.weight, ra.residual, ra.epsilon, ra.y = wn.data_ptr(), r1.data_ptr(), 1e-6, hidden.data_ptr()
        rb = N_.RmsArgs()
        rb.x, rb.x_dtype, rb.rows, rb.width = hidden.data_ptr(), N_.KQ_F32, 1, H
        rb.weight, rb.epsilon, rb.y = wn.data_ptr(), 1e-6, normed.data_ptr()
        a2, ws2 = E.args(dw, normed, 1, y)
        a2.x_dtype = N_.KQ_F32
        keep += [ra, rb, a2, ws2]
        composed += [lambda s, p=ctypes.byref(ra): _ok(lib, lib.kq_rms_norm(p, s)),
                     lambda s, p=ctypes.byref(rb): _ok(lib, lib.kq_rms_norm(p, s)),
                     lambda s, h=dw.handle, p=ctypes.byref(a2): _ok(lib, lib.kq_packed_linear_gelu_gate(h, p, s))]
    out["rms_residual_gate_up_M1"] = {"fused_us": round(E.time_calls(fused, 20), 3),
                                      "composed_us": round(E.time_calls(composed, 20) * 3, 3),
                                      "composed": "kq_rms_norm (residual) + kq_rms_norm + kq_packed_linear_gelu_gate"}
    del fused, composed, keep, gate_up, qkv, down
    torch.cuda.empty_cache()

    # mixed 2/4/8-bit projections K = 2048, N = 8192 at M = 1; output head int8 g = 32, N = 262,144
    mixed = {}
    xm = E.x(1, 2048)
    for name, bits, g, asym, in_s in (("int2_g32_calibrated", 2, 32, False, 0.03), ("int4_g128_asym", 4, 128, True, 0.0),
                                      ("int8_g32_sym", 8, 32, False, 0.0)):
        dws = E.weights(8192, 2048, bits, g, asym)
        calls, keep = E.linear_calls(dws, xm, 1, 8192, input_scale=in_s)
        us = E.time_calls(calls, 20)
        b = layer_bytes(1, 2048, 8192, g, bits, asym)
        mixed[name] = {"us": round(us, 3), "gbs": round(b / us / 1e3, 1), "rotated": len(dws)}
        del calls, keep, dws
    head = E.weights(262144, 2048, 8, 32, False, rotate=2)
    for M in (1, 8):
        xh = E.x(M, 2048)
        calls, keep = E.linear_calls(head, xh, M, 262144)
        us = E.time_calls(calls, 10)
        b = layer_bytes(M, 2048, 262144, 32, 8, False)
        tok = torch.empty((M,), dtype=torch.int32, device=dev)
        keep += [xh, tok]
        gcalls = []
        for dw in head:
            a, ws = E.args(dw, xh, M, None, ws_bytes=lib.kq_greedy_linear_workspace_size(dw.handle, M))
            keep += [a, ws]
            gcalls.append(lambda s, h=dw.handle, p=ctypes.byref(a): _ok(lib, lib.kq_packed_linear_greedy(h, p, tok.data_ptr(), s)))
        gus = E.time_calls(gcalls, 10)
        mixed[f"head_int8_g32_M{M}"] = {"us": round(us, 3), "gbs": round(b / us / 1e3, 1),
                                        "greedy_us": round(gus, 3),
                                        "greedy_gbs": round((b - M * 262144 * 4) / gus / 1e3, 1)}
        del calls, gcalls, keep
    out["configs4_mixed"] = mixed
    del head
    torch.cuda.empty_cache()
    return out


def load_traffic():
    """HBM bytes per decode_kernel launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes over
    `bench.py --pmc-workload`, each scaled by what the counter reads for a plain copy of known size."""
    path = os.path.join(ROOT, "profiles", "decode_kernel_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        t = json.load(f)
    return {"traffic_bytes_per_launch": t["traffic_bytes_per_launch"],
            "source": f"profiles/decode_kernel_traffic.json (FETCH_SIZE x {t['fetch_factor']}, "
                      f"WRITE_SIZE x {t['write_factor']})"}


def projs_bytes(N, K, g):
    return N * K // 2 + N * (K // g) * 2 + N * (K // g) // 2


if __name__ == "__main__":
    main()
