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
    return {"value": round(bytes_ / per / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{n} projections M=1 K={K_DEC} N={N_DEC} int4 g={g} asym (one weight, cache-warm), "
                      f"{el:.1f} s, {per * 1e3:.2f} ms each, oracle/kq_ref.cpp with {threads} threads"}


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

    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    run_steps(torch, projs, 0, args.steps, graph_full, graph_rem, stream_ptr)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    dev_ms = e0.elapsed_time(e1)
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
    e0.record(stream)
    for _ in range(20):
        g1.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    mall_ms = e0.elapsed_time(e1) / (20 * 64)
    del g1

    del graph_full, rem_graphs
    first_cpu = tuple(t.cpu() for t in first)
    x_cpu = x.cpu()
    projs.clear()
    torch.cuda.empty_cache()

    # ---------------- prefill GEMM (reported beside value) ----------------
    vp, sp, zpp = make_weight(torch, N_, dev, gen, M_PRE, K_PRE, N_PRE, G_PRE)
    xp = make_x(torch, dev, gen, M_PRE, K_PRE)
    pre = Projection(torch, N_, lib, vp, sp, zpp, K_PRE, G_PRE, M_PRE, xp, dev)
    pre(stream_ptr())
    torch.cuda.synchronize()
    gp = capture(torch, [pre], stream_ptr)
    for _ in range(3):
        gp.replay()
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(args.prefill_steps):
        gp.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    pre_ms = e0.elapsed_time(e1) / args.prefill_steps
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
    del gp, pre

    # ---------------- CPU baseline ----------------
    cpu = None
    if args.cpu_seconds > 0:
        cpu = cpu_baseline(torch, *first_cpu, x_cpu, G_DEC, args.cpu_seconds)

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
                   "rotated_weights": R, "weight_working_set_MB": round(R * projs_bytes(N_DEC, K_DEC, G_DEC) / 1e6, 1),
                   "launch": "HIP graph replay, one stream"},
        "roofline": roofline,
        "wall_s": round(wall, 4),
        "parity": parity,
        "mall_resident_gbs": round(bytes_step / (mall_ms * 1e-3) / 1e9, 1),
        "prefill": {"workload": "GEMM M=2048 K=2048 N=8192 asymmetric int4 g=128 (configs[2])",
                    "ms": round(pre_ms, 5), "tops": round(pre_tops, 2),
                    "mfma_frac": round(pre_tops / INT8_PEAK_TOPS, 4), "parity_ok": bool(pre_ok),
                    "max_abs_err": pre_err},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


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
