"""Benchmark of the MI355X quantized linear layer (one GPU).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--quick]

Prints ONE JSON line. The headline (``value``) is the benchmark metric's
GEMV half at the shape its target is stated on: configuration 2, the Q8_0
LM head (151936 x 2048) at batch 1 with the greedy argmax fused. One step is
one dnx_gemv_q8h_argmax call: x quantized in the prologue, the GEMV, the
token. ``value`` = algorithmic bytes per step (weights at the GGUF Q8_0 size
of 34 B per 32, x read and y written as fp32) / time, with inputs resident
in HBM. Two 331 MB weight copies alternate, so the 256 MB Infinity Cache
cannot serve them. The other configurations (the Q4 MLP pair, the small Q8
GEMV, the prefill GEMM with its M = 1..256 sweep, BF16 -> Q8 + the vision
pair) are reported under ``configs``; the prefill GEMM gives the metric's
TOPS half.

Timed regions are GPU time: the K steps are captured into one HIP graph and
its replay is bracketed by HIP events on the launch stream (host-driven
launches from Python cost more than the small kernels; config 1 reports
that figure as ``eager_host_driven_ms_per_step``). ``roofline`` is for the
headline call: algorithmic bytes per call / its mean time. ``traffic`` comes
from rocprofv3 FETCH_SIZE / WRITE_SIZE runs committed under profiles/ (null
when absent). ``cpu_baseline`` times the reference's own CPU kernels
(oracle/_ref, built from src/c/lab_native.c) on this host, on the headline
workload and on config 3's GEMM, all cores and 1 thread, medians of 12 runs
(oracle/cpu_bench.py).
"""

from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, GB/s
I8_PEAK_TOPS = 5000.0       # MI355X dense int8 MFMA, TOPS
METRIC = "Q4_0/Q8_0 GEMV GB/s (% HBM peak) @batch 1; prefill GEMM TOPS (% i8 MFMA peak)"
ROTATE_BYTES = 600 << 20    # distinct weight bytes cycled per config (> 2 x MALL)
SETTLE_S = 0.05             # untimed graph replays before each timed one


def q4_bytes(rows, cols):
    return rows * cols // 32 * 18


def q8_bytes(rows, cols):
    return rows * cols // 32 * 34


def copies_for(nbytes):
    return max(2, -(-ROTATE_BYTES // nbytes))


class Timer:
    """Times launches on the GPU, not on the host: the K timed launches are
    captured once into a HIP graph (torch's capture, on the stream the
    launchers enqueue on) and the graph's replay is bracketed by HIP events
    on that stream. Eager launches from Python cost ~7 us of host time each,
    more than most of these kernels take on the GPU."""

    def __init__(self, torch):
        self.torch = torch

    def graph(self, fn, steps):
        torch = self.torch
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(steps):
                fn(i)
        return g

    def time(self, fn, steps, warmup):
        """Mean ms per step over `steps` steps replayed from one graph. Before
        the timed replay the graph is replayed untimed for SETTLE_S: the
        first ~20 ms of work after the GPU has idled run up to 10% slower
        (the config-2 step measured 58-63 us per step over its first 15
        replays, then 56.5-57 us)."""
        torch = self.torch
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        g = self.graph(fn, steps)
        t0 = time.perf_counter()
        while True:  # untimed warm replays
            g.replay()
            torch.cuda.synchronize()
            if time.perf_counter() - t0 >= SETTLE_S:
                break
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        g.replay()
        stop.record()
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / steps

    def kernel_means(self, launches, steps):
        """Mean duration of each launch kind: a graph of `steps` launches of
        that kernel alone, replayed between events."""
        return [self.time(fn, steps, 2) for fn in launches]

    def eager(self, fn, steps, warmup):
        """Host-driven launches (includes the host's launch cost)."""
        torch = self.torch
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for i in range(steps):
            fn(i)
        stop.record()
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / steps


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


# ------------------------------------------------------------------ configs

def bench_c1(torch, D, synth, timer, steps, warmup):
    """Config 1 as two launches: gate + up + SiLU glue in one pass over x,
    then the down GEMV (its prologue quantizes h)."""
    (gq, gs), (uq, us), (dq, ds), x = synth.config1()
    per_set = 2 * q4_bytes(6144, 2048) + q4_bytes(2048, 6144)
    copies = copies_for(per_set)
    sets = []
    for c in range(copies):
        sets.append(tuple(dev(torch, a) for a in (gq, gs, uq, us, dq, ds)))
    xd = dev(torch, x)
    h = torch.empty(6144, device="cuda")
    g = torch.empty(6144, device="cuda")
    u = torch.empty(6144, device="cuda")
    y = torch.empty(2048, device="cuda")

    def gate_up(i):
        s = sets[i % copies]
        D.gate_up_q4(s[0], s[1], s[2], s[3], xd, h, 6144, 2048, 1)

    def down(i):
        s = sets[i % copies]
        D.gemv_q4(s[4], s[5], h, y, 2048, 6144, 1)

    def step(i):
        gate_up(i)
        down(i)

    ms = timer.time(step, steps, warmup)
    algo = per_set + (2048 * 4) * 2 + 6144 * 4 + 2 * 6144 * 4 + 2048 * 4
    means = timer.kernel_means([gate_up, down], min(steps, 200))
    gu_bytes = 2 * q4_bytes(6144, 2048) + 2048 * 4 + 6144 * 4
    resident = timer.time(lambda i: step(0), steps, warmup)

    # The same step unfused (four launches), for comparison.
    def unfused(i):
        s = sets[i % copies]
        D.gemv_q4(s[0], s[1], xd, g, 6144, 2048, 1)
        D.gemv_q4(s[2], s[3], xd, u, 6144, 2048, 1)
        D.swiglu(g, u)
        D.gemv_q4(s[4], s[5], g, y, 2048, 6144, 1)

    unfused_ms = timer.time(unfused, steps, warmup)
    eager_ms = timer.eager(step, steps, warmup)
    return {
        "ms_per_step": ms, "bytes_per_step": algo, "gbps": algo / ms / 1e6,
        "weight_copies": copies,
        "kernel_ms": {"gate_up_silu_q4": means[0], "gemv_q4_down": means[1]},
        "gate_up_bytes_per_launch": gu_bytes, "gate_up_gbps": gu_bytes / means[0] / 1e6,
        "down_gbps": (q4_bytes(2048, 6144) + 6144 * 4 + 2048 * 4) / means[1] / 1e6,
        "resident_gbps": algo / resident / 1e6,
        "unfused_ms_per_step": unfused_ms, "unfused_gbps": algo / unfused_ms / 1e6,
        "eager_host_driven_ms_per_step": eager_ms,
    }


def bench_c0(torch, D, synth, timer, steps, warmup):
    qs, sc, x = synth.config0()
    nbytes = q8_bytes(3072, 1024)
    copies = copies_for(nbytes)
    ws = [(dev(torch, qs), dev(torch, sc)) for _ in range(copies)]
    xd = dev(torch, x)
    y = torch.empty(3072, device="cuda")

    def step(i):
        q, s = ws[i % copies]
        D.gemv_q8(q, s, xd, y, 3072, 1024, 1)

    ms = timer.time(step, steps, warmup)
    algo = nbytes + 1024 * 4 + 3072 * 4
    resident = timer.time(lambda i: step(0), steps, warmup)
    return {"ms": ms, "gbps": algo / ms / 1e6, "frac_hbm": algo / ms / 1e6 / HBM_PEAK_GBS,
            "resident_gbps": algo / resident / 1e6, "weight_copies": copies}


def bench_c2(torch, D, synth, timer, steps, warmup):
    """Config 2: the LM-head GEMV with the greedy argmax fused into it, on the
    GGUF Q8_0 blocks' own fp16 scales (34 B per 32 weights); the engine
    layout's fp32 scales (36 B per 32) are timed beside it."""
    qs, sc, x = synth.config2()
    copies = 2
    half = sc.astype(np.float16).view(np.uint16)
    ws = [(dev(torch, qs), dev(torch, half)) for _ in range(copies)]
    xd = dev(torch, x)
    y = torch.empty(151936, device="cuda")
    out = torch.empty(1, dtype=torch.int64, device="cuda")
    wsp = D.gemv_argmax_workspace()

    def step(i):
        q, s = ws[i % copies]
        D.gemv_q8h_argmax(q, s, xd, y, out, wsp, 151936, 2048)

    n = max(20, steps // 2)
    ms = timer.time(step, n, max(2, warmup // 2))
    algo = q8_bytes(151936, 2048) + 2048 * 4 + 151936 * 4
    resident = timer.time(lambda i: step(0), n, 2)
    ws = [(q, dev(torch, sc)) for q, _ in ws]

    def step32(i):
        q, s = ws[i % copies]
        D.gemv_q8_argmax(q, s, xd, y, out, wsp, 151936, 2048)

    ms32 = timer.time(step32, n, 2)
    return {"ms": ms, "steps": n, "bytes_per_step": algo, "gbps": algo / ms / 1e6,
            "frac_hbm": algo / ms / 1e6 / HBM_PEAK_GBS,
            "kernel": "gemv_q8h + fused argmax (fp16 block scales)", "weight_copies": copies,
            "resident_gbps": algo / resident / 1e6,
            "engine_fp32_scales_ms": ms32, "engine_fp32_scales_gbps": algo / ms32 / 1e6}


def bench_c3(torch, D, synth, timer, steps, warmup):
    qs, sc, xs = synth.config3()
    M, N, K = 512, 6144, 2048
    copies = 8
    ws = [(dev(torch, qs), dev(torch, sc)) for _ in range(copies)]
    xd = dev(torch, xs)
    xq = torch.empty((M, K), dtype=torch.int8, device="cuda")
    xsc = torch.empty((M, K // 32), dtype=torch.float32, device="cuda")
    y = torch.empty((M, N), device="cuda")

    def quant(i):
        D.quantize_q8(xd, xq, xsc, M, K, K)

    def gemm(i):
        q, s = ws[i % copies]
        D.gemm_q4(q, s, xq, xsc, y, N, K, M)

    # The fp16/bf16-MFMA GEMM on the activation panel, which the quantizer
    # writes directly (dnx_quantize_q8_panel).
    panel = torch.empty((D.gemm_panel_bytes(M, K),), dtype=torch.uint8, device="cuda")

    def quant_p(i):
        D.quantize_q8_panel(xd, panel, M, K)

    def gemm_p(i):
        q, s = ws[i % copies]
        D.gemm_q4_panel(q, s, panel, y, N, K, M)

    # The fp6 matrix-core GEMM (gfx950 scaled MFMA): the quantizer writes
    # the fp6 activation panel; the weights are read in the engine's Q4
    # layout, or from the fp6 prepack a load-time converter writes once.
    f6panel = torch.empty((D.f6_panel_bytes(M, K),), dtype=torch.uint8, device="cuda")
    packed = [torch.empty((D.q4_f6pack_bytes(N, K),), dtype=torch.uint8, device="cuda")
              for _ in range(copies)]
    for c in range(copies):
        D.pack_q4_f6(ws[c][0], ws[c][1], packed[c], N, K)

    def quant_f6(i):
        D.quantize_q8_f6panel(xd, f6panel, M, K)

    def gemm_f6(i):
        q, s = ws[i % copies]
        D.gemm_q4_f6(q, s, f6panel, y, N, K, M)

    def gemm_f6p(i):
        D.gemm_q4_f6p(packed[i % copies], f6panel, y, N, K, M)

    def prepack(i):
        D.pack_q4_f6(ws[i % copies][0], ws[i % copies][1], packed[i % copies], N, K)

    n = max(10, steps // 4)
    ms_i8 = timer.time(lambda i: (quant(i), gemm(i)), n, max(2, warmup // 4))
    ms_p = timer.time(lambda i: (quant_p(i), gemm_p(i)), n, max(2, warmup // 4))
    ms_f6 = timer.time(lambda i: (quant_f6(i), gemm_f6(i)), n, max(2, warmup // 4))
    ms_f6p = timer.time(lambda i: (quant_f6(i), gemm_f6p(i)), n, max(2, warmup // 4))
    means = timer.kernel_means([quant, gemm, quant_p, gemm_p, quant_f6, gemm_f6, gemm_f6p, prepack], n)
    ops = 2 * M * N * K
    paths = {
        "int8_mfma": {"ms": ms_i8, "gemm_ms": means[1], "quantize_ms": means[0],
                      "kernel": "quantize_q8 + gemm_kernel (int8 MFMA, scale MFMA, cvt + fma)"},
        "fp16_panel": {"ms": ms_p, "gemm_ms": means[3], "quantize_ms": means[2],
                       "kernel": "quantize_q8_panel + gemm_f16_kernel (fp16 MFMA, scale MFMA, fma)"},
        "fp6_engine_layout": {"ms": ms_f6, "gemm_ms": means[5], "quantize_ms": means[4],
                              "kernel": "quantize_f6_panel + gemm_f6_q4_kernel (fp6 scaled MFMA on "
                                        "Q4 qs/scales, scale MFMA, fma)"},
        "fp6_prepacked": {"ms": ms_f6p, "gemm_ms": means[6], "quantize_ms": means[4],
                          "kernel": "quantize_f6_panel + gemm_f6p_kernel (fp6 scaled MFMA on the "
                                    "load-time fp6 prepack, scale MFMA, fma)",
                          "prepack_ms_load_time": means[7]},
    }
    best = min(paths, key=lambda k: paths[k]["gemm_ms"])
    b = paths[best]
    out = {"ms": b["ms"], "tops": ops / b["ms"] / 1e9, "gemm_ms": b["gemm_ms"],
           "quantize_ms": b["quantize_ms"], "gemm_tops": ops / b["gemm_ms"] / 1e9,
           "gemm_frac_i8": ops / b["gemm_ms"] / 1e9 / I8_PEAK_TOPS, "gemm_path": best,
           "paths": {k: dict(v, gemm_tops=ops / v["gemm_ms"] / 1e9) for k, v in paths.items()}}
    out["issue_floor"] = c3_issue_floor(M, N, K)
    # M = 1..256 sweep on the ABI's route (lab_gpu_enc_matmul_q4): the GEMV
    # (exact order) up to 4 tokens; from 5 tokens (prefill chunks of up to
    # 64, the reference's prefill, lib/src/model.dart:91, and the batch
    # shapes of the kernels' other callers) the fp6 panel quantizer + the
    # chunk GEMM on the weights' prepack (made once, at first use). Beside
    # each: the int8-MFMA route's time (quantize + int8 GEMM), the route of
    # the device-pointer entry points, which keep no prepack.
    sweep = {}
    for m in (1, 2, 4, 8, 16, 32, 64, 128, 256):
        xm = xd[:m].contiguous()
        ym = torch.empty((m, N), device="cuda")
        xqm = torch.empty((m, K), dtype=torch.int8, device="cuda")
        xsm = torch.empty((m, K // 32), device="cuda")
        pm = torch.empty((D.f6_panel_bytes(m, K),), dtype=torch.uint8, device="cuda")

        def int8_route(i, xm=xm, ym=ym, m=m, xqm=xqm, xsm=xsm):
            D.quantize_q8(xm, xqm, xsm, m, K, K)
            D.gemm_q4(ws[i % copies][0], ws[i % copies][1], xqm, xsm, ym, N, K, m)

        def chunk_route(i, xm=xm, ym=ym, m=m, pm=pm):
            D.quantize_q8_f6panel(xm, pm, m, K)
            D.gemm_q4_f6s(packed[i % copies], pm, ym, N, K, m)

        # The GEMM alone, on a panel made before: what the route costs in a
        # prefill chunk through the ABI, where the norm, SwiGLU or attention
        # that produces x writes its panel (about 1 us more in that kernel).
        def chunk_gemm(i, ym=ym, m=m, pm=pm):
            D.gemm_q4_f6s(packed[i % copies], pm, ym, N, K, m)

        nbytes = q4_bytes(N, K) + m * K * 4 + m * N * 4
        if m <= 4:
            fn = lambda i, xm=xm, ym=ym, m=m: D.gemv_q4(ws[i % copies][0], ws[i % copies][1],  # noqa: E731
                                                        xm, ym, N, K, m)
            kernel, other = "gemv_q4", None
        else:
            fn, kernel = chunk_route, "quantize_f6panel + gemm_f6s (prepacked chunk GEMM)"
            other = ("int8_route_ms", int8_route)
        t = timer.time(fn, n, 3)
        sweep[str(m)] = {"ms": t, "gbps": nbytes / t / 1e6, "tops": 2 * m * N * K / t / 1e9,
                         "kernel": kernel}
        if other is not None:
            sweep[str(m)][other[0]] = timer.time(other[1], n, 3)
            sweep[str(m)]["gemm_on_producer_panel_ms"] = timer.time(chunk_gemm, n, 3)
    out["sweep_m"] = sweep
    return out


def issue_bound(iters=3000, ctas=256):
    """The prefill GEMM's inner step run from registers only
    (libdnx_ubench.so, csrc/ubench_tile.hip): ns per step per SIMD for each
    mix of the step's instructions, with one and two waves per SIMD. A step
    is one 32x32 tile of one Q4 block: the f16 scale MFMA (mask bit 0), the
    fp6 scaled dot MFMA (bit 1) and `nvalu` fmas."""
    import ctypes
    import torch
    lib = ctypes.CDLL(os.path.join(ROOT, "dianoia_amd", "libdnx_ubench.so"))
    lib.dnx_ubench_tile_issue.argtypes = [ctypes.c_int] * 5 + [ctypes.c_void_p, ctypes.c_void_p]
    out = torch.zeros(ctas * 512, device="cuda")
    ms = ctypes.c_float()
    rows = {}
    for mask, label in ((3, "scale MFMA + dot MFMA"), (2, "dot MFMA"), (1, "scale MFMA"),
                        (0, "VALU only")):
        for nv in (0, 8, 16, 24, 32):
            if mask == 0 and nv == 0:
                continue
            row = {}
            for threads in (256, 512):
                waves = threads // 256
                rc = lib.dnx_ubench_tile_issue(nv, mask, 100, ctas, threads, out.data_ptr(),
                                               ctypes.byref(ms))
                rc = rc or lib.dnx_ubench_tile_issue(nv, mask, iters, ctas, threads,
                                                     out.data_ptr(), ctypes.byref(ms))
                if rc != 0:
                    raise RuntimeError(f"dnx_ubench_tile_issue returned {rc}")
                # ctas workgroups on 256 CUs x 4 SIMDs: `waves` waves per SIMD,
                # each doing iters x 3 steps.
                row[f"{waves}_wave"] = round(ms.value * 1e6 / (iters * 3 * waves), 2)
            rows[f"{label}, {nv} fma"] = row
    return {"unit": "ns per step per SIMD", "iters": iters, "workgroups": ctas, "steps": rows}


_ISSUE = {}


def c3_issue_floor(M, N, K):
    """The GEMM's compute floor from the measured step: tile-blocks per SIMD
    (32-token x 32-row x one-block steps over 1024 SIMDs) x the
    two-waves-per-SIMD time of the full step (both MFMAs + 16 fmas)."""
    if "t" not in _ISSUE:
        _ISSUE["t"] = issue_bound(iters=1500)
    t = _ISSUE["t"]["steps"]["scale MFMA + dot MFMA, 16 fma"]["2_wave"]
    steps_per_simd = (M // 32) * (N // 32) * (K // 32) / 1024
    floor_ms = steps_per_simd * t * 1e-6
    ops = 2 * M * N * K
    return {"step_ns": t, "steps_per_simd": steps_per_simd, "floor_ms": floor_ms,
            "floor_frac_i8": ops / floor_ms / 1e9 / I8_PEAK_TOPS,
            "note": "compute issue only: launch, prologue and the output store come on top"}


def bench_c4(torch, D, synth, timer, steps, warmup):
    fc1, fc2, x = synth.config4()
    M = 1024
    w1 = dev(torch, fc1)
    w2 = dev(torch, fc2)
    q1 = torch.zeros((4320, 1152), dtype=torch.int8, device="cuda")  # 16 zero rows of padding
    s1 = torch.zeros((4320, 36), device="cuda")
    q2 = torch.empty((1152, 4320), dtype=torch.int8, device="cuda")
    s2 = torch.empty((1152, 135), device="cuda")
    xd = dev(torch, x)
    xq = torch.empty((M, 4320), dtype=torch.int8, device="cuda")
    xs = torch.empty((M, 135), device="cuda")
    h = torch.empty((M, 4320), device="cuda")
    y = torch.empty((M, 1152), device="cuda")

    def quant_w(i):
        D.quantize_q8_bf16(w1, q1, s1, 4304, 1152, 1152)
        D.quantize_q8_bf16(w2, q2, s2, 1152, 4304, 4320)

    def fc1_(i):
        D.quantize_q8(xd, xq, xs, M, 1152, 1152)
        D.gemm_q8(q1, s1, xq, xs, h, 4320, 1152, M)

    def gelu_(i):
        D.gelu(h)

    def fc2_(i):
        D.quantize_q8(h, xq, xs, M, 4320, 4320)
        D.gemm_q8(q2, s2, xq, xs, y, 1152, 4320, M)

    # The same pair with float inputs (mode 0, the vision encoder's CPU
    # products, vision_encoder.dart:252-271): the bf16-MFMA float GEMM.
    def fc1f_(i):
        D.gemm_q8_float(q1, s1, xd, h, 4320, 1152, M)

    def fc2f_(i):
        D.gemm_q8_float(q2, s2, h, y, 1152, 4320, M)

    # The scaled-fp6 MFMA route: weights re-encoded once at load (two fp6
    # digits per int8, the scale's mantissa in two pieces), the activations
    # quantized straight into the fp6 panel.
    p1 = torch.empty(D.q8_f6pack_bytes(4320, 1152), dtype=torch.uint8, device="cuda")
    p2 = torch.empty(D.q8_f6pack_bytes(1152, 4320), dtype=torch.uint8, device="cuda")
    pan1 = torch.empty(D.f6_panel_bytes(M, 1152), dtype=torch.uint8, device="cuda")
    pan2 = torch.empty(D.f6_panel_bytes(M, 4320), dtype=torch.uint8, device="cuda")

    def pack_w(i):
        D.pack_q8_f6(q1, s1, p1, 4320, 1152)
        D.pack_q8_f6(q2, s2, p2, 1152, 4320)

    def fc1p_(i):
        D.quantize_q8_f6panel(xd, pan1, M, 1152)
        D.gemm_q8_f6p(p1, pan1, h, 4320, 1152, M)

    def fc2p_(i):
        D.quantize_q8_f6panel(h, pan2, M, 4320)
        D.gemm_q8_f6p(p2, pan2, y, 1152, 4320, M)

    # The int8-MFMA route on prepacked operands: weights re-encoded once at
    # load into fragment order, the activations quantized into the int8 panel.
    i1 = torch.empty(D.q8_i8pack_bytes(4320, 1152), dtype=torch.uint8, device="cuda")
    i2 = torch.empty(D.q8_i8pack_bytes(1152, 4320), dtype=torch.uint8, device="cuda")
    ipan1 = torch.empty(D.i8_panel_bytes(M, 1152), dtype=torch.uint8, device="cuda")
    ipan2 = torch.empty(D.i8_panel_bytes(M, 4320), dtype=torch.uint8, device="cuda")

    def pack_i(i):
        D.pack_q8_i8(q1, s1, i1, 4320, 1152)
        D.pack_q8_i8(q2, s2, i2, 1152, 4320)

    def fc1i_(i):
        D.quantize_q8_i8panel(xd, ipan1, M, 1152)
        D.gemm_q8_i8p(i1, ipan1, h, 4320, 1152, M)

    def fc2i_(i):
        D.quantize_q8_i8panel(h, ipan2, M, 4320)
        D.gemm_q8_i8p(i2, ipan2, y, 1152, 4320, M)

    def fc1i_gemm(i):
        D.gemm_q8_i8p(i1, ipan1, h, 4320, 1152, M)

    def fc2i_gemm(i):
        D.gemm_q8_i8p(i2, ipan2, y, 1152, 4320, M)

    n = max(10, steps // 4)
    quant_w(0)
    pack_w(0)
    pack_i(0)
    fc1i_(0)
    fc2i_(0)
    means = timer.kernel_means([quant_w, fc1_, gelu_, fc2_, fc1f_, fc2f_, pack_w, fc1p_, fc2p_,
                                pack_i, fc1i_, fc2i_, fc1i_gemm, fc2i_gemm], n)
    qbytes = (4304 * 1152 * 2 + 4320 * 1152 + 4320 * 36 * 4) + (1152 * 4304 * 2 + 1152 * 4320 + 1152 * 135 * 4)
    ops = 2 * M * 4304 * 1152
    # fc1_ms / fc2_ms: the route lab_gpu_enc_matmul_q8 takes at these shapes
    # (dnx::matmul_uses_i8p: the int8 panel quantizer + the int8 GEMM on the
    # weights' prepack, which the command buffer keeps per weight region).
    return {"quantize_weights_ms": means[0], "quantize_weights_gbps": qbytes / means[0] / 1e6,
            "fc1_ms": means[10], "fc1_tops": ops / means[10] / 1e9, "gelu_ms": means[2],
            "fc2_ms": means[11], "fc2_tops": ops / means[11] / 1e9,
            "pair_tops": 2 * ops / (means[10] + means[2] + means[11]) / 1e9,
            "route": "lab_gpu_enc_matmul_q8: quantize_i8_panel_kernel + gemm_i8p_kernel "
                     "(fc1: 128 x 160 tiles, fc2: 128 x 128 tiles in 3 K parts) on the "
                     "prepack",
            "int8_route": {"fc1_ms": means[1], "fc1_tops": ops / means[1] / 1e9,
                           "fc2_ms": means[3], "fc2_tops": ops / means[3] / 1e9,
                           "kernels": "quantize_kernel + gemm_kernel<Q8, 64, 64> (+ split-K "
                                      "reduce for fc2): dnx_matmul_q8, no prepack"},
            "fp6_route": {"pack_weights_ms": means[6],
                          "fc1_ms": means[7], "fc1_tops": ops / means[7] / 1e9,
                          "fc2_ms": means[8], "fc2_tops": ops / means[8] / 1e9,
                          "pair_tops": 2 * ops / (means[7] + means[2] + means[8]) / 1e9,
                          "kernels": "quantize_f6_panel4_kernel + gemm_f6p_kernel<3, Q8> "
                                     "(scaled fp6 MFMA)"},
            "i8_prepacked_route": {"pack_weights_ms": means[9],
                                   "fc1_ms": means[10], "fc1_tops": ops / means[10] / 1e9,
                                   "fc2_ms": means[11], "fc2_tops": ops / means[11] / 1e9,
                                   "fc1_gemm_ms": means[12], "fc2_gemm_ms": means[13],
                                   "pair_tops": 2 * ops / (means[10] + means[2] + means[11]) / 1e9,
                                   "tiles_rows_tokens": [D.gemm_q8_i8p_tile(4320, 1152, M),
                                                         D.gemm_q8_i8p_tile(1152, 4320, M)],
                                   "kernels": "quantize_i8_panel_kernel + gemm_i8p_kernel "
                                              "(int8 MFMA, bf16 scale MFMA, prepacked operands)"},
            "float_inputs": {"fc1_ms": means[4], "fc1_tops": ops / means[4] / 1e9,
                             "fc2_ms": means[5], "fc2_tops": ops / means[5] / 1e9,
                             "kernel": "gemm_float_kernel (x in three exact bf16 pieces, "
                                       "bf16 MFMA, fma with the row scale)"}}


def bench_callers(torch, D, synth, timer, steps):
    """The quantized products' other callers at their own shapes, on the
    product route (dnx_matmul_*, what lab_gpu_enc_matmul_* runs): the audio
    encoder's Q4 linears (hidden 768, FFN 1792, projector into 2048;
    audio_encoder.dart:197-205) at 1, 13 and 375 rows, and the vision
    encoder's Q8 attention projections (1024 x 1024) and projector
    (4096 -> 4096 -> 2048; vision_encoder.dart:252-316) at its patch and
    image-token counts; int8 inputs (the ABI's default), plus the float-input
    route at two vision shapes. Weights rotate over copies past the MALL."""
    rng = np.random.default_rng(9)
    cases = ([("audio_enc", "q4", r, c, n, True)
              for r, c in ((1792, 768), (768, 1792), (2304, 768), (768, 768), (2048, 768),
                           (2048, 2048)) for n in (1, 13, 375)] +
             [("vision", "q8", r, c, n, True)
              for r, c, n in ((1024, 1024, 1024), (1024, 1024, 4096), (4096, 4096, 256),
                              (4096, 4096, 1024), (2048, 4096, 256), (2048, 4096, 1024))] +
             [("vision", "q8", 1024, 1024, 1024, False), ("vision", "q8", 4096, 4096, 256, False)])
    out = {}
    reps = max(10, steps // 10)
    for who, fmt, rows, cols, n, int8 in cases:
        if fmt == "q4":
            q, sc = synth.q4_weights(rng, rows, cols)
            nbytes = q4_bytes(rows, cols)
            f = D.matmul_q4
        else:
            q, sc = synth.q8_weights(rng, rows, cols)
            nbytes = q8_bytes(rows, cols)
            f = D.matmul_q8
        copies = min(copies_for(nbytes), 256)
        q0, s0 = dev(torch, q), dev(torch, sc)
        ws = [(q0, s0)] + [(q0.clone(), s0.clone()) for _ in range(copies - 1)]
        x = dev(torch, synth.activations(rng, n, cols))
        y = torch.empty((n, rows), device="cuda")
        wsp = D.matmul_workspace(cols, n)

        def fn(i, ws=ws, x=x, y=y, wsp=wsp, f=f, rows=rows, cols=cols, n=n, int8=int8):
            w = ws[i % len(ws)]
            f(w[0], w[1], x, y, rows, cols, n, int8, wsp)

        ms = timer.time(fn, reps, 3)
        key = f"{who}_{fmt}_{rows}x{cols}_n{n}" + ("" if int8 else "_float_inputs")
        out[key] = {"ms": ms, "weight_gbps": nbytes / ms / 1e6,
                    "tops": 2 * n * rows * cols / ms / 1e9, "weight_copies": copies}
        if fmt == "q4" and int8 and n > 4:
            # The chunk GEMM on the weights' prepack, which the lab_gpu_*
            # command buffer keeps per weight region (its route for 5..512
            # tokens where the tiled fp6 route does not apply: every shape
            # here).
            packs = [torch.empty((D.q4_f6pack_bytes(rows, cols),), dtype=torch.uint8,
                                 device="cuda") for _ in range(len(ws))]
            for w, pk in zip(ws, packs):
                D.pack_q4_f6(w[0], w[1], pk, rows, cols)
            pnl = torch.empty((D.f6_panel_bytes(n, cols),), dtype=torch.uint8, device="cuda")

            def chunk(i, packs=packs, pnl=pnl, x=x, y=y, rows=rows, cols=cols, n=n):
                D.quantize_q8_f6panel(x, pnl, n, cols)
                D.gemm_q4_f6s(packs[i % len(packs)], pnl, y, rows, cols, n)

            cms = timer.time(chunk, reps, 3)
            out[key]["chunk_route_ms"] = cms

            # The GEMM alone on that panel (a producer-written panel in an
            # ABI prefill).
            def chunk_gemm(i, packs=packs, pnl=pnl, y=y, rows=rows, cols=cols, n=n):
                D.gemm_q4_f6s(packs[i % len(packs)], pnl, y, rows, cols, n)

            out[key]["gemm_on_producer_panel_ms"] = timer.time(chunk_gemm, reps, 3)
            if 5 <= n <= 512:
                out[key].update({"dnx_matmul_ms": ms, "ms": cms,
                                 "weight_gbps": nbytes / cms / 1e6,
                                 "tops": 2 * n * rows * cols / cms / 1e9,
                                 "route": "lab_gpu_enc_matmul_q4: quantize_f6panel + gemm_f6s "
                                          "(prepack)"})
            del packs
        if fmt == "q8" and int8 and n >= 128:
            # The int8 GEMM on prepacked operands (weights re-encoded once
            # into fragment order, x quantized into the int8 panel).
            packs = [torch.empty((D.q8_i8pack_bytes(rows, cols),), dtype=torch.uint8,
                                 device="cuda") for _ in range(len(ws))]
            for w, pk in zip(ws, packs):
                D.pack_q8_i8(w[0], w[1], pk, rows, cols)
            pnl = torch.empty((D.i8_panel_bytes(n, cols),), dtype=torch.uint8, device="cuda")

            def i8p(i, packs=packs, pnl=pnl, x=x, y=y, rows=rows, cols=cols, n=n):
                D.quantize_q8_i8panel(x, pnl, n, cols)
                D.gemm_q8_i8p(packs[i % len(packs)], pnl, y, rows, cols, n)

            def i8p_gemm(i, packs=packs, pnl=pnl, y=y, rows=rows, cols=cols, n=n):
                D.gemm_q8_i8p(packs[i % len(packs)], pnl, y, rows, cols, n)

            ims = timer.time(i8p, reps, 3)
            out[key]["i8p_route_ms"] = ims
            out[key]["i8p_gemm_ms"] = timer.time(i8p_gemm, reps, 3)
            out[key]["i8p_tile_rows_tokens"] = D.gemm_q8_i8p_tile(rows, cols, n)
            if n >= 256 and rows * cols * n >= 1 << 28:
                # The route lab_gpu_enc_matmul_q8 takes (dnx::matmul_uses_i8p).
                out[key].update({"dnx_matmul_ms": ms, "ms": ims,
                                 "weight_gbps": nbytes / ims / 1e6,
                                 "tops": 2 * n * rows * cols / ims / 1e9,
                                 "route": "lab_gpu_enc_matmul_q8: quantize_i8panel + gemm_i8p "
                                          "(prepack)"})
            del packs
        del ws
        torch.cuda.empty_cache()
    return out


def bench_layers(torch, D, timer, steps):
    """The decoder's other layer steps (lab_gpu_enc_* semantics): attention
    decode over a 4096-position cache (32 query heads, 8 KV heads, hd 128;
    HBM-bound on the cached keys and values), RMSNorm over a 4096 x 2048
    prefill block, causal prefill attention of 512 tokens (same heads;
    fp32 matrix cores) and the short convolution at 1 and 512 tokens.
    Inputs generated on the GPU."""
    gen = torch.Generator(device="cuda").manual_seed(6)
    heads, kv, hd, pos = 32, 8, 128, 4095
    q = torch.randn(heads * hd, device="cuda", generator=gen)
    keys = torch.randn((pos + 1, kv * hd), device="cuda", generator=gen)
    values = torch.randn((pos + 1, kv * hd), device="cuda", generator=gen)
    out = torch.empty(heads * hd, device="cuda")
    x = torch.randn((4096, 2048), device="cuda", generator=gen)
    w = torch.rand(2048, device="cuda", generator=gen)
    y = torch.empty_like(x)
    # Prefill: 512 tokens from position 0 over their own keys (causal).
    npre = 512
    qp = torch.randn(npre * heads * hd, device="cuda", generator=gen)
    outp = torch.empty(npre * heads * hd, device="cuda")

    def attn(i):
        D.attention(q, keys, values, None, out, pos, 1, heads, kv, hd, 0)

    def norm(i):
        D.rms_norm(x, w, y, 4096, 2048, 1e-5)

    def prefill(i):
        D.attention(qp, keys, values, None, outp, 0, npre, heads, kv, hd, 0)

    # The short convolution (LFM2 conv block: width 2048, 3 taps) at decode
    # (1 token) and prefill (512 tokens).
    cw, ck = 2048, 3
    bcx = torch.randn((npre, 3 * cw), device="cuda", generator=gen)
    cweight = torch.randn((cw, ck), device="cuda", generator=gen)
    chist = torch.randn((ck - 1, cw), device="cuda", generator=gen)
    cy = torch.empty((npre, cw), device="cuda")

    def conv1(i):
        D.short_conv(bcx, cweight, chist, cy, cw, ck, 1)

    def conv512(i):
        D.short_conv(bcx, cweight, chist, cy, cw, ck, npre)

    means = timer.kernel_means([attn, norm, prefill, conv1, conv512], max(10, steps // 4))
    attn_bytes = 2 * (pos + 1) * kv * hd * 4 + 2 * heads * hd * 4
    norm_bytes = 2 * 4096 * 2048 * 4 + 2048 * 4
    # q.k and p.v: 2 flops per multiply-add, hd each, per visible key.
    pre_flops = 4 * hd * heads * (npre * (npre + 1) // 2)
    # Conv: B, C, X read and y written once, the taps and two state rows.
    conv_bytes = npre * 4 * cw * 4 + cw * ck * 4 + 2 * (ck - 1) * cw * 4
    return {"attention_decode_4096_ms": means[0],
            "attention_decode_4096_gbps": attn_bytes / means[0] / 1e6,
            "rms_norm_4096x2048_ms": means[1],
            "rms_norm_4096x2048_gbps": norm_bytes / means[1] / 1e6,
            "attention_prefill_512_ms": means[2],
            "attention_prefill_512_tflops": pre_flops / means[2] / 1e9,
            "attention_prefill_512_frac_fp32_mfma": pre_flops / means[2] / 1e9 / 157.3,
            "short_conv_2048x3_decode_ms": means[3],
            "short_conv_2048x3_prefill_512_ms": means[4],
            "short_conv_2048x3_prefill_512_gbps": conv_bytes / means[4] / 1e6,
            "bytes": {"attention_decode_4096": attn_bytes, "rms_norm_4096x2048": norm_bytes,
                      "short_conv_prefill_512": conv_bytes},
            "flops": {"attention_prefill_512": pre_flops}}


def bench_loaders(torch, D, timer, steps):
    """The other load-time converters (beyond the north star's BF16 -> Q8):
    BF16 -> Q4 (lab_quantize_q4 after _widenBf16) on a 32768 x 4096 matrix
    (256 MiB of BF16), and the Q6_K -> Q8 adapter (dequantizeQ6K +
    lab_quantize_q8, gguf.dart:402-414) at the LM-head shape 151936 x 2048,
    and the GGUF Q8_0 split (splitQ8_0, gguf.dart:270-282) at that shape;
    the north star's BF16 -> Q8 quantizer (part 4) at 32768 x 4096 too.
    Inputs are generated on the GPU; the kernels are HBM-bound."""
    gen = torch.Generator(device="cuda").manual_seed(5)
    wbig = (torch.randn((32768, 4096), device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
    wbig = wbig.view(torch.int16)
    q4 = torch.empty((32768, 2048), dtype=torch.uint8, device="cuda")
    d4 = torch.empty((32768, 128), dtype=torch.int16, device="cuda")
    rows, cols = 151936, 2048
    # Q6_K blocks with random low/high bits and scales and a small positive d.
    blocks = torch.randint(0, 256, (rows * cols // 256, 210), dtype=torch.uint8, device="cuda",
                           generator=gen)
    d = (torch.rand(rows * cols // 256, device="cuda", generator=gen) * 0.004).to(torch.float16)
    blocks[:, 208:210] = d.view(torch.uint8).view(-1, 2)
    q8 = torch.empty((rows, cols), dtype=torch.int8, device="cuda")
    s8 = torch.empty((rows, cols // 32), device="cuda")
    # GGUF Q8_0 blocks of the same LM head, split on the GPU (splitQ8_0).
    count = rows * cols // 32
    gguf = torch.randint(0, 256, (count * 34,), dtype=torch.uint8, device="cuda", generator=gen)

    q8b = torch.empty((32768, 4096), dtype=torch.int8, device="cuda")
    s8b = torch.empty((32768, 128), device="cuda")

    def q4_(i):
        D.quantize_q4_bf16(wbig, q4, d4, 32768, 4096)

    def q8b_(i):
        D.quantize_q8_bf16(wbig, q8b, s8b, 32768, 4096, 4096)

    def q6k_(i):
        D.q6k_to_q8(blocks, q8, s8, rows, cols)

    def split_(i):
        D.split_q8_0(gguf, q8, s8, count)

    means = timer.kernel_means([q4_, q6k_, split_, q8b_], max(10, steps // 4))
    q4_bytes = 32768 * 4096 * 2 + 32768 * 2048 + 32768 * 128 * 2
    q8b_bytes = 32768 * 4096 * 2 + 32768 * 4096 + 32768 * 128 * 4
    q6k_bytes = rows * cols // 256 * 210 + rows * cols + rows * (cols // 32) * 4
    split_bytes = count * 34 + count * 36
    del wbig, blocks, gguf
    return {"bf16_to_q4_32768x4096_ms": means[0],
            "bf16_to_q4_32768x4096_gbps": q4_bytes / means[0] / 1e6,
            "q6k_to_q8_151936x2048_ms": means[1],
            "q6k_to_q8_151936x2048_gbps": q6k_bytes / means[1] / 1e6,
            "split_q8_0_151936x2048_ms": means[2],
            "split_q8_0_151936x2048_gbps": split_bytes / means[2] / 1e6,
            "bf16_to_q8_32768x4096_ms": means[3],
            "bf16_to_q8_32768x4096_gbps": q8b_bytes / means[3] / 1e6,
            "bytes": {"bf16_to_q4": q4_bytes, "q6k_to_q8": q6k_bytes,
                      "split_q8_0": split_bytes, "bf16_to_q8": q8b_bytes}}


def bench_cache_wrap(reps=3):
    """Weight loading from disk to HBM (gpu.dart:938-979): a 324 MiB
    LFM3Q8C1 cache (eight 6144 x 6144 Q8 matrices, written to a temporary
    file, so its pages are in the page cache) opened, mapped and placed in
    HBM by GpuLinear.wrap_cache (lab_gpu_wrap: one pageable host-to-device
    copy). Host wall-clock per wrap; PCIe-bound, not an HBM figure."""
    import tempfile
    from dianoia_amd.formats import QuantMatrix
    from dianoia_amd.gpu import GpuLinear
    from dianoia_amd.q8_cache import Q8Cache
    rows = cols = 6144
    m = QuantMatrix.q8(np.full((rows, cols), 3, np.int8),
                       np.full(rows * cols // 32, 0.5, np.float32))
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "lfm3-q8.cache")
        Q8Cache.write(path, "bench", {f"m{i}": m for i in range(8)})
        nbytes = os.path.getsize(path) - (1 << 20)
        times = []
        for _ in range(reps):
            cache = Q8Cache.open(path, "bench")
            g = GpuLinear.start()
            t0 = time.perf_counter()
            g.wrap_cache(cache)
            times.append(time.perf_counter() - t0)
            g.dispose()
            cache.close()
    best = min(times)
    return {"cache_bytes": nbytes, "wrap_ms": best * 1e3, "wrap_gbps": nbytes / best / 1e9,
            "reps": reps}


def bench_decode_step(steps=20, position=4095, child=False):
    """One decode step of a Qwen3-1.7B-shaped decoder (28 layers, random Q4
    body, Q8 LM head) through the lab_gpu_* ABI, encoded as GpuForward.forward
    does (dianoia_amd/forward.py, gpu.dart:1036-1239): host wall-clock per
    token (ctypes encoding + commit + wait), the command buffer's GPU time
    (lab_gpu_last_ms), and the PCIe bytes per token. The KV history is
    `position` rows of 8 KV heads x 128 (fp32, as the reference keeps it).
    With host-write tracking (the default) a step uploads the token's
    embedding and RoPE row; the same step with DIANOIA_GPU_TRACK_WRITES=0 (a
    child process: the switch is read at lab_gpu_init) uploads every region
    it reads, including the whole KV history."""
    from dianoia_amd import forward as F
    cfg = F.qwen3_1_7b()
    fwd = F.GpuForward(cfg, max_seq=position + 1, max_chunk=1, seed=11)
    rng = np.random.default_rng(12)
    try:
        emb = (rng.standard_normal(cfg.hidden) * 0.5).astype(np.float32)
        for _ in range(3):
            fwd.residual[:cfg.hidden] = emb
            fwd.forward(1, position)
        wall, gpu, ups, downs = [], [], [], []
        for _ in range(steps):
            u0, d0 = F.transfer_bytes()
            t0 = time.perf_counter()
            fwd.residual[:cfg.hidden] = emb
            fwd.forward(1, position)
            wall.append(time.perf_counter() - t0)
            gpu.append(fwd.last_ms())
            u1, d1 = F.transfer_bytes()
            ups.append(u1 - u0)
            downs.append(d1 - d0)
        token = int(np.argmax(fwd.logits))
    finally:
        fwd.dispose()
    weights = sum(b for b in (
        cfg.layers * (q4_bytes(cfg.heads * cfg.head_dim, cfg.hidden)
                      + 2 * q4_bytes(cfg.kv_dim, cfg.hidden)
                      + q4_bytes(cfg.hidden, cfg.heads * cfg.head_dim)
                      + 2 * q4_bytes(cfg.intermediate, cfg.hidden)
                      + q4_bytes(cfg.hidden, cfg.intermediate)),
        q8_bytes(cfg.vocab, cfg.hidden)))
    kv = cfg.layers * 2 * (position + 1) * cfg.kv_dim * 4
    out = {"model": "Qwen3-1.7B-shaped: 28 layers, hidden 2048, SwiGLU 6144, 16/8 heads of 128, "
                    "vocab 151936; random Q4 body, Q8 LM head",
           "position": position, "steps": steps,
           "tracking_writes": F.tracking_writes(),
           "wall_ms": float(np.median(wall)) * 1e3, "gpu_ms": float(np.median(gpu)),
           "up_bytes_per_token": int(np.median(ups)), "down_bytes_per_token": int(np.median(downs)),
           "weight_bytes": int(weights), "kv_bytes_read": int(kv),
           "gpu_gbps": (weights + kv) / float(np.median(gpu)) / 1e6, "token": token}
    if child:
        return out
    env = dict(os.environ, DIANOIA_GPU_TRACK_WRITES="0")
    r = subprocess.run([sys.executable, os.path.abspath(__file__), "--decode-child"], env=env,
                       capture_output=True, text=True, timeout=600)
    if r.returncode == 0:
        off = json.loads(r.stdout.strip().splitlines()[-1])
        out["tracking_off"] = {k: off[k] for k in ("tracking_writes", "wall_ms", "gpu_ms",
                                                   "up_bytes_per_token", "down_bytes_per_token",
                                                   "token")}
    else:
        out["tracking_off"] = {"error": r.stderr[-500:]}
    return out


def bench_prefill_chunk(reps=10, n=64, position=256):
    """Prefill chunks of the same Qwen3-1.7B-shaped decoder through the
    lab_gpu_* ABI: `n` tokens per forward pass (the reference prefills in
    chunks of up to 64, lib/src/model.dart:91) after `position` tokens of
    history; the command buffer's GPU time per chunk (lab_gpu_last_ms,
    median over `reps` chunks at growing positions), and tokens per second.
    The chunk's matmuls take the prepacked fp6 chunk GEMM, the q/k/v and
    gate/up matmuls of one x sharing its activation panel; attention is the
    matrix-core prefill kernel."""
    from dianoia_amd import forward as F
    cfg = F.qwen3_1_7b()
    fwd = F.GpuForward(cfg, max_seq=position + n * (reps + 2), max_chunk=n, seed=11)
    rng = np.random.default_rng(13)
    try:
        emb = (rng.standard_normal(n * cfg.hidden) * 0.5).astype(np.float32)
        for k in range(2):   # first uses: the weights' prepacks
            fwd.residual[:n * cfg.hidden] = emb
            fwd.forward(n, k * n)
        gpu, wall = [], []
        for k in range(reps):
            fwd.residual[:n * cfg.hidden] = emb
            t0 = time.perf_counter()
            fwd.forward(n, position + k * n)
            wall.append(time.perf_counter() - t0)
            gpu.append(fwd.last_ms())
    finally:
        fwd.dispose()
    g = float(np.median(gpu))
    return {"model": "Qwen3-1.7B-shaped (as decode_step_abi)", "tokens_per_chunk": n,
            "first_position": position, "chunks": reps, "gpu_ms": g,
            "wall_ms": float(np.median(wall)) * 1e3, "tokens_per_s_gpu": n / g * 1e3}


# ------------------------------------------------------------------ CPU

def cpu_baseline(runs):
    """The reference's CPU kernels on this host (oracle/cpu_bench.py in a
    child process, so that OMP_PROC_BIND=close and OMP_PLACES=cores reach
    its OpenMP runtime at start-up): lab_gemm_q8 mode 1 + argmaxToken over
    the config-2 LM head (the headline's workload; `value`), and
    lab_gemm_q4 mode 1 at config 3's M = 512 (the metric's TOPS half), each
    on every core this job may use and on 1 thread, median of `runs` runs
    after 2 warm-ups, built from the reference's src/c/lab_native.c."""
    import subprocess
    env = dict(os.environ, OMP_PROC_BIND="close", OMP_PLACES="cores")
    r = subprocess.run([sys.executable, "-m", "oracle.cpu_bench", "--runs", str(runs),
                        "--warmup", "2"], cwd=ROOT, env=env, capture_output=True, text=True,
                       timeout=600)
    if r.returncode != 0:
        raise RuntimeError(f"oracle.cpu_bench failed ({r.returncode}):\n{r.stderr[-2000:]}")
    d = json.loads(r.stdout.strip().splitlines()[-1])
    c2a, c21, c3a, c31 = d["c2_all"], d["c2_1"], d["c3_all"], d["c3_1"]
    return {"value": c2a["gbps"], "unit": "GB/s", "cores": d["threads"], "kind": d["kind"],
            "sample": f"config-2 LM-head step (lab_gemm_q8 mode 1 + argmaxToken, 2 rotated "
                      f"weight copies), median of {d['runs']} runs after {d['warmup']} warm-ups "
                      f"on {d['threads']} threads ({c2a['ms']:.3f} ms), "
                      f"{d['library']} built from the reference's src/c/lab_native.c",
            "ms_per_step": c2a["ms"],
            "host": {"nproc": d["nproc"], "affinity_cores": d["affinity_cores"],
                     "omp_num_threads": d["omp_num_threads"], "omp_proc_bind": d["omp_proc_bind"],
                     "omp_places": d["omp_places"],
                     "threads_rule": "every core in the affinity mask, capped by the job's "
                                     "OMP_NUM_THREADS share where set"},
            "single_thread": {"value": c21["gbps"], "unit": "GB/s", "cores": 1,
                              "ms_per_step": c21["ms"]},
            "c3_prefill_gemm_m512": {
                "unit": "TOPS", "ops": d["c3_ops"],
                "all_cores": {"value": c3a["tops"], "cores": c3a["threads"], "ms": c3a["ms"]},
                "single_thread": {"value": c31["tops"], "cores": 1, "ms": c31["ms"]}}}


def traffic_from_profiles():
    """HBM bytes per launch of the headline's dominant kernel, from the
    committed FETCH_SIZE / WRITE_SIZE summary (None when absent)."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic_pmc.json")
    if not os.path.exists(path):
        return None
    try:
        with open(path) as f:
            k = json.load(f)["kernels"]
        return (k["c2 LM head Q8 (fp16 scales) + argmax, 151936x2048"]["hbm_bytes_per_launch"] +
                k.get("c2 argmax finisher", {}).get("hbm_bytes_per_launch", 0))
    except (OSError, ValueError, KeyError):
        return None


PMC_COPY_BYTES = 1 << 30  # the calibration copy: reads and writes this many bytes
kArgmaxWordsBytes = 32 * 8  # the finisher reads 32 rank words
PMC_KERNELS = {  # kernel-name fragment -> (workload, algorithmic bytes per launch)
    "gemv_kernel<1, 2, 1, true, false, false, 4, false>": (
        "c1 gate+up Q4 pair, 6144x2048", 2 * q4_bytes(6144, 2048) + 2048 * 4 + 6144 * 4),
    "gemv_kernel<1, 1, 1, false, false, false, 8, false>": (
        "c1 down Q4, 2048x6144", q4_bytes(2048, 6144) + 6144 * 4 + 2048 * 4),
    "gemv_kernel<2, 8, 1, false, true, false, 4, false>": (
        "c2 LM head Q8 (fp16 scales) + argmax, 151936x2048",
        q8_bytes(151936, 2048) + 2048 * 4 + 151936 * 4),
    "argmax_finish_kernel": ("c2 argmax finisher", kArgmaxWordsBytes + 8),
    "gemm_kernel<true, 64, 64, 2, 4>": (
        "c3 Q4 GEMM M=512, 6144x2048", q4_bytes(6144, 2048) + 512 * 2048 + 512 * 64 * 4
        + 512 * 6144 * 4),
    "gemm_f16_kernel<true, 3>": (
        "c3 Q4 panel GEMM M=512, 6144x2048", q4_bytes(6144, 2048) + 512 * 2048 + 512 * 64 * 4
        + 512 * 6144 * 4),
    # The fp6 GEMM reads the prepacked weights (32 B per row and block) and
    # the codes and scales of the fp6 activation panel (2048 of its 2176 B
    # per 32 tokens and block).
    "gemm_f6p_kernel<3, false>": (
        "c3 Q4 fp6 GEMM (prepacked) M=512, 6144x2048", 6144 * 64 * 32 + 16 * 64 * 2048
        + 512 * 6144 * 4),
    "gemm_kernel<false, 64, 64, 2, 4>": (
        "c4 fc1 Q8 GEMM (int8 MFMA) M=1024, 4320x1152", q8_bytes(4320, 1152) + 4320 * 36 * 2
        + 1024 * 1152 + 1024 * 36 * 4 + 1024 * 4320 * 4),
    # Q8 prepack: 80 B per row and block.
    "gemm_f6p_kernel<3, true>": (
        "c4 fc1 Q8 fp6 GEMM (prepacked) M=1024, 4320x1152", 4320 * 36 * 80 + 32 * 36 * 2048
        + 1024 * 4320 * 4),
    "gemm_float_kernel<false, 4>": (
        "c4 fc1 float-input Q8 GEMM M=1024, 4320x1152", 4320 * 1152 + 4320 * 36 * 4
        + 1024 * 1152 * 4 + 1024 * 4320 * 4),
}


def pmc_workload(torch, D, synth, reps):
    """Eager launches for the rocprofv3 --pmc runs: a plain device copy of
    PMC_COPY_BYTES (the calibration of WRITE_SIZE) and a read-only stream
    over as many bytes (the calibration of FETCH_SIZE), then the config-1
    step, the config-2 LM head and the config-3 GEMM, each over rotating
    weight copies so that every launch reads its weights from HBM, config
    4's fc1 on its three GEMMs, then the causal prefill attention of 512
    tokens."""
    src = torch.empty(PMC_COPY_BYTES // 4, device="cuda")
    src.fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    del dst
    print("pmc: copy calibration done", file=sys.stderr, flush=True)
    # The read-only calibration: the GEMV's 16-byte streaming load over the
    # same PMC_COPY_BYTES (libdnx_ubench.so, dnx_ubench_stream_read).
    import ctypes
    ub = ctypes.CDLL(os.path.join(ROOT, "dianoia_amd", "libdnx_ubench.so"))
    ub.dnx_ubench_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                                          ctypes.c_void_p, ctypes.c_void_p]
    ctas = 2048
    words = torch.empty(ctas * 256, dtype=torch.int32, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for _ in range(reps):
        rc = ub.dnx_ubench_stream_read(src.data_ptr(), PMC_COPY_BYTES, ctas, words.data_ptr(),
                                       stream)
        if rc != 0:
            raise RuntimeError(f"dnx_ubench_stream_read returned {rc}")
    torch.cuda.synchronize()
    del src, words
    print("pmc: read calibration done", file=sys.stderr, flush=True)

    (gq, gs), (uq, us), (dq, ds), x = synth.config1()
    copies = copies_for(2 * q4_bytes(6144, 2048) + q4_bytes(2048, 6144))
    sets = [tuple(dev(torch, a) for a in (gq, gs, uq, us, dq, ds)) for _ in range(copies)]
    xd = dev(torch, x)
    h = torch.empty(6144, device="cuda")
    y = torch.empty(2048, device="cuda")
    for i in range(reps):
        s = sets[i % copies]
        D.gate_up_q4(s[0], s[1], s[2], s[3], xd, h, 6144, 2048, 1)
        D.gemv_q4(s[4], s[5], h, y, 2048, 6144, 1)
    torch.cuda.synchronize()
    del sets
    print("pmc: config 1 done", file=sys.stderr, flush=True)

    qs, sc, x = synth.config2()
    half = sc.astype(np.float16).view(np.uint16)
    ws = [(dev(torch, qs), dev(torch, half)) for _ in range(2)]
    xd = dev(torch, x)
    y = torch.empty(151936, device="cuda")
    out = torch.empty(1, dtype=torch.int64, device="cuda")
    wsp = D.gemv_argmax_workspace()
    for i in range(reps):
        q, s = ws[i % 2]
        D.gemv_q8h_argmax(q, s, xd, y, out, wsp, 151936, 2048)
    torch.cuda.synchronize()
    del ws
    print("pmc: config 2 done", file=sys.stderr, flush=True)

    qs, sc, xs = synth.config3()
    M, N, K = 512, 6144, 2048
    ws = [(dev(torch, qs), dev(torch, sc)) for _ in range(8)]
    xd = dev(torch, xs)
    xq = torch.empty((M, K), dtype=torch.int8, device="cuda")
    xsc = torch.empty((M, K // 32), dtype=torch.float32, device="cuda")
    y = torch.empty((M, N), device="cuda")
    D.quantize_q8(xd, xq, xsc, M, K, K)
    panel = torch.empty((D.gemm_panel_bytes(M, K),), dtype=torch.uint8, device="cuda")
    D.quantize_q8_panel(xd, panel, M, K)
    f6panel = torch.empty((D.f6_panel_bytes(M, K),), dtype=torch.uint8, device="cuda")
    D.quantize_q8_f6panel(xd, f6panel, M, K)
    packed = [torch.empty((D.q4_f6pack_bytes(N, K),), dtype=torch.uint8, device="cuda")
              for _ in range(8)]
    for c in range(8):
        D.pack_q4_f6(ws[c][0], ws[c][1], packed[c], N, K)
    for i in range(reps):
        q, s = ws[i % 8]
        D.gemm_q4(q, s, xq, xsc, y, N, K, M)
        D.gemm_q4_panel(q, s, panel, y, N, K, M)
        D.gemm_q4_f6p(packed[i % 8], f6panel, y, N, K, M)
    torch.cuda.synchronize()
    del ws, packed
    print("pmc: config 3 done", file=sys.stderr, flush=True)

    # Config 4's fc1 with float inputs (the bf16-MFMA float GEMM).
    fc1, _, x4 = synth.config4()
    w1 = dev(torch, fc1)
    q1 = torch.zeros((4320, 1152), dtype=torch.int8, device="cuda")
    s1 = torch.zeros((4320, 36), device="cuda")
    D.quantize_q8_bf16(w1, q1, s1, 4304, 1152, 1152)
    x4d = dev(torch, x4)
    h4 = torch.empty((1024, 4320), device="cuda")
    for i in range(reps):
        D.gemm_q8_float(q1, s1, x4d, h4, 4320, 1152, 1024)
    torch.cuda.synchronize()
    print("pmc: config 4 float done", file=sys.stderr, flush=True)
    # Config 4's fc1 on int8 inputs: the int8-MFMA GEMM and the Q8 fp6 GEMM.
    xq4 = torch.empty((1024, 1152), dtype=torch.int8, device="cuda")
    xs4 = torch.empty((1024, 36), device="cuda")
    D.quantize_q8(x4d, xq4, xs4, 1024, 1152, 1152)
    p1 = torch.empty(D.q8_f6pack_bytes(4320, 1152), dtype=torch.uint8, device="cuda")
    D.pack_q8_f6(q1, s1, p1, 4320, 1152)
    pan4 = torch.empty(D.f6_panel_bytes(1024, 1152), dtype=torch.uint8, device="cuda")
    D.quantize_q8_f6panel(x4d, pan4, 1024, 1152)
    for i in range(reps):
        D.gemm_q8(q1, s1, xq4, xs4, h4, 4320, 1152, 1024)
        D.gemm_q8_f6p(p1, pan4, h4, 4320, 1152, 1024)
    torch.cuda.synchronize()
    print("pmc: config 4 int8 inputs done", file=sys.stderr, flush=True)
    # The ABI's route for both projections: the int8 GEMM on prepacked
    # operands (fc1 on 160-row tiles, fc2 on 128-row tiles in three K parts).
    _, fc2, _ = synth.config4()
    w2 = dev(torch, fc2)
    q2 = torch.empty((1152, 4320), dtype=torch.int8, device="cuda")
    s2 = torch.empty((1152, 135), device="cuda")
    D.quantize_q8_bf16(w2, q2, s2, 1152, 4304, 4320)
    i1 = torch.empty(D.q8_i8pack_bytes(4320, 1152), dtype=torch.uint8, device="cuda")
    i2 = torch.empty(D.q8_i8pack_bytes(1152, 4320), dtype=torch.uint8, device="cuda")
    D.pack_q8_i8(q1, s1, i1, 4320, 1152)
    D.pack_q8_i8(q2, s2, i2, 1152, 4320)
    ip1 = torch.empty(D.i8_panel_bytes(1024, 1152), dtype=torch.uint8, device="cuda")
    ip2 = torch.empty(D.i8_panel_bytes(1024, 4320), dtype=torch.uint8, device="cuda")
    D.quantize_q8_i8panel(x4d, ip1, 1024, 1152)
    D.quantize_q8_i8panel(h4, ip2, 1024, 4320)
    y4 = torch.empty((1024, 1152), device="cuda")
    for i in range(reps):
        D.gemm_q8_i8p(i1, ip1, h4, 4320, 1152, 1024)
        D.gemm_q8_i8p(i2, ip2, y4, 1152, 4320, 1024)
    torch.cuda.synchronize()
    print("pmc: config 4 int8 prepacked route done", file=sys.stderr, flush=True)

    # Causal prefill attention, 512 tokens (the layer steps' matrix-core kernel).
    gen = torch.Generator(device="cuda").manual_seed(6)
    heads, kv, hd, n = 32, 8, 128, 512
    q = torch.randn(n * heads * hd, device="cuda", generator=gen)
    keys = torch.randn((n, kv * hd), device="cuda", generator=gen)
    values = torch.randn((n, kv * hd), device="cuda", generator=gen)
    out = torch.empty(n * heads * hd, device="cuda")
    for i in range(reps):
        D.attention(q, keys, values, None, out, 0, n, heads, kv, hd, 0)
    torch.cuda.synchronize()
    print("pmc: prefill attention done", file=sys.stderr, flush=True)


# Matrix-core kernels in the pmc workload -> (workload, ops per launch, peak
# TOPS of the MFMA type they run on).
MFMA_KERNELS = {
    "gemm_kernel<true, 64, 64, 2, 4>": ("c3 Q4 GEMM M=512 (int8 MFMA)", 2 * 512 * 6144 * 2048,
                                         I8_PEAK_TOPS),
    "gemm_f16_kernel<true, 3>": ("c3 Q4 GEMM M=512 (fp16 panel)", 2 * 512 * 6144 * 2048,
                                 I8_PEAK_TOPS),
    "gemm_f6p_kernel<3, false>": ("c3 Q4 GEMM M=512 (fp6, prepacked)", 2 * 512 * 6144 * 2048,
                                  I8_PEAK_TOPS),
    "gemm_kernel<false, 64, 64, 2, 4>": ("c4 fc1 Q8 GEMM M=1024 (int8 MFMA)",
                                         2 * 1024 * 4304 * 1152, I8_PEAK_TOPS),
    "gemm_f6p_kernel<3, true>": ("c4 fc1 Q8 GEMM M=1024 (fp6, prepacked)",
                                 2 * 1024 * 4304 * 1152, I8_PEAK_TOPS),
    "gemm_i8p_kernel<5, 4>": ("c4 fc1 Q8 GEMM M=1024 (int8 MFMA, prepacked: the ABI's route)",
                              2 * 1024 * 4304 * 1152, I8_PEAK_TOPS),
    "gemm_i8p_kernel<4, 4>": ("c4 fc2 Q8 GEMM M=1024 (int8 MFMA, prepacked, 3 K parts)",
                              2 * 1024 * 4304 * 1152, I8_PEAK_TOPS),
    "gemm_float_kernel<false, 4>": ("c4 fc1 float inputs M=1024 (bf16)",
                                    2 * 1024 * 4320 * 1152, 2500.0),
    "attention_prefill_kernel<128, 4>": ("prefill attention 512 tokens, 32/8 heads, hd 128",
                                         4 * 128 * 32 * (512 * 513 // 2), 157.3),
}
MFMA_COUNTERS = ("SQ_INSTS_MFMA", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU", "SQ_INSTS_LDS",
                 "SQ_LDS_BANK_CONFLICT", "SQ_WAIT_INST_LDS", "SQ_BUSY_CU_CYCLES", "SQ_WAVES")


def mfma_summary(csv_path, clock_ghz=2.4, simds=1024):
    """Matrix-core use per launch from one rocprofv3 counter run
    (MFMA_COUNTERS): mean counters and duration per dispatch of the
    MFMA_KERNELS, and the fraction of the GPU's SIMD-cycles the matrix
    cores were busy, SQ_VALU_MFMA_BUSY_CYCLES / (duration x clock x
    SIMDs), at the peak clock (so a lower bound when the clock drops)."""
    import csv
    per = {}
    with open(csv_path) as f:
        for r in csv.DictReader(f):
            name = r["Kernel_Name"]
            frag = next((k for k in MFMA_KERNELS if k in name), None)
            if frag is None:
                continue
            d = per.setdefault(frag, {"name": name, "dispatches": {}, "counters": {}})
            d["dispatches"][r["Dispatch_Id"]] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
            d["counters"].setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    out = {}
    for frag, d in per.items():
        workload, ops, peak = MFMA_KERNELS[frag]
        c = {k: sum(v) / len(v) for k, v in d["counters"].items()}
        ns = sum(d["dispatches"].values()) / len(d["dispatches"])
        busy = c.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0)
        out[workload] = {"kernel": d["name"], "launches": len(d["dispatches"]),
                         "duration_ns_under_counters": round(ns),
                         "counters_per_launch": {k: round(v) for k, v in c.items()},
                         "mfma_busy_frac": round(busy / (ns * 1e-9 * clock_ghz * 1e9 * simds), 4),
                         "ops_per_launch": ops,
                         "tops_under_counters": round(ops / ns / 1e3, 1),
                         "frac_of_peak_under_counters": round(ops / ns / 1e3 / peak, 4)}
    return {"clock_ghz_assumed": clock_ghz, "simds": simds, "kernels": out}


def _pmc_means(path, counter):
    """Mean value of `counter` per kernel name in a rocprofv3
    counter_collection.csv (one row per dispatch and counter)."""
    import csv
    sums, calls = {}, {}
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            if row.get("Counter_Name") != counter:
                continue
            name = row["Kernel_Name"]
            sums[name] = sums.get(name, 0.0) + float(row["Counter_Value"])
            calls[name] = calls.get(name, 0) + 1
    return {k: (sums[k] / calls[k], calls[k]) for k in sums}


def pmc_summary(fetch_csv, write_csv):
    """HBM bytes per launch of the kernels in PMC_KERNELS from a FETCH_SIZE
    run and a WRITE_SIZE run (KiB per dispatch). Reads are scaled by what
    FETCH_SIZE reads for the read-only streaming kernel over PMC_COPY_BYTES
    (the GEMV's own load), writes by what WRITE_SIZE reads for the copy of
    PMC_COPY_BYTES; the copy's FETCH_SIZE factor is reported beside."""
    fetch = _pmc_means(fetch_csv, "FETCH_SIZE")
    write = _pmc_means(write_csv, "WRITE_SIZE")

    def calib(table, frag):
        cands = [(v[0], k) for k, v in table.items() if frag in k.lower()]
        if not cands:
            raise SystemExit(f"no {frag} kernel in the counter run")
        kib, name = max(cands)
        return PMC_COPY_BYTES / (kib * 1024.0), name, kib

    ff, fname, fkib = calib(fetch, "stream_read")
    cf, _, ckib = calib(fetch, "copy")
    wf, wname, wkib = calib(write, "copy")
    kernels = {}
    for frag, (workload, algo) in PMC_KERNELS.items():
        fk = [(v, k) for k, v in fetch.items() if frag in k]
        wk = [(v, k) for k, v in write.items() if frag in k]
        if not fk or not wk:
            continue
        (fv, fc), name = fk[0]
        (wv, _), _ = wk[0]
        rd, wr = fv * 1024.0 * ff, wv * 1024.0 * wf
        kernels[workload] = {"kernel": name, "launches": fc, "fetch_kib": round(fv, 1),
                             "write_kib": round(wv, 1), "hbm_read_bytes": round(rd),
                             "hbm_write_bytes": round(wr), "hbm_bytes_per_launch": round(rd + wr),
                             "algorithmic_bytes": algo,
                             "traffic_over_algorithmic": round((rd + wr) / algo, 4)}
    return {"calibration": {"fetch_kernel": fname, "bytes": PMC_COPY_BYTES,
                            "fetch_kib": round(fkib, 1), "fetch_factor": round(ff, 5),
                            "write_kernel": wname, "write_kib": round(wkib, 1),
                            "write_factor": round(wf, 5),
                            "copy_fetch_kib": round(ckib, 1),
                            "copy_fetch_factor": round(cf, 5)},
            "kernels": kernels}


def check_graph_replay(torch, D, synth):
    """A graph replay gives the same bits as eager launches (checked once,
    on config 1's step, with eager work and syncs between replays)."""
    (gq, gs), (uq, us), (dq, ds), x = synth.config1()
    t = [dev(torch, a) for a in (gq, gs, uq, us, dq, ds)]
    xd = dev(torch, x)
    h = torch.empty(6144, device="cuda")
    y = torch.empty(2048, device="cuda")

    def step(i):
        D.gate_up_q4(t[0], t[1], t[2], t[3], xd, h, 6144, 2048, 1)
        D.gemv_q4(t[4], t[5], h, y, 2048, 6144, 1)

    step(0)
    torch.cuda.synchronize()
    want = y.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step(0)
    for _ in range(3):
        y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        if not torch.equal(y, want):
            raise RuntimeError("graph replay differs from eager launches")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-runs", type=int, default=12,
                    help="timed runs per CPU-baseline figure (median reported)")
    ap.add_argument("--quick", action="store_true", help="headline config only")
    ap.add_argument("--only", default=None,
                    help="comma-separated names of the other configs to run (default: all)")
    ap.add_argument("--pmc-workload", action="store_true",
                    help="eager launches for rocprofv3 --pmc runs (no JSON line)")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="HBM traffic per launch from two rocprofv3 counter_collection.csv files")
    ap.add_argument("--issue-bound", action="store_true",
                    help="the prefill GEMM step's issue-bound microbenchmark (JSON table)")
    ap.add_argument("--decode-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--mfma-summary", metavar="COUNTER_CSV",
                    help="matrix-core use per launch from a rocprofv3 counter_collection.csv "
                         "of the MFMA counters")
    args = ap.parse_args()
    if args.mfma_summary:
        print(json.dumps(mfma_summary(args.mfma_summary), indent=1))
        return
    if args.pmc_summary:
        print(json.dumps(pmc_summary(*args.pmc_summary), indent=1))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the quantized linear layer runs on one MI355X; sharding is design-only)",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from dianoia_amd import device as D
    from dianoia_amd import synth
    if not torch.cuda.is_available():
        print("bench.py needs the GPU", file=sys.stderr)
        sys.exit(1)
    if args.pmc_workload:
        pmc_workload(torch, D, synth, max(1, min(args.steps, 20)))
        return
    if args.issue_bound:
        print(json.dumps(issue_bound(), indent=1))
        return
    if args.decode_child:
        print(json.dumps(bench_decode_step(child=True)), flush=True)
        return
    timer = Timer(torch)
    check_graph_replay(torch, D, synth)
    print(f"bench: config 2 (steps={args.steps}, warmup={args.warmup})", file=sys.stderr, flush=True)
    c2 = bench_c2(torch, D, synth, timer, args.steps, args.warmup)
    configs = {"c2_q8_lmhead_argmax": c2}
    torch.cuda.empty_cache()
    if not args.quick:
        only = set(args.only.split(",")) if args.only else None
        for name, fn in (("c1_q4_mlp", bench_c1), ("c0_q8_gemv", bench_c0),
                         ("c3_q4_prefill_gemm", bench_c3), ("c4_vision_bf16_pair", bench_c4)):
            if only is not None and name not in only:
                continue
            print(f"bench: {name}", file=sys.stderr, flush=True)
            configs[name] = fn(torch, D, synth, timer, args.steps, args.warmup)
            torch.cuda.empty_cache()
        for name, fn in (("other_callers", lambda: bench_callers(torch, D, synth, timer, args.steps)),
                         ("load_time_converters", lambda: bench_loaders(torch, D, timer, args.steps)),
                         ("layer_steps", lambda: bench_layers(torch, D, timer, args.steps)),
                         ("decode_step_abi", bench_decode_step),
                         ("prefill_chunk_abi", bench_prefill_chunk),
                         ("weight_cache_wrap", bench_cache_wrap)):
            if only is not None and name not in only:
                continue
            print(f"bench: {name}", file=sys.stderr, flush=True)
            configs[name] = fn()
            torch.cuda.empty_cache()
    cpu = None
    if not args.no_cpu:
        print("bench: cpu baseline", file=sys.stderr, flush=True)
        cpu = cpu_baseline(args.cpu_runs)

    line = {
        "metric": METRIC,
        "value": round(c2["gbps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": c2["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(c2["ms"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded PCG64, seed 2: int8 uniform in [-127, 127], fp16 d = "
                "|N(0,1)|*0.01, x ~ N(0,1))",
        "config": {"workload": "c2_q8_lmhead_151936x2048_argmax_batch1", "batch": 1,
                   "rows": 151936, "cols": 2048, "weights": "Q8_0 (int8 + fp16 block scale)",
                   "greedy_argmax": "fused", "weight_copies": c2["weight_copies"],
                   "frac_hbm": round(c2["frac_hbm"], 4),
                   "resident_gbps_mall": round(c2["resident_gbps"], 2)},
        "roofline": {"bound": "hbm",
                     "kernel": "gemv_kernel<Q8 fp16-scale, 8-row tiles, argmax> + "
                               "argmax_finish_kernel (one dnx_gemv_q8h_argmax call)",
                     "achieved": round(c2["gbps"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(c2["gbps"] / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profiles(),
                     "bytes_per_launch": c2["bytes_per_step"],
                     "launch_ms": round(c2["ms"], 6)},
        "cpu_baseline": cpu,
        "configs": configs,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
