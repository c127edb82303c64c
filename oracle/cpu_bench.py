"""CPU baseline runs for bench.py's cpu_baseline leg. TEST INFRASTRUCTURE ONLY.

    python -m oracle.cpu_bench [--threads T] [--runs R] [--warmup W]

Times the reference's own CPU kernels (oracle/_ref/liblab_native.so, built
from src/c/lab_native.c; the scalar restatement when that is absent) on the
benchmark's seeded synthetic inputs and prints one JSON object:

* C2: lab_gemm_q8 mode 1 (src/c/lab_native.c:553-579: the single-threaded
  activation quantization, then the OpenMP row loop) over the 151936 x 2048
  LM head at batch 1, then argmaxToken (lib/src/sampler.dart:137-152, the
  oracle's C form), two weight copies alternating so the 331 MB matrix
  streams from DRAM;
* C3: lab_gemm_q4 mode 1 (:1059-1080) at M = 512, K = 2048, N = 6144;

each on T threads and on 1 thread, as the median of R runs after W
warm-ups. bench.py starts this in a child process with
OMP_PROC_BIND=close and OMP_PLACES=cores, so the OpenMP runtime reads them
at start-up.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

import numpy as np

# Taken before any OpenMP runtime loads: with OMP_PROC_BIND set, the runtime
# binds this (initial) thread to one core when it starts.
AFFINITY_CORES = len(os.sched_getaffinity(0))

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402


def _p(a):
    return ctypes.c_void_p(a.ctypes.data)


class Call:
    """One lab_gemm_* call with its buffers allocated once (the timed region
    is the C call alone)."""

    def __init__(self, lib, prefix, name, qs, scales, xs, rows, cols, n):
        self.f = getattr(lib, prefix + name)
        self.qs, self.scales = qs, scales
        self.xs = np.ascontiguousarray(xs, np.float32).reshape(n, cols)
        self.xq = np.zeros(n * cols, np.int8)
        self.xsc = np.zeros(n * cols // 32 + 1, np.float32)
        self.ys = np.zeros((n, rows), np.float32)
        self.rows, self.cols, self.n = rows, cols, n

    def __call__(self, threads, qs=None, scales=None):
        qs = self.qs if qs is None else qs
        scales = self.scales if scales is None else scales
        self.f(_p(qs), _p(scales), _p(self.xs), _p(self.xq), _p(self.xsc), _p(self.ys),
               self.rows, self.cols, self.n, threads, 1)
        return self.ys


def median_ms(fn, runs, warmup):
    for i in range(warmup):
        fn(i)
    ts = []
    for i in range(runs):
        t0 = time.perf_counter()
        fn(warmup + i)
        ts.append((time.perf_counter() - t0) * 1e3)
    return statistics.median(ts), ts


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--threads", type=int, default=0, help="0: every core this process may use")
    ap.add_argument("--runs", type=int, default=12)
    ap.add_argument("--warmup", type=int, default=2)
    args = ap.parse_args()

    from dianoia_amd import synth
    O.build()
    kind = "reference" if O.reference_available() else "port"
    kern = O.Reference() if kind == "reference" else O.get()
    lib, prefix = kern.lib, kern.prefix
    orc = O.get()
    cores = AFFINITY_CORES
    # The cores this job may use: every core in its affinity mask, capped by
    # OMP_NUM_THREADS where the host sets it (the GPU box's per-job CPU share).
    share = int(os.environ["OMP_NUM_THREADS"]) if os.environ.get("OMP_NUM_THREADS") else cores
    threads = args.threads or min(cores, share)

    out = {"kind": kind, "library": os.path.relpath(kern.path, ROOT), "nproc": os.cpu_count(),
           "affinity_cores": cores, "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
           "threads": threads,
           "omp_proc_bind": os.environ.get("OMP_PROC_BIND"),
           "omp_places": os.environ.get("OMP_PLACES"), "runs": args.runs,
           "warmup": args.warmup, "statistic": "median"}

    # C2: LM head + argmax, two weight copies alternating.
    qs, sc, x = synth.config2()
    rows, cols = qs.shape
    sets = [(qs, sc), (qs.copy(), sc.copy())]
    c2 = Call(lib, prefix, "gemm_q8", qs, sc, x, rows, cols, 1)
    c2_bytes = rows * cols // 32 * 34 + cols * 4 + rows * 4
    for t in (threads, 1):
        def step(i, t=t):
            q, s = sets[i % 2]
            return orc.argmax(c2(t, q, s)[0])
        ms, ts = median_ms(step, args.runs, args.warmup)
        out[f"c2_{'all' if t == threads else '1'}"] = {
            "threads": t, "ms": ms, "gbps": c2_bytes / ms / 1e6, "runs_ms": ts}
    del sets, c2

    # C3: the prefill GEMM's CPU kernel, M = 512.
    qs, sc, xs = synth.config3()
    rows, cols = qs.shape[0], qs.shape[1] * 2
    m = xs.size // cols
    c3 = Call(lib, prefix, "gemm_q4", qs, sc, xs, rows, cols, m)
    ops = 2 * m * rows * cols
    for t in (threads, 1):
        ms, ts = median_ms(lambda i, t=t: c3(t), args.runs, args.warmup)
        out[f"c3_{'all' if t == threads else '1'}"] = {
            "threads": t, "ms": ms, "tops": ops / ms / 1e9, "runs_ms": ts}
    out["c2_bytes"] = c2_bytes
    out["c3_ops"] = ops
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
