"""Writes the golden vectors in tests/golden/ from the reference's own CPU kernels.

Runs in the build container, where oracle/Makefile has compiled the
reference's src/c/lab_native.c into oracle/_ref/liblab_native.so. Every
expected output below is computed by that library (lab_quantize_q8,
lab_quantize_q4, lab_gemm_q8, lab_gemm_q4), never by the repo's own oracle,
so the fixtures pin the oracle restatement and, through it, the GPU path.

    python tests/golden/make_golden.py

Inputs are seeded (numpy PCG64) and stored next to the outputs, so the
fixtures are self-contained data: nothing of the reference travels.
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402


def f32(*v):
    return np.array(v, dtype=np.float32)


def edge_rows() -> np.ndarray:
    """Rows of 64 values whose blocks hit the quantizer's edge cases."""
    rows = []
    z = np.zeros(32, np.float32)
    # all-zero block, and one of negative zeros
    rows.append(np.concatenate([z, -z]))
    # +-amax -> +-127; 0.49999997 with scale 1 rounds to 1 (not roundf's 0)
    b = np.zeros(32, np.float32)
    b[:6] = f32(127.0, -127.0, 0.49999997, -0.49999997, 2.5, -3.5)
    c = np.zeros(32, np.float32)
    c[:4] = f32(127.0, 63.5, -63.5, 0.5)
    rows.append(np.concatenate([b, c]))
    # tiny amax: 1/scale overflows to inf (x86 (int) gives INT_MIN -> -127)
    t = np.zeros(32, np.float32)
    t[:4] = f32(1e-38, -5e-39, 2e-39, 0.0)
    d = np.zeros(32, np.float32)
    d[:3] = f32(1e-45, -1e-45, 3e-45)  # denormals only
    rows.append(np.concatenate([t, d]))
    # large magnitudes, and one value per block dominating
    big = np.linspace(-1e30, 1e30, 32, dtype=np.float32)
    one = np.full(32, 1e-3, np.float32)
    one[7] = -1000.0
    rows.append(np.concatenate([big, one]))
    # values just around k + 0.5 after scaling by exactly 1
    h = (np.arange(32, dtype=np.float32) - 16.0) + np.float32(0.5)
    h[0] = 127.0
    h2 = np.nextafter(h, np.float32(0)).astype(np.float32)
    h2[0] = 127.0
    rows.append(np.concatenate([h, h2]))
    return np.stack(rows).astype(np.float32)


def q4_edge_rows() -> np.ndarray:
    """Rows of 64 values whose blocks hit lab_quantize_q4's edge cases."""
    rows = []
    z = np.zeros(32, np.float32)
    # all-zero block (max stays +0: d = -0, id = 0), and one of negative zeros
    rows.append(np.concatenate([z, -z]))
    # equal magnitudes of both signs: the first in column order sets d's sign
    a = np.zeros(32, np.float32)
    a[[2, 5, 20]] = f32(3.0, -3.0, 1.5)
    b = np.zeros(32, np.float32)
    b[[1, 17, 30]] = f32(-3.0, 3.0, -2.0)
    rows.append(np.concatenate([a, b]))
    # max = -8 gives d = 1, id = 1: x + 8.5 lands on k + 0.5 and just below
    h = (np.arange(32, dtype=np.float32) - 8.0) / np.float32(2.0)
    h[0] = -8.0
    h2 = np.nextafter(h, np.float32(-np.inf)).astype(np.float32)
    h2[0] = -8.0
    rows.append(np.concatenate([h, h2]))
    # NaN never wins; an infinite max gives d = -inf, id = -0 (inf * -0 is NaN)
    n = np.linspace(-1.0, 1.0, 32, dtype=np.float32)
    n[[0, 9]] = np.float32(np.nan)
    i = np.linspace(-2.0, 2.0, 32, dtype=np.float32)
    i[4] = np.float32(np.inf)
    i[6] = np.float32(np.nan)
    rows.append(np.concatenate([n, i]))
    # all-NaN block (max stays 0), and a fp16-overflowing scale (|d| > 65504)
    nn = np.full(32, np.nan, np.float32)
    big = np.linspace(-1e30, 6e29, 32, dtype=np.float32)
    rows.append(np.concatenate([nn, big]))
    # scales below fp16's range (subnormal and zero halves), fp32 denormals
    tiny = np.linspace(-3e-6, 2e-6, 32, dtype=np.float32)
    den = np.zeros(32, np.float32)
    den[:4] = f32(1e-45, -3e-45, 2e-44, -1e-40)
    rows.append(np.concatenate([tiny, den]))
    return np.stack(rows).astype(np.float32)


def main() -> None:
    ref = O.Reference()
    out = {}

    # ---- lab_quantize_q8: edges + seeded random rows of several magnitudes
    rng = np.random.default_rng(1234)
    edges = edge_rows()
    rand = rng.standard_normal((12, 256), dtype=np.float32)
    rand *= np.float32(10.0) ** rng.integers(-6, 7, size=(12, 1)).astype(np.float32)
    for name, x in (("edges", edges), ("random", rand)):
        qs, sc = ref.quantize_q8(x)
        np.savez_compressed(os.path.join(HERE, f"quantize_q8_{name}.npz"), x=x, qs=qs, scales=sc)

    # ---- lab_quantize_q4
    w = (rng.random((8, 256), dtype=np.float32) - np.float32(0.5)).astype(np.float32)
    w[0, :32] = 0.0
    w[1, 5] = -3.0
    qs4, sc4 = ref.quantize_q4(w)
    np.savez_compressed(os.path.join(HERE, "quantize_q4.npz"), x=w, qs=qs4, scales=sc4)
    e4 = q4_edge_rows()
    qs4, sc4 = ref.quantize_q4(e4)
    np.savez_compressed(os.path.join(HERE, "quantize_q4_edges.npz"), x=e4, qs=qs4, scales=sc4)

    # ---- lab_gemm_q8 / lab_gemm_q4, both modes, shapes from the reference's
    # tests (37 x 2048, n = 3 and 6) and from the benchmark widths.
    cases = [
        ("q8", 37, 2048, 3), ("q4", 37, 2048, 3), ("q8", 37, 2048, 6), ("q4", 37, 2048, 6),
        ("q8", 64, 1152, 5), ("q4", 16, 6144, 2), ("q8", 3, 32, 1), ("q4", 5, 64, 1),
    ]
    for i, (fmt, rows, cols, n) in enumerate(cases):
        g = np.random.default_rng(100 + i)
        wf = (g.random((rows, cols), dtype=np.float32) - np.float32(0.5)).astype(np.float32)
        xs = (g.random((n, cols), dtype=np.float32) * 2 - 1).astype(np.float32)
        if fmt == "q8":
            qs, sc = ref.quantize_q8(wf)
            y0 = ref.gemm_q8(qs, sc, xs, n, threads=2, mode=0)
            y1 = ref.gemm_q8(qs, sc, xs, n, threads=2, mode=1)
        else:
            qs, sc = ref.quantize_q4(wf)
            y0 = ref.gemm_q4(qs, sc, xs, n, threads=2, mode=0)
            y1 = ref.gemm_q4(qs, sc, xs, n, threads=2, mode=1)
        np.savez_compressed(os.path.join(HERE, f"gemm_{fmt}_{rows}x{cols}_n{n}.npz"),
                            qs=qs, scales=sc, xs=xs, y_mode0=y0, y_mode1=y1)
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
