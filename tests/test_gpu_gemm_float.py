"""The float-input GEMM (lab_gemm_q8 / lab_gemm_q4 mode 0 for many tokens,
lab_native.c:489-501, :1013-1023) on bf16 MFMA: x split exactly into three
bf16 pieces, weights exact in bf16, so every product is exact and only the
summation order of each block's 32 products differs from the CPU's fma
chain (the per-block scaling runs in the CPU's order). Against the exact
products, error / sum|terms| < 1e-5 (the reference kernels' own bar,
native_kernels_test.dart:56-59, which the CPU kernels meet too); against the
CPU outputs, the reference GPU test's bar, 1e-4 + 1e-5 |cpu|
(gpu_linear_test.dart:44): unlike the int8 path, whose block dots are exact
integers, both the CPU and the GPU round every block's float sum, so outputs
near zero differ by the rounding of sums far larger than themselves."""

import numpy as np
import pytest
import torch

from dianoia_amd import device as D
from dianoia_amd import synth
from gpu_util import bits, dev, host

pytestmark = pytest.mark.gpu


def gemm_float(fmt, qs, sc, xs, rows, cols, n):
    y = torch.full((n, rows), float("nan"), dtype=torch.float32, device="cuda")
    f = D.gemm_q4_float if fmt == "q4" else D.gemm_q8_float
    f(dev(qs), dev(sc), dev(xs), y, rows, cols, n)
    return host(y)


def exact_mode0(fmt, qs, sc, xs):
    """sum_b sw * sum_k x w in float64, and sum_b |sw| sum_k |x w|."""
    rows = qs.shape[0]
    if fmt == "q4":
        lo = (qs & 15).astype(np.int64) - 8
        hi = (qs >> 4).astype(np.int64) - 8
        b = qs.shape[1] // 16
        w = np.concatenate([lo.reshape(rows, b, 16), hi.reshape(rows, b, 16)], axis=2)
        sw = sc.view(np.float16).astype(np.float64)
    else:
        b = qs.shape[1] // 32
        w = qs.astype(np.int64).reshape(rows, b, 32)
        sw = sc.astype(np.float64)
    x = xs.astype(np.float64).reshape(xs.shape[0], b, 32)
    w = w.astype(np.float64)
    y = np.zeros((xs.shape[0], rows))
    mag = np.zeros((xs.shape[0], rows))
    for j in range(b):
        y += (x[:, j, :] @ w[:, j, :].T) * sw[None, :, j]
        mag += (np.abs(x[:, j, :]) @ np.abs(w[:, j, :]).T) * np.abs(sw)[None, :, j]
    return y, mag


@pytest.mark.parametrize("fmt", ["q8", "q4"])
@pytest.mark.parametrize("rows,cols,n", [(4304, 1152, 1024), (1152, 4320, 1024), (1024, 1024, 1024),
                                         (768, 1792, 375), (70, 96, 13), (36, 64, 9),
                                         (128, 128, 40), (1, 32, 5), (97, 160, 129),
                                         (2048, 6144, 64), (300, 8192, 7)])
def test_float_gemm_within_tolerance(gpu_ready, orc, fmt, rows, cols, n):
    print(f"float gemm {fmt} {rows}x{cols} n={n}", flush=True)
    rng = np.random.default_rng(rows * 5 + cols + n)
    if fmt == "q8":
        qs, sc = synth.q8_weights(rng, rows, cols)
    else:
        qs, sc = synth.q4_weights(rng, rows, cols)
    xs = synth.activations(rng, n, cols)
    ref = (orc.gemm_q8 if fmt == "q8" else orc.gemm_q4)(qs, sc, xs, n, threads=8, mode=0)
    y = gemm_float(fmt, qs, sc, xs, rows, cols, n)
    exact, mag = exact_mode0(fmt, qs, sc, xs)
    mag = np.maximum(mag, 1e-30)
    assert np.max(np.abs(y - exact) / mag) < 1e-5
    assert np.max(np.abs(ref - exact) / mag) < 1e-5
    assert np.all(np.abs(y - ref) <= 1e-4 + 1e-5 * np.abs(ref))


def test_float_gemm_reference_gpu_test_shapes(gpu_ready, orc):
    """The reference's own GPU linear test (test/gpu_linear_test.dart:26-45):
    weights and inputs uniform in [-1, 1), within 1e-4 + 1e-5 |cpu| of CPU
    mode 0."""
    rng = np.random.default_rng(5)
    for fmt in ("q8", "q4"):
        for rows, cols, n in ((70, 96, 13), (36, 64, 9), (128, 128, 40)):
            w = rng.uniform(-1, 1, size=(rows, cols)).astype(np.float32)
            qs, sc = orc.quantize_q8(w) if fmt == "q8" else orc.quantize_q4(w)
            xs = rng.uniform(-1, 1, size=(n, cols)).astype(np.float32)
            ref = (orc.gemm_q8 if fmt == "q8" else orc.gemm_q4)(qs, sc, xs, n, threads=4, mode=0)
            y = gemm_float(fmt, qs, sc, xs, rows, cols, n)
            assert np.all(np.abs(y - ref) <= 1e-4 + 1e-5 * np.abs(ref)), (fmt, rows, cols, n)


def test_float_gemm_special_values(gpu_ready, orc):
    """An infinity in x gives the CPU's infinities (no NaN from splitting
    it), a NaN stays NaN, and an all-zero row gives zeros."""
    rng = np.random.default_rng(11)
    qs, sc = synth.q8_weights(rng, 64, 128)
    qs[:, 5] = 3  # row sign of inf * w is then +inf for every output of token 0
    xs = synth.activations(rng, 6, 128)
    xs[0, 5] = np.inf
    xs[1, 40] = np.nan
    xs[2, :] = 0.0
    ref = orc.gemm_q8(qs, sc, xs, 6, threads=2, mode=0)
    y = gemm_float("q8", qs, sc, xs, 64, 128, 6)
    assert np.array_equal(np.isposinf(y[0]), np.isposinf(ref[0])) and np.isposinf(y[0]).all()
    assert np.isnan(y[1]).all() and np.isnan(ref[1]).all()
    assert (y[2] == 0).all()
    assert np.all(np.abs(y[3:] - ref[3:]) <= 1e-4 + 1e-5 * np.abs(ref[3:]))


@pytest.mark.parametrize("rows,cols,n", [(1152, 4320, 1024), (64, 2048, 8), (4304, 1152, 300)])
def test_float_gemm_is_deterministic(gpu_ready, rows, cols, n):
    rng = np.random.default_rng(rows + n)
    qs, sc = synth.q4_weights(rng, rows, cols)
    xs = synth.activations(rng, n, cols)
    outs = [gemm_float("q4", qs, sc, xs, rows, cols, n) for _ in range(3)]
    assert all(np.array_equal(bits(o), bits(outs[0])) for o in outs[1:])


def test_float_gemm_rejects_unsupported(gpu_ready):
    z = torch.zeros(4096, device="cuda")
    with pytest.raises(RuntimeError):
        D.gemm_q8_float(z, z, z, z, 4, 48, 8)   # cols not a multiple of 32
    with pytest.raises(RuntimeError):
        D.gemm_q8_float(z, z, z, z, 4, 64, 0)   # no tokens
