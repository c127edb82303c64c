"""Float-input products (lab_gemm_q8 / lab_gemm_q4 mode 0) on the GPU: the
CPU's exact float order, so the outputs are bit-identical to the reference's
mode 0 (lab_native.c:489-501, :1013-1023) for any n."""

import glob
import os

import numpy as np
import pytest
import torch

from dianoia_amd import device as D
from dianoia_amd import synth
from gpu_util import bits, dev, host

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def gemv_float(fmt, qs, sc, xs, rows, cols, n):
    y = torch.full((n, rows), float("nan"), dtype=torch.float32, device="cuda")
    f = D.gemv_q4_float if fmt == "q4" else D.gemv_q8_float
    f(dev(qs), dev(sc), dev(xs), y, rows, cols, n)
    return host(y)


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "gemm_*.npz"))),
                         ids=lambda p: os.path.basename(p)[:-4])
def test_float_inputs_match_golden_mode0(gpu_ready, path):
    """The compiled reference's own mode-0 outputs (all tokens in one call)."""
    d = np.load(path)
    fmt = os.path.basename(path)[5:7]
    n = d["xs"].shape[0]
    rows = d["qs"].shape[0]
    cols = d["qs"].shape[1] * (2 if fmt == "q4" else 1)
    y = gemv_float(fmt, d["qs"], d["scales"], d["xs"], rows, cols, n)
    assert np.array_equal(bits(y), bits(d["y_mode0"]))


@pytest.mark.parametrize("fmt", ["q8", "q4"])
@pytest.mark.parametrize("rows,cols,n", [(1, 32, 1), (17, 64, 3), (3072, 1024, 1), (6144, 2048, 1),
                                         (2048, 6144, 2), (4097, 2048, 4), (70, 96, 13),
                                         (36, 64, 9), (128, 128, 40), (40000, 2048, 1),
                                         (300, 8192, 1), (1000, 4320, 5)])
def test_float_inputs_match_oracle(gpu_ready, orc, fmt, rows, cols, n):
    rng = np.random.default_rng(rows * 7 + cols + n)
    if fmt == "q8":
        qs, sc = synth.q8_weights(rng, rows, cols)
    else:
        qs, sc = synth.q4_weights(rng, rows, cols)
    xs = synth.activations(rng, n, cols)
    ref = (orc.gemm_q8 if fmt == "q8" else orc.gemm_q4)(qs, sc, xs, n, threads=8, mode=0)
    y = gemv_float(fmt, qs, sc, xs, rows, cols, n)
    assert np.array_equal(bits(y), bits(ref))


@pytest.mark.parametrize("fmt", ["q8", "q4"])
def test_float_inputs_reference_gpu_test_shapes(gpu_ready, orc, fmt):
    """The shapes and input range of the reference's own GPU linear test
    (test/gpu_linear_test.dart:26-45: values uniform in [-1, 1), compared to
    CPU mode 0 there at 1e-4 + 1e-5 |y|): here bit-exact."""
    rng = np.random.default_rng(5)
    for rows, cols, n in ((64, 64, 1), (70, 96, 13), (36, 64, 9), (128, 128, 40)):
        w = rng.uniform(-1, 1, size=(rows, cols)).astype(np.float32)
        if fmt == "q8":
            qs, sc = orc.quantize_q8(w)
        else:
            qs, sc = orc.quantize_q4(w)
        xs = rng.uniform(-1, 1, size=(n, cols)).astype(np.float32)
        ref = (orc.gemm_q8 if fmt == "q8" else orc.gemm_q4)(qs, sc, xs, n, threads=4, mode=0)
        y = gemv_float(fmt, qs, sc, xs, rows, cols, n)
        assert np.array_equal(bits(y), bits(ref)), (rows, cols, n)


def test_float_inputs_special_values(gpu_ready, orc):
    """Signed zeros, infinities and NaN in x follow the CPU's fma chain."""
    rng = np.random.default_rng(11)
    qs, sc = synth.q8_weights(rng, 64, 128)
    xs = synth.activations(rng, 3, 128)
    xs[0, 5] = np.inf
    xs[1, 40] = np.nan
    xs[2, :] = -0.0
    ref = orc.gemm_q8(qs, sc, xs, 3, threads=2, mode=0)
    y = gemv_float("q8", qs, sc, xs, 64, 128, 3)
    assert np.array_equal(bits(y), bits(ref))


def test_float_inputs_reject_bad_shapes(gpu_ready):
    z = torch.zeros(4096, dtype=torch.float32, device="cuda")
    with pytest.raises(RuntimeError):
        D.gemv_q8_float(z, z, z, z, 4, 48, 1)      # cols not a multiple of 32
    with pytest.raises(RuntimeError):
        D.gemv_q8_float(z, z, z, z, 4, 64, 0)      # no tokens
