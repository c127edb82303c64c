"""Decode GEMV (n <= 4) against lab_gemm_q8 / lab_gemm_q4 mode 1: bit-exact."""

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


def gemv(fmt, qs, sc, xs, rows, cols, n):
    y = torch.full((n, rows), float("nan"), dtype=torch.float32, device="cuda")
    f = D.gemv_q4 if fmt == "q4" else D.gemv_q8
    f(dev(qs), dev(sc), dev(xs), y, rows, cols, n)
    return host(y)


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "gemm_*.npz"))),
                         ids=lambda p: os.path.basename(p)[:-4])
def test_gemv_matches_golden(gpu_ready, path):
    d = np.load(path)
    fmt = os.path.basename(path)[5:7]
    n = d["xs"].shape[0]
    rows = d["qs"].shape[0]
    cols = d["qs"].shape[1] * (2 if fmt == "q4" else 1)
    for t0 in range(0, n, 4):
        t1 = min(n, t0 + 4)
        y = gemv(fmt, d["qs"], d["scales"], d["xs"][t0:t1], rows, cols, t1 - t0)
        assert np.array_equal(bits(y), bits(d["y_mode1"][t0:t1]))


@pytest.mark.parametrize("fmt", ["q8", "q4"])
@pytest.mark.parametrize("rows,cols,n", [(1, 32, 1), (17, 64, 1), (4097, 2048, 1), (3072, 1024, 1),
                                         (6144, 2048, 1), (2048, 6144, 1), (1000, 4320, 1),
                                         (513, 1152, 2), (33, 2048, 3), (130, 2048, 4),
                                         (70, 96, 4)])
def test_gemv_matches_oracle(gpu_ready, orc, fmt, rows, cols, n):
    rng = np.random.default_rng(rows * 31 + cols + n)
    if fmt == "q8":
        qs, sc = synth.q8_weights(rng, rows, cols)
    else:
        qs, sc = synth.q4_weights(rng, rows, cols)
    xs = synth.activations(rng, n, cols)
    ref = (orc.gemm_q8 if fmt == "q8" else orc.gemm_q4)(qs, sc, xs, n, threads=8, mode=1)
    y = gemv(fmt, qs, sc, xs, rows, cols, n)
    assert np.array_equal(bits(y), bits(ref))


def test_lm_head_and_argmax_config2(gpu_ready, orc):
    """Config 2: Q8 151936 x 2048 + greedy argmax, bit-exact logits and token."""
    qs, sc, x = synth.config2()
    ref = orc.gemm_q8(qs, sc, x, 1, threads=8, mode=1)[0]
    y = torch.empty(151936, dtype=torch.float32, device="cuda")
    D.gemv_q8(dev(qs), dev(sc), dev(x), y, 151936, 2048, 1)
    out = torch.empty(1, dtype=torch.int64, device="cuda")
    D.argmax(y, out, D.argmax_workspace(151936))
    logits = host(y)
    assert np.array_equal(bits(logits), bits(ref))
    assert int(host(out)[0]) == orc.argmax(ref)


@pytest.mark.parametrize("values,want", [
    ([1, 3, 3, 2], 1), ([-0.0, 0.0], 0), ([float("nan"), 5, 7], 0), ([1, float("nan"), 0.5], 0),
    ([1, float("nan"), 4], 2), ([-float("inf"), -1e38], 1), ([float("nan")] * 3, 0),
])
def test_argmax_edge_cases(gpu_ready, orc, values, want):
    v = np.array(values, np.float32)
    assert orc.argmax(v) == want
    out = torch.empty(1, dtype=torch.int64, device="cuda")
    D.argmax(dev(v), out, D.argmax_workspace(v.size))
    assert int(host(out)[0]) == want


def test_argmax_ties_far_apart(gpu_ready, orc):
    v = np.random.default_rng(3).standard_normal(1 << 20).astype(np.float32)
    v[[7, 400000, 1048575]] = 9.0
    out = torch.empty(1, dtype=torch.int64, device="cuda")
    D.argmax(dev(v), out, D.argmax_workspace(v.size))
    assert int(host(out)[0]) == 7 == orc.argmax(v)


def test_gemv_rejects_unsupported(gpu_ready):
    z = torch.zeros(4096, device="cuda")
    with pytest.raises(RuntimeError):
        D.gemv_q8(z, z, z, z, 4, 48, 1)   # cols not a multiple of 32
    with pytest.raises(RuntimeError):
        D.gemv_q8(z, z, z, z, 4, 64, 5)   # n above the GEMV's 4
