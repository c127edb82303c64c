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


def half_scales(sc):
    """fp32 scales that are fp16 values -> their fp16 bits (the Q8_0 d)."""
    h = sc.astype(np.float16)
    assert np.array_equal(h.astype(np.float32), sc)
    return h.view(np.uint16)


def gemv(fmt, qs, sc, xs, rows, cols, n):
    y = torch.full((n, rows), float("nan"), dtype=torch.float32, device="cuda")
    f = {"q4": D.gemv_q4, "q8": D.gemv_q8, "q8h": D.gemv_q8h}[fmt]
    if fmt == "q8h":
        sc = half_scales(sc)
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


@pytest.mark.parametrize("fmt", ["q8", "q4", "q8h"])
@pytest.mark.parametrize("rows,cols,n", [(1, 32, 1), (17, 64, 1), (4097, 2048, 1), (3072, 1024, 1),
                                         (6144, 2048, 1), (2048, 6144, 1), (1000, 4320, 1),
                                         (513, 1152, 2), (33, 2048, 3), (130, 2048, 4),
                                         (70, 96, 4), (40000, 2048, 1), (33000, 1024, 2),
                                         (9000, 4096, 4), (300, 16384, 1)])
def test_gemv_matches_oracle(gpu_ready, orc, fmt, rows, cols, n):
    rng = np.random.default_rng(rows * 31 + cols + n)
    if fmt == "q4":
        qs, sc = synth.q4_weights(rng, rows, cols)
    else:
        qs, sc = synth.q8_weights(rng, rows, cols)
    xs = synth.activations(rng, n, cols)
    ref = (orc.gemm_q4 if fmt == "q4" else orc.gemm_q8)(qs, sc, xs, n, threads=8, mode=1)
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
    # the fused LM head on the GGUF fp16 scales: same logits, same token
    y.fill_(float("nan"))
    out.fill_(-1)
    D.gemv_q8h_argmax(dev(qs), dev(half_scales(sc)), dev(x), y, out, D.gemv_argmax_workspace(),
                      151936, 2048)
    assert np.array_equal(bits(host(y)), bits(ref))
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


@pytest.mark.parametrize("fmt", ["q8", "q4", "q8h"])
@pytest.mark.parametrize("rows,cols", [(151936, 2048), (1000, 1024), (7, 64), (50000, 4320),
                                       (1100000, 32)])
def test_fused_argmax_gemv(gpu_ready, orc, fmt, rows, cols):
    """GEMV + argmax (the GEMV, then a one-wave finisher): logits bit-exact,
    token = argmaxToken; the workspace is reused across calls (each call
    leaves it zero)."""
    rng = np.random.default_rng(rows + cols)
    if fmt == "q4":
        qs, sc = synth.q4_weights(rng, rows, cols)
    else:
        qs, sc = synth.q8_weights(rng, rows, cols)
    dq, ds = dev(qs), dev(half_scales(sc) if fmt == "q8h" else sc)
    ws = D.gemv_argmax_workspace()
    f = {"q4": D.gemv_q4_argmax, "q8": D.gemv_q8_argmax, "q8h": D.gemv_q8h_argmax}[fmt]
    for trial in range(3):
        x = synth.activations(rng, 1, cols)
        ref = (orc.gemm_q4 if fmt == "q4" else orc.gemm_q8)(qs, sc, x, 1, threads=8, mode=1)[0]
        y = torch.empty(rows, device="cuda")
        out = torch.full((1,), -1, dtype=torch.int64, device="cuda")
        f(dq, ds, dev(x), y, out, ws, rows, cols)
        assert np.array_equal(bits(host(y)), bits(ref))
        assert int(host(out)[0]) == orc.argmax(ref)
        assert not host(ws).any()  # rank slots cleared by the call


def test_fused_argmax_ties_and_nan(gpu_ready, orc):
    """Rows that are copies of one another tie exactly: the lowest index wins.
    A NaN logit at index 0 (a NaN scale) is the answer; elsewhere it loses."""
    rng = np.random.default_rng(8)
    qs, sc = synth.q8_weights(rng, 5000, 256)
    qs[4000] = qs[123]
    sc[4000] = sc[123]
    qs[4999] = qs[123]
    sc[4999] = sc[123]
    x = synth.activations(rng, 1, 256)
    ref = orc.gemm_q8(qs, sc, x, 1, threads=8, mode=1)[0]
    # make row 123 the maximum by scaling its block scales up
    sc[[123, 4000, 4999]] *= np.float32(50.0)
    ref = orc.gemm_q8(qs, sc, x, 1, threads=8, mode=1)[0]
    if ref[123] < 0:
        sc[[123, 4000, 4999]] *= np.float32(-1.0)
        ref = orc.gemm_q8(qs, sc, x, 1, threads=8, mode=1)[0]
    assert orc.argmax(ref) == 123 and ref[4000] == ref[123]
    ws = D.gemv_argmax_workspace()
    y = torch.empty(5000, device="cuda")
    out = torch.empty(1, dtype=torch.int64, device="cuda")
    D.gemv_q8_argmax(dev(qs), dev(sc), dev(x), y, out, ws, 5000, 256)
    assert int(host(out)[0]) == 123
    for nan_row, want in ((0, 0), (123, None)):
        s2 = sc.copy()
        s2[nan_row, 0] = np.nan
        r2 = orc.gemm_q8(qs, s2, x, 1, threads=8, mode=1)[0]
        D.gemv_q8_argmax(dev(qs), dev(s2), dev(x), y, out, ws, 5000, 256)
        assert int(host(out)[0]) == orc.argmax(r2)
        if want is not None:
            assert orc.argmax(r2) == want
    assert not host(ws).any()


@pytest.mark.parametrize("fmt", ["q8", "q4", "q8h"])
@pytest.mark.parametrize("rows,cols,n", [(6144, 2048, 1), (100, 512, 2), (4000, 1024, 3),
                                         (33, 2048, 4), (2048, 6144, 1)])
def test_gate_up_pair(gpu_ready, orc, fmt, rows, cols, n):
    """Gate and up products and the SiLU glue in one kernel: g and u
    bit-identical to the GEMV, h = SiLU(g) * u as the CPU glue rounds it."""
    rng = np.random.default_rng(rows * 5 + cols + n)
    make = synth.q4_weights if fmt == "q4" else synth.q8_weights
    gq, gs = make(rng, rows, cols)
    uq, us = make(rng, rows, cols)
    x = synth.activations(rng, n, cols)
    gemm = orc.gemm_q4 if fmt == "q4" else orc.gemm_q8
    g = gemm(gq, gs, x, n, threads=8, mode=1)
    u = gemm(uq, us, x, n, threads=8, mode=1)
    h_ref = orc.silu_mul(g, u)
    h = torch.empty((n, rows), device="cuda")
    ud = torch.empty((n, rows), device="cuda")
    f = {"q4": D.gate_up_q4, "q8": D.gate_up_q8, "q8h": D.gate_up_q8h}[fmt]
    if fmt == "q8h":
        gs, us = half_scales(gs), half_scales(us)
    f(dev(gq), dev(gs), dev(uq), dev(us), dev(x), h, rows, cols, n, u=ud)
    assert np.array_equal(bits(host(ud)), bits(u))
    hh = host(h)
    ulp = np.abs(bits(hh).astype(np.int64) - bits(h_ref).astype(np.int64))
    # SiLU runs in double on both sides (GPU exp vs the C library's): the
    # float results agree except, rarely, by one ulp at a rounding boundary.
    assert ulp.max() <= 1 and np.mean(ulp == 0) > 0.999


@pytest.mark.parametrize("fmt", ["q8", "q4", "q8h"])
@pytest.mark.parametrize("rows,cols", [((2048, 1024, 1024), 2048), ((2048, 1024, 1024, 2048), 2048),
                                       ((70, 1, 129), 96), ((3072, 512), 1024),
                                       ((1000, 33), 6144), ((4097, 8, 300, 17), 64)])
def test_multi_gemv(gpu_ready, orc, fmt, rows, cols):
    """Up to four one-token GEMVs over the same x in one launch (the
    attention projections of a decode step): each output bit-identical to
    lab_gemm mode 1 on its own matrix, and nothing written past its rows."""
    rng = np.random.default_rng(sum(rows) * 7 + cols)
    make = synth.q4_weights if fmt == "q4" else synth.q8_weights
    mats = [make(rng, r, cols) for r in rows]
    x = synth.activations(rng, 1, cols)
    gemm = orc.gemm_q4 if fmt == "q4" else orc.gemm_q8
    refs = [gemm(q, s, x, 1, threads=8, mode=1) for q, s in mats]
    ys = [torch.full((r + 64,), float("nan"), device="cuda") for r in rows]
    args = [(dev(q), dev(half_scales(s) if fmt == "q8h" else s), r) for (q, s), r in zip(mats, rows)]
    D.gemv_multi(fmt, args, dev(x), ys, cols)
    for y, ref, r in zip(ys, refs, rows):
        yh = host(y)
        assert np.array_equal(bits(yh[:r]), bits(ref[0]))
        assert np.isnan(yh[r:]).all()


def test_multi_gemv_rejects_unsupported(gpu_ready):
    z = torch.zeros(4096, device="cuda")
    q = torch.zeros(4096, dtype=torch.int8, device="cuda")
    with pytest.raises(RuntimeError):
        D.gemv_multi("q8", [], z, [], 64)                               # no matrices
    with pytest.raises(RuntimeError):
        D.gemv_multi("q8", [(q, z, 4)] * 5, z, [z] * 5, 64)              # more than four
    with pytest.raises(RuntimeError):
        D.gemv_multi("q8", [(q, z, 4), (q, z, 0)], z, [z, z], 64)        # an empty matrix
    with pytest.raises(RuntimeError):
        D.gemv_multi("q8", [(q, z, 4)], z, [z], 48)                      # cols % 32 != 0
