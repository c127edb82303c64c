"""The decode step's fused residual add and RMSNorm (dnx_gemv_add_*,
dnx_gate_up_norm_*, dnx_gemv_multi_norm_*): every output bit-identical to
the separate launches they replace (the GEMV, dnx_add, dnx_rms_norm, the
gate/up pair, the segmented GEMV), which the other tests pin to the oracle;
the normed row is also held to the oracle's rms_norm here at the bar of the
layer steps' reductions (relative 1e-5, absolute 1e-6: the row sum runs in
another order than the CPU's)."""

import numpy as np
import pytest
import torch

from dianoia_amd import device as D
from dianoia_amd import synth
from gpu_util import bits, dev, host

pytestmark = pytest.mark.gpu

EPS = 1e-6


def close_to_oracle(gpu, cpu, rtol=1e-5, atol=1e-6):
    gpu, cpu = np.asarray(gpu, np.float64), np.asarray(cpu, np.float64)
    return bool((np.abs(gpu - cpu) <= atol + rtol * np.abs(cpu)).all())


def weights(fmt, rng, rows, cols):
    return synth.q4_weights(rng, rows, cols) if fmt == "q4" else synth.q8_weights(rng, rows, cols)


def gemv_fn(fmt):
    return D.gemv_q4 if fmt == "q4" else D.gemv_q8


@pytest.mark.parametrize("fmt,rows,cols", [("q4", 2048, 2048), ("q4", 2048, 6144),
                                           ("q8", 1000, 4320), ("q8", 17, 64),
                                           ("q8", 40000, 1024), ("q4", 3, 32)])
def test_gemv_add_matches_gemv_then_add(gpu_ready, fmt, rows, cols):
    """y as dnx_gemv_*, then resid + y as dnx_add rounds it (one fp32 add)."""
    rng = np.random.default_rng(rows + cols)
    qs, sc = weights(fmt, rng, rows, cols)
    x = dev(synth.activations(rng, 1, cols))
    r0 = rng.standard_normal(rows).astype(np.float32)
    y_ref = torch.full((rows,), float("nan"), device="cuda")
    gemv_fn(fmt)(dev(qs), dev(sc), x, y_ref, rows, cols, 1)
    resid_ref = dev(r0)
    D.add(y_ref, resid_ref, rows)
    y = torch.full((rows + 64,), float("nan"), device="cuda")
    resid = torch.full((rows + 64,), float("nan"), device="cuda")
    resid[:rows] = dev(r0)
    D.gemv_add(fmt, dev(qs), dev(sc), x, y, resid, rows, cols)
    yh, rh = host(y), host(resid)
    assert np.array_equal(bits(yh[:rows]), bits(host(y_ref)))
    assert np.array_equal(bits(rh[:rows]), bits(host(resid_ref)))
    assert np.isnan(yh[rows:]).all() and np.isnan(rh[rows:]).all()


def test_gemv_add_rejects_overlap(gpu_ready):
    rng = np.random.default_rng(3)
    qs, sc = weights("q8", rng, 64, 64)
    buf = torch.zeros(256, device="cuda")
    with pytest.raises(RuntimeError):   # resid over x
        D.gemv_add("q8", dev(qs), dev(sc), buf, buf[128:], buf[32:], 64, 64)
    with pytest.raises(RuntimeError):   # resid over y
        D.gemv_add("q8", dev(qs), dev(sc), buf, buf[128:], buf[160:], 64, 64)


def norm_row(rng, cols, special):
    x = rng.standard_normal(cols).astype(np.float32) * 3
    if special == "zeros":
        x[:] = 0
    elif special == "tiny":
        x *= 1e-22
    w = (rng.standard_normal(cols) * 0.5 + 1).astype(np.float32)
    return x, w


@pytest.mark.parametrize("fmt,rows,cols,special", [("q4", 6144, 2048, None), ("q8", 2048, 1024, None),
                                                   ("q4", 100, 8192, None), ("q8", 37, 96, None),
                                                   ("q4", 512, 2048, "zeros"), ("q8", 512, 4096, "tiny")])
def test_gate_up_norm_matches_norm_then_pair(gpu_ready, orc, fmt, rows, cols, special):
    rng = np.random.default_rng(rows * 3 + cols)
    gq, gs = weights(fmt, rng, rows, cols)
    uq, us = weights(fmt, rng, rows, cols)
    xr, wr = norm_row(rng, cols, special)
    x, w = dev(xr), dev(wr)
    a_ref = torch.empty(cols, device="cuda")
    D.rms_norm(x, w, a_ref, 1, cols, EPS)
    h_ref = torch.empty(rows, device="cuda")
    u_ref = torch.empty(rows, device="cuda")
    pair = D.gate_up_q4 if fmt == "q4" else D.gate_up_q8
    pair(dev(gq), dev(gs), dev(uq), dev(us), a_ref, h_ref, rows, cols, 1, u=u_ref)
    a = torch.full((cols,), float("nan"), device="cuda")
    h = torch.full((rows,), float("nan"), device="cuda")
    u = torch.full((rows,), float("nan"), device="cuda")
    D.gate_up_norm(fmt, dev(gq), dev(gs), dev(uq), dev(us), x, w, a, EPS, h, u, rows, cols)
    assert np.array_equal(bits(host(a)), bits(host(a_ref)))
    assert close_to_oracle(host(a), orc.rms_norm(xr[None, :], wr, EPS)[0])
    assert np.array_equal(bits(host(h)), bits(host(h_ref)))
    assert np.array_equal(bits(host(u)), bits(host(u_ref)))
    assert np.array_equal(bits(host(x)), bits(xr))   # x is only read


@pytest.mark.parametrize("fmt,rows,cols", [("q4", (2048, 1024, 1024), 2048), ("q8", (4096,), 1024),
                                           ("q4", (64, 96, 32, 128), 256), ("q8", (3, 5), 8192),
                                           ("q8", (50000,), 2048), ("q4", (7,), 64)])
def test_multi_norm_matches_norm_then_multi(gpu_ready, orc, fmt, rows, cols):
    rng = np.random.default_rng(sum(rows) + cols)
    mats = [weights(fmt, rng, r, cols) for r in rows]
    xr, wr = norm_row(rng, cols, None)
    x, w = dev(xr), dev(wr)
    a_ref = torch.empty(cols, device="cuda")
    D.rms_norm(x, w, a_ref, 1, cols, EPS)
    args = [(dev(q), dev(s), r) for (q, s), r in zip(mats, rows)]
    ys_ref = [torch.empty(r, device="cuda") for r in rows]
    D.gemv_multi(fmt, args, a_ref, ys_ref, cols)
    a = torch.full((cols,), float("nan"), device="cuda")
    ys = [torch.full((r + 64,), float("nan"), device="cuda") for r in rows]
    D.gemv_multi_norm(fmt, args, x, w, a, EPS, ys, cols)
    assert np.array_equal(bits(host(a)), bits(host(a_ref)))
    assert close_to_oracle(host(a), orc.rms_norm(xr[None, :], wr, EPS)[0])
    for y, y_ref, r in zip(ys, ys_ref, rows):
        yh = host(y)
        assert np.array_equal(bits(yh[:r]), bits(host(y_ref)))
        assert np.isnan(yh[r:]).all()


def test_fused_norm_rejects_unsupported(gpu_ready):
    rng = np.random.default_rng(5)
    cols = 8224  # past one batch of quads per thread
    q, s = weights("q8", rng, 8, cols)
    x = torch.zeros(cols + 64, device="cuda")
    w = torch.ones(cols, device="cuda")
    out = torch.zeros(cols, device="cuda")
    y = torch.zeros(8, device="cuda")
    with pytest.raises(RuntimeError):
        D.gemv_multi_norm("q8", [(dev(q), dev(s), 8)], x, w, out, EPS, [y], cols)
    q, s = weights("q8", rng, 8, 64)
    with pytest.raises(RuntimeError):   # norm output over x
        D.gemv_multi_norm("q8", [(dev(q), dev(s), 8)], x, w, x[16:], EPS, [y], 64)
    with pytest.raises(RuntimeError):   # x not 16-byte aligned
        D.gemv_multi_norm("q8", [(dev(q), dev(s), 8)], x[1:], w, out, EPS, [y], 64)
