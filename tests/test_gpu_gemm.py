"""Prefill GEMMs: per-block int32 dots exact, fp32 outputs within 1e-4.

Two paths: "i8" is dnx_gemm_q8/q4 on int8 xq + fp32 xsc; "panel" packs the
same xq/xsc into the fp16/bf16-MFMA kernel's activation panel
(dnx_pack_panel) and runs dnx_gemm_q8/q4_panel."""

import numpy as np
import pytest
import torch

from dianoia_amd import device as D
from dianoia_amd import synth
from gpu_util import bits, dev, host, within_tolerance

pytestmark = pytest.mark.gpu


PATHS = ["i8", "panel"]


def gemm(fmt, qs, sc, xq, xsc, rows, cols, n, path="i8"):
    y = torch.full((n, rows), float("nan"), dtype=torch.float32, device="cuda")
    if path == "panel":
        panel = torch.full((D.gemm_panel_bytes(n, cols),), 0x7f, dtype=torch.uint8, device="cuda")
        D.pack_panel(dev(xq), dev(xsc), panel, n, cols)
        f = D.gemm_q4_panel if fmt == "q4" else D.gemm_q8_panel
        f(dev(qs), dev(sc), panel, y, rows, cols, n)
    else:
        f = D.gemm_q4 if fmt == "q4" else D.gemm_q8
        f(dev(qs), dev(sc), dev(xq), dev(xsc), y, rows, cols, n)
    return host(y)


@pytest.mark.parametrize("path", PATHS)
@pytest.mark.parametrize("fmt", ["q8", "q4"])
@pytest.mark.parametrize("rows,cols,n", [(130, 256, 70), (128, 128, 128), (33, 96, 5),
                                         (200, 320, 300), (70, 256, 37), (40, 1024, 64),
                                         (17, 2048, 16)])
def test_block_dots_are_exact(gpu_ready, orc, fmt, rows, cols, n, path):
    """With scale 1 on one block and 0 on the others, y is that block's
    int32 dot product as a float (exact below 2^24): the MFMA's integer
    result for every block, compared with brute-force sums."""
    rng = np.random.default_rng(rows + cols + n)
    B = cols // 32
    xq = rng.integers(-127, 128, (n, cols), dtype=np.int8)
    if fmt == "q8":
        qs = rng.integers(-127, 128, (rows, cols), dtype=np.int8)
        want = orc.block_dots_q8(qs, xq)
        one, zero = np.float32(1.0), np.float32(0.0)
    else:
        qs = rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8)
        want = orc.block_dots_q4(qs, xq)
        one, zero = np.uint16(0x3C00), np.uint16(0)
    for b in range(B):
        sw = np.full((rows, B), zero)
        sw[:, b] = one
        xsc = np.zeros((n, B), np.float32)
        xsc[:, b] = 1.0
        y = gemm(fmt, qs, sw, xq, xsc, rows, cols, n, path)
        assert np.array_equal(y, want[:, :, b].astype(np.float32)), f"block {b}"


@pytest.mark.parametrize("fmt", ["q8", "q4"])
def test_panel_unit_scales_sum_blocks_exactly(gpu_ready, orc, fmt):
    """All scales 1: y is the sum over blocks of the exact int32 dots, exact
    in float while the total stays below 2^24 (the MFMA's integer-valued
    fp16 products and the outer-product scale of exactly 1)."""
    rows, cols, n = 96, 2048, 160
    rng = np.random.default_rng(7)
    xq = rng.integers(-127, 128, (n, cols), dtype=np.int8)
    if fmt == "q8":
        qs = rng.integers(-127, 128, (rows, cols), dtype=np.int8)
        want = orc.block_dots_q8(qs, xq).sum(axis=2)
        sw = np.ones((rows, cols // 32), np.float32)
    else:
        qs = rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8)
        want = orc.block_dots_q4(qs, xq).sum(axis=2)
        sw = np.full((rows, cols // 32), np.uint16(0x3C00))
    assert np.abs(want).max() < 2 ** 24
    xsc = np.ones((n, cols // 32), np.float32)
    y = gemm(fmt, qs, sw, xq, xsc, rows, cols, n, "panel")
    assert np.array_equal(y, want.astype(np.float32))


def exact_products(orc, fmt, qs, sc, xq, xsc):
    """The reference arithmetic without rounding: sum_b d_b * fp32(sw * sx),
    in float64, and the magnitude sum_b |d_b * s_b| native_kernels_test.dart
    measures errors against (:50-59)."""
    d = (orc.block_dots_q4 if fmt == "q4" else orc.block_dots_q8)(qs, xq).astype(np.float64)
    sw = sc.view(np.float16).astype(np.float32) if fmt == "q4" else sc
    s = (sw[None, :, :] * xsc[:, None, :]).astype(np.float32).astype(np.float64)
    return (d * s).sum(axis=2), np.abs(d * s).sum(axis=2)


@pytest.mark.parametrize("path", PATHS)
@pytest.mark.parametrize("fmt", ["q8", "q4"])
@pytest.mark.parametrize("rows,cols,n", [(6144, 2048, 512), (70, 96, 13), (36, 64, 9),
                                         (128, 128, 40), (4304, 1152, 64), (1152, 4320, 33),
                                         (257, 2048, 1), (100, 2048, 64), (6144, 2048, 8),
                                         (6144, 2048, 32), (2048, 6144, 16), (6144, 2048, 64),
                                         (4304, 1152, 300), (1152, 4320, 200), (97, 160, 129),
                                         (1152, 4096, 960)])
def test_gemm_within_tolerance(gpu_ready, orc, fmt, rows, cols, n, path):
    """Against the exact products: the reference kernels' own bar (error /
    sum|terms| < 1e-5, native_kernels_test.dart:56-59), met by the CPU kernels
    too. Against the CPU outputs: the per-element bar (relative 1e-4, absolute
    1e-5 near zero) on the Q4 distribution of the prefill configuration,
    whose outputs are O(1). Random Q8 blocks give |y| ~ 30, where any float
    order other than the CPU's differs by more than 1e-5 absolute near zero;
    there the reference's GPU-vs-CPU tolerance applies (gpu_linear_test.dart:44)."""
    rng = np.random.default_rng(rows * 3 + cols + n)
    if fmt == "q8":
        qs, sc = synth.q8_weights(rng, rows, cols)
    else:
        qs, sc = synth.q4_weights(rng, rows, cols)
    xs = synth.activations(rng, n, cols)
    xq, xsc = orc.quantize_q8(xs)
    ref = (orc.gemm_q8 if fmt == "q8" else orc.gemm_q4)(qs, sc, xs, n, threads=8, mode=1)
    y = gemm(fmt, qs, sc, xq, xsc, rows, cols, n, path)
    exact, mag = exact_products(orc, fmt, qs, sc, xq, xsc)
    assert np.max(np.abs(y - exact) / mag) < 1e-5
    assert np.max(np.abs(ref - exact) / mag) < 1e-5
    if fmt == "q4":
        ok, worst_rel, worst_abs = within_tolerance(y, ref)
        assert ok, (worst_rel, worst_abs)
    else:
        assert np.all(np.abs(y - ref) <= 1e-4 + 1e-5 * np.abs(ref))


def test_gemm_rejects_unsupported(gpu_ready):
    z = torch.zeros(4096, device="cuda")
    with pytest.raises(RuntimeError):
        D.gemm_q8(z, z, z, z, z, 4, 40, 2)


@pytest.mark.parametrize("rows,cols,n", [(6144, 2048, 8), (2048, 6144, 40), (6144, 2048, 512)])
def test_gemm_is_deterministic(gpu_ready, rows, cols, n):
    """Split-K partials are summed in a fixed order: repeated calls (and
    calls after a larger one regrew the workspace) give identical bits."""
    rng = np.random.default_rng(rows + n)
    qs, sc = synth.q4_weights(rng, rows, cols)
    xs = synth.activations(rng, n, cols)
    xq, xsc = dev(np.zeros((n, cols), np.int8)), dev(np.zeros((n, cols // 32), np.float32))
    D.quantize_q8(dev(xs), xq, xsc, n, cols, cols)
    outs = []
    for _ in range(3):
        y = torch.full((n, rows), float("nan"), device="cuda")
        D.gemm_q4(dev(qs), dev(sc), xq, xsc, y, rows, cols, n)
        outs.append(host(y))
    assert all(np.array_equal(bits(o), bits(outs[0])) for o in outs[1:])


@pytest.mark.parametrize("n,cols", [(512, 2048), (33, 96), (1, 32), (100, 4320)])
def test_quantize_panel_matches_pack(gpu_ready, n, cols):
    """dnx_quantize_q8_panel writes the same panel bytes as dnx_quantize_q8
    followed by dnx_pack_panel (the quantized values are lab_quantize_q8's),
    including the zero rows that pad the last 32-row group."""
    rng = np.random.default_rng(n + cols)
    x = dev(synth.activations(rng, n, cols))
    xq = torch.empty((n, cols), dtype=torch.int8, device="cuda")
    xsc = torch.empty((n, cols // 32), dtype=torch.float32, device="cuda")
    D.quantize_q8(x, xq, xsc, n, cols, cols)
    size = D.gemm_panel_bytes(n, cols)
    a = torch.full((size,), 0x5a, dtype=torch.uint8, device="cuda")
    b = torch.full((size,), 0xa5, dtype=torch.uint8, device="cuda")
    D.pack_panel(xq, xsc, a, n, cols)
    D.quantize_q8_panel(x, b, n, cols)
    assert np.array_equal(host(a), host(b))
