"""The Q8 GEMM on the int8 matrix cores over prepacked operands
(dnx_gemm_q8_i8p): its activation panel carries lab_quantize_q8's xq and
scale bits, its weight prepack the engine's Q8 codes and scales, its block
dots are exact, and its fp32 outputs meet the north-star bar against the CPU
kernel (lab_gemm_q8 mode 1, lab_native.c:553-579)."""

import numpy as np
import pytest
import torch

from dianoia_amd import device as D
from dianoia_amd import synth
from gpu_util import bits, dev, host, within_tolerance

pytestmark = pytest.mark.gpu

REC = 1536   # bytes per (32 rows or tokens, block)


def bf16(u16):
    return (np.asarray(u16, np.uint32) << 16).view(np.float32).astype(np.float64)


def record_parts(buf, count, cols):
    """Codes [count][cols] (int8) and the lane-half-1 scale slots [count][B][4]
    (uint16) of a panel or prepack."""
    p = host(buf).view(np.uint8)
    B = cols // 32
    codes = np.zeros((count, cols), np.int8)
    slots = np.zeros((count, B, 2, 4), np.uint16)
    for r in range(count):
        g, i = divmod(r, 32)
        for b in range(B):
            rec = (g * B + b) * REC
            codes[r, b * 32:b * 32 + 16] = p[rec + i * 16:rec + i * 16 + 16].view(np.int8)
            codes[r, b * 32 + 16:b * 32 + 32] = p[rec + 512 + i * 16:rec + 512 + i * 16 + 16].view(np.int8)
            for h in range(2):
                o = rec + 1024 + h * 256 + i * 8
                slots[r, b, h] = p[o:o + 8].view(np.uint16)
    return codes, slots


@pytest.mark.parametrize("n,cols", [(70, 256), (5, 96), (32, 1152), (131, 4320)])
def test_panel_holds_lab_quantize_q8(gpu_ready, orc, n, cols):
    """Every live token's int8 codes are lab_quantize_q8's xq; its scale's
    three bf16 pieces (lane half 1: p0, p1, p2; half 0: p0, p0, p1) sum
    exactly to lab_quantize_q8's scale. Padding tokens hold zero records."""
    rng = np.random.default_rng(n + cols)
    x = synth.activations(rng, n, cols)
    x[0, :32] = 0.0                      # an all-zero block: scale 0
    xq, xsc = orc.quantize_q8(x)
    groups = (n + 31) // 32
    panel = torch.full((D.i8_panel_bytes(n, cols),), 0x7f, dtype=torch.uint8, device="cuda")
    D.quantize_q8_i8panel(dev(x), panel, n, cols)
    codes, slots = record_parts(panel, groups * 32, cols)
    assert np.array_equal(codes[:n], xq)
    assert not codes[n:].any() and not slots[n:].any()
    h0, h1 = slots[:n, :, 0], slots[:n, :, 1]
    assert np.array_equal(h0[..., 0], h1[..., 0]) and np.array_equal(h0[..., 1], h1[..., 0])
    assert np.array_equal(h0[..., 2], h1[..., 1]) and not h0[..., 3].any() and not h1[..., 3].any()
    total = bf16(h1[..., 0]) + bf16(h1[..., 1]) + bf16(h1[..., 2])
    assert np.array_equal(total, xsc.astype(np.float64))


@pytest.mark.parametrize("rows,cols", [(70, 96), (4320, 1152), (33, 4320)])
def test_prepack_holds_the_weights(gpu_ready, orc, rows, cols):
    """The prepack's codes are the Q8 codes (rows past the matrix zero); its
    scale slots (half 0: w0, w1, w0; half 1: w2, w1, w0) hold three bf16
    pieces that sum exactly to the fp32 weight scale."""
    rng = np.random.default_rng(rows + cols)
    qs, sc = orc.quantize_q8((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
    padded = (rows + 31) // 32 * 32
    pk = torch.full((D.q8_i8pack_bytes(rows, cols),), 0x7f, dtype=torch.uint8, device="cuda")
    D.pack_q8_i8(dev(qs), dev(sc), pk, rows, cols)
    codes, slots = record_parts(pk, padded, cols)
    assert np.array_equal(codes[:rows], qs)
    assert not codes[rows:].any() and not slots[rows:].any()
    h0, h1 = slots[:rows, :, 0], slots[:rows, :, 1]
    assert np.array_equal(h0[..., 0], h1[..., 2]) and np.array_equal(h0[..., 1], h1[..., 1])
    assert np.array_equal(h0[..., 2], h1[..., 2])
    total = bf16(h1[..., 2]) + bf16(h1[..., 1]) + bf16(h1[..., 0])
    assert np.array_equal(total, sc.astype(np.float64))


def gemm_i8p(qs, sc, x, rows, cols, n):
    panel = torch.full((D.i8_panel_bytes(n, cols),), 0x7f, dtype=torch.uint8, device="cuda")
    D.quantize_q8_i8panel(dev(x), panel, n, cols)
    packed = torch.empty(D.q8_i8pack_bytes(rows, cols), dtype=torch.uint8, device="cuda")
    D.pack_q8_i8(dev(qs), dev(sc), packed, rows, cols)
    y = torch.full((n, rows), float("nan"), dtype=torch.float32, device="cuda")
    D.gemm_q8_i8p(packed, panel, y, rows, cols, n)
    return host(y)


def activations_for(xq):
    """fp32 rows whose lab_quantize_q8 gives exactly xq with scale 1 in every
    block holding 127 or -127 (x = xq)."""
    return xq.astype(np.float32)


@pytest.mark.parametrize("rows,cols,n", [(130, 256, 70), (33, 96, 5), (97, 1024, 131),
                                         (200, 320, 300)])
def test_block_dots_are_exact(gpu_ready, orc, rows, cols, n):
    """Weight scale 1 on one block and 0 on the others, activations whose
    blocks all quantize with scale 1 (each holds a 127): y is that block's
    exact dot sum_k xq * w against brute force, for every block. The weights
    cover every int8 value including -128."""
    rng = np.random.default_rng(rows + cols + n + 5)
    B = cols // 32
    xq = rng.integers(-127, 128, (n, cols), dtype=np.int8)
    xq[:, ::32] = 127
    xq[-1, 1:32] = -127
    x = activations_for(xq)
    xq_o, xsc_o = orc.quantize_q8(x)
    assert np.array_equal(xq_o, xq) and np.all(xsc_o == 1.0)
    qs = rng.integers(-128, 128, (rows, cols), dtype=np.int16).astype(np.int8)
    qs[0, :32] = -128
    qs[-1, -32:] = 127
    qs[1 % rows, :min(cols, 256)] = np.arange(-128, 128, dtype=np.int16)[:min(cols, 256)].astype(np.int8)
    want = orc.block_dots_q8(qs, xq)
    for b in range(B):
        sw = np.zeros((rows, B), np.float32)
        sw[:, b] = 1.0
        y = gemm_i8p(qs, sw, x, rows, cols, n)
        assert np.array_equal(y, want[:, :, b].astype(np.float32)), f"block {b}"


@pytest.mark.parametrize("rows,cols,n,fp32_scales", [(4320, 1152, 1024, True),
                                                     (1152, 4320, 1024, True),
                                                     (1024, 1024, 1024, False),
                                                     (70, 96, 13, True), (128, 128, 40, False),
                                                     (97, 160, 129, True),
                                                     (2048, 4096, 256, False),
                                                     (300, 8192, 64, True)])
def test_gemm_within_tolerance(gpu_ready, orc, rows, cols, n, fp32_scales):
    """Against the exact products (error / sum|terms| below 1e-5) and the CPU
    kernel's outputs (relative 1e-4, absolute 1e-5 near zero): weights
    quantized by lab_quantize_q8 (the vision encoder's BF16 -> Q8 path,
    fp32 scales) and GGUF-style fp16-exact scales. The shapes take one or
    two rounds of tiles and K splits of 1 to 32 parts."""
    rng = np.random.default_rng(rows * 7 + cols + n)
    if fp32_scales:
        qs, sc = orc.quantize_q8((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
    else:
        qs, sc = synth.q8_weights(rng, rows, cols)
        sc = (sc / np.float32(16)).astype(np.float16).astype(np.float32)
    xs = synth.activations(rng, n, cols)
    xq, xsc = orc.quantize_q8(xs)
    ref = orc.gemm_q8(qs, sc, xs, n, threads=8, mode=1)
    y = gemm_i8p(qs, sc, xs, rows, cols, n)
    d = orc.block_dots_q8(qs, xq).astype(np.float64)
    s = (sc[None, :, :].astype(np.float32) * xsc[:, None, :]).astype(np.float32).astype(np.float64)
    exact, mag = (d * s).sum(axis=2), np.abs(d * s).sum(axis=2)
    assert np.all(np.abs(y - exact) <= 1e-5 * mag)
    ok, worst_rel, worst_abs = within_tolerance(y, ref)
    assert ok, (worst_rel, worst_abs)


@pytest.mark.parametrize("rows,cols,n,tile", [(4303, 1152, 1000, (160, 128)),
                                               (2001, 256, 2100, (160, 128)),
                                               (2900, 256, 1100, (128, 128)),
                                               (999, 256, 2100, (96, 128)),
                                               (333, 1024, 1100, (128, 64)),
                                               (771, 1024, 333, (96, 64)),
                                               (333, 256, 130, (96, 64))])
def test_every_tile(gpu_ready, orc, rows, cols, n, tile):
    """Every tile: 128 tokens x 96, 128 or 160 rows (160 adds the two block
    parities in place, in half the LDS) and 64 tokens x 96 or 128 rows (four
    block parities), at ragged shapes: rows not a multiple of the tile or
    of 4 (no 16-byte stores), tokens not a multiple of the tile, against the
    exact products and the CPU kernel."""
    assert D.gemm_q8_i8p_tile(rows, cols, n) == tile
    rng = np.random.default_rng(rows + cols * 3 + n)
    qs, sc = orc.quantize_q8((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
    xs = synth.activations(rng, n, cols)
    xq, xsc = orc.quantize_q8(xs)
    ref = orc.gemm_q8(qs, sc, xs, n, threads=8, mode=1)
    y = gemm_i8p(qs, sc, xs, rows, cols, n)
    d = orc.block_dots_q8(qs, xq).astype(np.float64)
    s = (sc[None, :, :].astype(np.float32) * xsc[:, None, :]).astype(np.float32).astype(np.float64)
    exact, mag = (d * s).sum(axis=2), np.abs(d * s).sum(axis=2)
    assert np.all(np.abs(y - exact) <= 1e-5 * mag)
    ok, worst_rel, worst_abs = within_tolerance(y, ref)
    assert ok, (worst_rel, worst_abs)


def test_tile_choice_of_the_vision_pair(gpu_ready):
    """fc1 (4320 x 1152 at 1024 tokens) takes 128 x 160 tiles, one round of
    216 workgroups; fc2 (1152 x 4320) 128 x 128 tiles in three K parts; the
    1024 x 1024 projections at 1024 tokens 64 x 96 tiles with no K split;
    refused shapes give None."""
    assert D.gemm_q8_i8p_tile(4320, 1152, 1024) == (160, 128)
    assert D.gemm_q8_i8p_tile(1152, 4320, 1024) == (128, 128)
    assert D.gemm_q8_i8p_tile(1024, 1024, 1024) == (96, 64)
    assert D.gemm_q8_i8p_tile(64, 48, 5) is None


def test_gemm_is_deterministic(gpu_ready, orc):
    """Two launches give the same bits (the K split's partials are added in
    a fixed order)."""
    rows, cols, n = 1152, 4320, 1024
    rng = np.random.default_rng(3)
    qs, sc = orc.quantize_q8((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
    xs = synth.activations(rng, n, cols)
    a = gemm_i8p(qs, sc, xs, rows, cols, n)
    b = gemm_i8p(qs, sc, xs, rows, cols, n)
    assert np.array_equal(bits(a), bits(b))


def test_refuses_bad_shapes(gpu_ready):
    z = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    y = torch.zeros(64 * 64, device="cuda")
    x = torch.zeros(64 * 64, device="cuda")
    with pytest.raises(RuntimeError):
        D.gemm_q8_i8p(z, z, y, 64, 48, 5)     # cols not a multiple of 32
    with pytest.raises(RuntimeError):
        D.gemm_q8_i8p(z, z, y, 64, 64, 0)     # no tokens
    with pytest.raises(RuntimeError):
        D.quantize_q8_i8panel(x[1:], z, 2, 64)  # x not 16-byte aligned
