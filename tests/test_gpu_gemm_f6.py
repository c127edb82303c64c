"""The fp6-MFMA Q4 GEMM (dnx_gemm_q4_f6): per-block dots exact, fp32 outputs
within the north-star bar of the CPU kernels (lab_gemm_q4 mode 1).

The activations reach it as an "f6 panel", written either from fp32 x by the
quantizer (dnx_quantize_q8_f6panel, lab_quantize_q8's values) or from
already quantized xq + xsc (dnx_pack_f6panel)."""

import numpy as np
import pytest
import torch

from dianoia_amd import device as D
from dianoia_amd import synth
from gpu_util import bits, dev, host, within_tolerance

pytestmark = pytest.mark.gpu


def gemm_f6(qs, sc, xq, xsc, rows, cols, n):
    panel = torch.full((D.f6_panel_bytes(n, cols),), 0x7f, dtype=torch.uint8, device="cuda")
    D.pack_f6panel(dev(xq), dev(xsc), panel, n, cols)
    y = torch.full((n, rows), float("nan"), dtype=torch.float32, device="cuda")
    D.gemm_q4_f6(dev(qs), dev(sc), panel, y, rows, cols, n)
    return host(y)


@pytest.mark.parametrize("rows,cols,n", [(130, 256, 70), (96, 128, 128), (33, 96, 5),
                                         (200, 320, 300), (17, 2048, 16), (97, 1024, 131)])
def test_block_dots_are_exact(gpu_ready, orc, rows, cols, n):
    """Scale 1 on one block and 0 on the others: y is that block's exact dot
    sum_k xq * (q - 8) as a float, for every block, against brute force.
    Covers both fp6 pieces of every |xq| up to 127, negative xq, every
    nibble, and the -8 * sum(xq) C input."""
    rng = np.random.default_rng(rows + cols + n)
    B = cols // 32
    xq = rng.integers(-127, 128, (n, cols), dtype=np.int8)
    xq[0, :32] = 127
    xq[-1, -32:] = -127
    qs = rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8)
    qs[0, :16] = 0x00
    qs[-1, -16:] = 0xff
    want = orc.block_dots_q4(qs, xq)
    for b in range(B):
        sw = np.zeros((rows, B), np.uint16)
        sw[:, b] = 0x3C00
        xsc = np.zeros((n, B), np.float32)
        xsc[:, b] = 1.0
        y = gemm_f6(qs, sw, xq, xsc, rows, cols, n)
        assert np.array_equal(y, want[:, :, b].astype(np.float32)), f"block {b}"


def test_unit_scales_sum_blocks_exactly(gpu_ready, orc):
    """All scales 1: y is the exact sum over blocks of the integer dots
    (below 2^24, so every fp32 partial sum is exact)."""
    rows, cols, n = 200, 2048, 160
    rng = np.random.default_rng(7)
    xq = rng.integers(-127, 128, (n, cols), dtype=np.int8)
    qs = rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8)
    want = orc.block_dots_q4(qs, xq).sum(axis=2)
    assert np.abs(want).max() < 2 ** 24
    y = gemm_f6(qs, np.full((rows, cols // 32), np.uint16(0x3C00)), xq,
                np.ones((n, cols // 32), np.float32), rows, cols, n)
    assert np.array_equal(y, want.astype(np.float32))


def test_power_of_two_scales_are_exact(gpu_ready, orc):
    """Scales that are powers of two (the activation scale's exponent rides
    in the MFMA's E8M0 scale, its mantissa in the outer product) give the
    exact scaled sum: every term is an integer times a power of two."""
    rows, cols, n = 64, 512, 96
    rng = np.random.default_rng(11)
    B = cols // 32
    xq = rng.integers(-127, 128, (n, cols), dtype=np.int8)
    qs = rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8)
    ex = rng.integers(-20, 10, (n, B))
    ew = rng.integers(-10, 5, (rows, B))
    xsc = np.ldexp(np.ones((n, B)), ex).astype(np.float32)
    sw = np.ldexp(np.ones((rows, B), np.float32), ew).astype(np.float16).view(np.uint16)
    d = orc.block_dots_q4(qs, xq).astype(np.float64)
    want = (d * np.ldexp(1.0, ex)[:, None, :] * np.ldexp(1.0, ew)[None, :, :]).sum(axis=2)
    y = gemm_f6(qs, sw, xq, xsc, rows, cols, n)
    # Exact terms; only the fp32 rounding of the running sum remains.
    mag = (np.abs(d) * np.ldexp(1.0, ex)[:, None, :] * np.ldexp(1.0, ew)[None, :, :]).sum(axis=2)
    assert np.max(np.abs(y - want) / mag) < 2 ** -20


def exact_products(orc, qs, sc, xq, xsc):
    """sum_b d_b * fp32(sw * sx) in float64, and sum_b |d_b * s_b|."""
    d = orc.block_dots_q4(qs, xq).astype(np.float64)
    sw = sc.view(np.float16).astype(np.float32)
    s = (sw[None, :, :] * xsc[:, None, :]).astype(np.float32).astype(np.float64)
    return (d * s).sum(axis=2), np.abs(d * s).sum(axis=2)


@pytest.mark.parametrize("rows,cols,n", [(6144, 2048, 512), (70, 96, 13), (36, 64, 9),
                                         (128, 128, 40), (4304, 1152, 64), (1152, 4320, 33),
                                         (257, 2048, 1), (100, 2048, 64), (6144, 2048, 128),
                                         (2048, 6144, 256), (6144, 2048, 1024), (97, 160, 129),
                                         (1152, 4320, 1024), (4304, 1152, 1024), (96, 32, 200)])
def test_gemm_within_tolerance(gpu_ready, orc, rows, cols, n):
    """Against the exact products: error / sum|terms| below 1e-5 (the
    reference kernels' own bar, native_kernels_test.dart:56-59). Against the
    CPU kernel's outputs: relative 1e-4, or absolute 1e-5 near zero."""
    rng = np.random.default_rng(rows * 3 + cols + n)
    qs, sc = synth.q4_weights(rng, rows, cols)
    xs = synth.activations(rng, n, cols)
    xq, xsc = orc.quantize_q8(xs)
    ref = orc.gemm_q4(qs, sc, xs, n, threads=8, mode=1)
    y = gemm_f6(qs, sc, xq, xsc, rows, cols, n)
    exact, mag = exact_products(orc, qs, sc, xq, xsc)
    assert np.all(np.abs(y - exact) <= 1e-5 * mag)
    ok, worst_rel, worst_abs = within_tolerance(y, ref)
    assert ok, (worst_rel, worst_abs)


@pytest.mark.parametrize("n,cols", [(512, 2048), (33, 96), (1, 32), (100, 4320), (257, 1152)])
def test_quantizer_panel_matches_pack(gpu_ready, n, cols):
    """dnx_quantize_q8_f6panel writes the same bytes as dnx_quantize_q8
    followed by dnx_pack_f6panel (lab_quantize_q8's values), including the
    zero rows that pad the last group of 32 tokens."""
    rng = np.random.default_rng(n + cols)
    x = dev(synth.activations(rng, n, cols))
    xq = torch.empty((n, cols), dtype=torch.int8, device="cuda")
    xsc = torch.empty((n, cols // 32), dtype=torch.float32, device="cuda")
    D.quantize_q8(x, xq, xsc, n, cols, cols)
    size = D.f6_panel_bytes(n, cols)
    a = torch.full((size,), 0x5a, dtype=torch.uint8, device="cuda")
    b = torch.full((size,), 0xa5, dtype=torch.uint8, device="cuda")
    D.pack_f6panel(xq, xsc, a, n, cols)
    D.quantize_q8_f6panel(x, b, n, cols)
    assert np.array_equal(host(a), host(b))


def test_quantizer_edges_through_the_gemm(gpu_ready, orc):
    """Rows with an all-zero block, a single nonzero value, tiny (subnormal
    scale) and large values go through the quantizer's panel and the GEMM
    within the bar of the CPU kernels."""
    rows, cols, n = 96, 256, 40
    rng = np.random.default_rng(3)
    qs, sc = synth.q4_weights(rng, rows, cols)
    xs = synth.activations(rng, n, cols)
    xs[0, :32] = 0.0
    xs[1, :] = 0.0
    xs[1, 5] = 3.0
    xs[2, 32:64] *= 1e-40
    xs[3, :] *= 1e30
    xs[4, 64:96] = -2.5
    ref = orc.gemm_q4(qs, sc, xs, n, threads=8, mode=1)
    panel = torch.empty((D.f6_panel_bytes(n, cols),), dtype=torch.uint8, device="cuda")
    D.quantize_q8_f6panel(dev(xs), panel, n, cols)
    y = torch.full((n, rows), float("nan"), device="cuda")
    D.gemm_q4_f6(dev(qs), dev(sc), panel, y, rows, cols, n)
    ok, worst_rel, worst_abs = within_tolerance(host(y), ref)
    assert ok, (worst_rel, worst_abs)


def test_rejects_unsupported(gpu_ready):
    z = torch.zeros(4096, device="cuda")
    with pytest.raises(RuntimeError):
        D.gemm_q4_f6(z, z, z, z, 4, 40, 2)   # cols % 32 != 0
    with pytest.raises(RuntimeError):
        D.quantize_q8_f6panel(z, z, 0, 32)   # n = 0


@pytest.mark.parametrize("rows,cols,n", [(6144, 2048, 512), (1152, 4320, 1024), (2048, 6144, 64)])
def test_deterministic(gpu_ready, rows, cols, n):
    """Split-K partials are summed in a fixed order: repeated calls give
    identical bits."""
    rng = np.random.default_rng(rows + n)
    qs, sc = synth.q4_weights(rng, rows, cols)
    xs = dev(synth.activations(rng, n, cols))
    panel = torch.empty((D.f6_panel_bytes(n, cols),), dtype=torch.uint8, device="cuda")
    D.quantize_q8_f6panel(xs, panel, n, cols)
    outs = []
    for _ in range(3):
        y = torch.full((n, rows), float("nan"), device="cuda")
        D.gemm_q4_f6(dev(qs), dev(sc), panel, y, rows, cols, n)
        outs.append(host(y))
    assert all(np.array_equal(bits(o), bits(outs[0])) for o in outs[1:])


# ------------------------------------------------------------ prepacked weights

# The field order of a block's 32 weights in the fp6 operand (a property of
# the conversion the kernels use; the token panel follows the same order).
FIELD_K = [0, 20, 17, 6, 3, 23, 16, 5, 2, 22, 19, 4, 1, 21, 18, 7,
           8, 28, 25, 14, 11, 31, 24, 13, 10, 30, 27, 12, 9, 29, 26, 15]


def packed_records(packed, rows, cols):
    """The tile-major prepack ([32-row group][block][half][32 rows][16 B])
    as one 32-byte record per (row, block); also checks that the rows that
    pad the last group hold zero records."""
    groups, nb = (rows + 31) // 32, cols // 32
    chunks = packed.reshape(groups, nb, 2, 32, 16)
    rec = chunks.transpose(0, 3, 1, 2, 4).reshape(groups * 32, nb, 32)
    assert not rec[rows:].any()
    return np.ascontiguousarray(rec[:rows])


def decode_packed(packed, rows, cols):
    """Record (row, block) -> the 32 signed weights its fp6 fields encode
    (E2M3: sign bit 5, magnitude code |w| <= 8 is the value |w| / 8, here
    times the kernel's scale 8) and its two operand dwords."""
    rec = packed_records(packed, rows, cols)
    words = rec[:, :, :24].copy().view(np.uint32).astype(np.uint64)   # 6 dwords
    bits = np.zeros(words.shape[:2], dtype=object)
    w = np.zeros((rows, cols // 32, 32), np.int64)
    stream = sum(words[:, :, j].astype(object) << (32 * j) for j in range(6))
    for f in range(32):
        code = (stream >> (6 * f)) & 63
        code = np.vectorize(int)(code)
        mag = code & 31
        assert np.all(mag <= 8)
        w[:, :, FIELD_K[f]] = np.where(code & 32, -mag, mag)
    ops = rec[:, :, 24:].copy().view(np.uint32)
    return w, ops


def test_prepack_encodes_signed_weights(gpu_ready):
    """Every field of the load-time re-encoding holds q - 8 of its weight
    (decoded from the E2M3 bits, not by the kernels' own code), for every
    nibble value, and the operand dwords hold (sw, sw, 0, sw)."""
    rows, cols = 40, 256
    rng = np.random.default_rng(5)
    qs = rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8)
    qs[0, :16] = np.arange(16, dtype=np.uint8) * 17   # both nibbles take every value
    sc = rng.integers(0, 0x7c00, (rows, cols // 32)).astype(np.uint16)
    packed = torch.empty(D.q4_f6pack_bytes(rows, cols), dtype=torch.uint8, device="cuda")
    D.pack_q4_f6(dev(qs), dev(sc), packed, rows, cols)
    w, ops = decode_packed(host(packed), rows, cols)
    blocks = qs.reshape(rows, cols // 32, 16).astype(np.int64)
    q = np.concatenate([blocks & 15, blocks >> 4], axis=2)   # weight k: low nibble of byte k, k+16 high
    assert np.array_equal(w, q - 8)
    sw = sc.astype(np.uint32)
    assert np.array_equal(ops[:, :, 0], sw | (sw << 16))
    assert np.array_equal(ops[:, :, 1], sw << 16)


@pytest.mark.parametrize("rows,cols,n", [(6144, 2048, 512), (130, 256, 70), (1152, 4320, 1024),
                                         (4304, 1152, 1024), (97, 160, 129), (257, 2048, 40)])
def test_prepacked_gemm_equals_engine_layout(gpu_ready, orc, rows, cols, n):
    """The GEMM on the prepacked weights gives the same bits as the GEMM on
    the engine's layout (both block dots are exact and the epilogues run the
    same operations), and so meets the same bar against the CPU kernels."""
    rng = np.random.default_rng(rows + 7 * n)
    qs, sc = synth.q4_weights(rng, rows, cols)
    xs = synth.activations(rng, n, cols)
    panel = torch.empty((D.f6_panel_bytes(n, cols),), dtype=torch.uint8, device="cuda")
    D.quantize_q8_f6panel(dev(xs), panel, n, cols)
    packed = torch.empty(D.q4_f6pack_bytes(rows, cols), dtype=torch.uint8, device="cuda")
    D.pack_q4_f6(dev(qs), dev(sc), packed, rows, cols)
    y0 = torch.full((n, rows), float("nan"), device="cuda")
    y1 = torch.full((n, rows), float("nan"), device="cuda")
    D.gemm_q4_f6(dev(qs), dev(sc), panel, y0, rows, cols, n)
    D.gemm_q4_f6p(packed, panel, y1, rows, cols, n)
    a, b = host(y0), host(y1)
    assert np.array_equal(bits(a), bits(b))
    ref = orc.gemm_q4(qs, sc, xs, n, threads=8, mode=1)
    ok, worst_rel, worst_abs = within_tolerance(b, ref)
    assert ok, (worst_rel, worst_abs)


# ------------------------------------------- the prefill chunk GEMM (5..512 tokens)

def gemm_f6s(qs, sc, xq, xsc, rows, cols, n):
    panel = torch.full((D.f6_panel_bytes(n, cols),), 0x7f, dtype=torch.uint8, device="cuda")
    D.pack_f6panel(dev(xq), dev(xsc), panel, n, cols)
    packed = torch.empty(D.q4_f6pack_bytes(rows, cols), dtype=torch.uint8, device="cuda")
    D.pack_q4_f6(dev(qs), dev(sc), packed, rows, cols)
    y = torch.full((n, rows), float("nan"), dtype=torch.float32, device="cuda")
    D.gemm_q4_f6s(packed, panel, y, rows, cols, n)
    return host(y)


@pytest.mark.parametrize("rows,cols,n", [(130, 256, 64), (33, 96, 5), (17, 2048, 16),
                                         (97, 1024, 33), (64, 512, 32), (40, 1568, 20)])
def test_chunk_gemm_block_dots_are_exact(gpu_ready, orc, rows, cols, n):
    """dnx_gemm_q4_f6s: scale 1 on one block and 0 on the others gives that
    block's exact dot, for every block (every |xq| up to 127, every nibble)."""
    rng = np.random.default_rng(rows + cols + n + 1)
    B = cols // 32
    xq = rng.integers(-127, 128, (n, cols), dtype=np.int8)
    xq[0, :32] = 127
    xq[-1, -32:] = -127
    qs = rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8)
    qs[0, :16] = 0x00
    qs[-1, -16:] = 0xff
    want = orc.block_dots_q4(qs, xq)
    for b in range(B):
        sw = np.zeros((rows, B), np.uint16)
        sw[:, b] = 0x3C00
        xsc = np.zeros((n, B), np.float32)
        xsc[:, b] = 1.0
        y = gemm_f6s(qs, sw, xq, xsc, rows, cols, n)
        assert np.array_equal(y, want[:, :, b].astype(np.float32)), f"block {b}"


def test_chunk_gemm_unit_scales_sum_blocks_exactly(gpu_ready, orc):
    rows, cols, n = 200, 4096, 64
    rng = np.random.default_rng(8)
    xq = rng.integers(-127, 128, (n, cols), dtype=np.int8)
    qs = rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8)
    want = orc.block_dots_q4(qs, xq).sum(axis=2)
    assert np.abs(want).max() < 2 ** 24
    y = gemm_f6s(qs, np.full((rows, cols // 32), np.uint16(0x3C00)), xq,
                 np.ones((n, cols // 32), np.float32), rows, cols, n)
    assert np.array_equal(y, want.astype(np.float32))


@pytest.mark.parametrize("rows,cols,n", [(6144, 2048, 64), (6144, 2048, 8), (2048, 6144, 33),
                                         (768, 768, 13), (97, 160, 5), (257, 2048, 32),
                                         (1152, 4320, 17), (100, 96, 64), (1792, 768, 48),
                                         (4304, 1152, 64), (768, 768, 375), (2048, 768, 130),
                                         (300, 1568, 24), (2048, 2048, 64), (1024, 1536, 7),
                                         (1792, 768, 375), (2304, 1024, 300), (10000, 1536, 40)])
def test_chunk_gemm_within_tolerance(gpu_ready, orc, rows, cols, n):
    """Against the exact products (error / sum|terms| below 1e-5) and the CPU
    kernel's outputs (relative 1e-4, absolute 1e-5 near zero); the same
    inputs twice give the same bits (a fixed order of the K parts)."""
    rng = np.random.default_rng(rows * 5 + cols + n)
    qs, sc = synth.q4_weights(rng, rows, cols)
    xs = synth.activations(rng, n, cols)
    xq, xsc = orc.quantize_q8(xs)
    ref = orc.gemm_q4(qs, sc, xs, n, threads=8, mode=1)
    y = gemm_f6s(qs, sc, xq, xsc, rows, cols, n)
    exact, mag = exact_products(orc, qs, sc, xq, xsc)
    assert np.all(np.abs(y - exact) <= 1e-5 * mag)
    ok, worst_rel, worst_abs = within_tolerance(y, ref)
    assert ok, (worst_rel, worst_abs)
    assert np.array_equal(bits(y), bits(gemm_f6s(qs, sc, xq, xsc, rows, cols, n)))


@pytest.mark.parametrize("rows_list,cols,n", [((2048, 1024, 1024), 2048, 13),
                                              ((6144, 6144), 2048, 64),
                                              ((1792, 256), 768, 375),
                                              ((97, 300, 33, 130), 160, 40),
                                              ((70,), 96, 5)])
def test_chunk_gemm_segments_equal_separate_launches(gpu_ready, orc, rows_list, cols, n):
    """dnx_gemm_q4_f6s_multi (one launch over up to four matrices reading one
    panel: a chunk's q, k, v or gate, up) gives every matrix the bits of its
    own dnx_gemm_q4_f6s, rows not multiples of 32 included."""
    rng = np.random.default_rng(sum(rows_list) + cols + n)
    xs = synth.activations(rng, n, cols)
    xq, xsc = orc.quantize_q8(xs)
    panel = torch.full((D.f6_panel_bytes(n, cols),), 0x7f, dtype=torch.uint8, device="cuda")
    D.pack_f6panel(dev(xq), dev(xsc), panel, n, cols)
    packs, ys, want = [], [], []
    for rows in rows_list:
        qs, sc = synth.q4_weights(rng, rows, cols)
        pk = torch.empty(D.q4_f6pack_bytes(rows, cols), dtype=torch.uint8, device="cuda")
        D.pack_q4_f6(dev(qs), dev(sc), pk, rows, cols)
        y1 = torch.full((n, rows), float("nan"), device="cuda")
        D.gemm_q4_f6s(pk, panel, y1, rows, cols, n)
        packs.append(pk)
        ys.append(torch.full((n, rows), float("nan"), device="cuda"))
        want.append(host(y1))
    D.gemm_q4_f6s_multi(packs, ys, list(rows_list), panel, cols, n)
    for k, rows in enumerate(rows_list):
        assert np.array_equal(bits(host(ys[k])), bits(want[k])), f"matrix {k} ({rows} rows)"


def test_chunk_gemm_refuses_bad_shapes(gpu_ready):
    z = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    y = torch.zeros(65 * 64, device="cuda")
    with pytest.raises(RuntimeError):
        D.gemm_q4_f6s(z, z, y, 64, 48, 5)    # cols not a multiple of 32
    with pytest.raises(RuntimeError):
        D.gemm_q4_f6s(z, z, y, 64, 64, 0)    # no tokens


# --------------------------------------------- Q8 weights on the fp6 GEMM

def gemm_q8_f6(qs, sc, xq, xsc, rows, cols, n):
    panel = torch.full((D.f6_panel_bytes(n, cols),), 0x7f, dtype=torch.uint8, device="cuda")
    D.pack_f6panel(dev(xq), dev(xsc), panel, n, cols)
    packed = torch.empty(D.q8_f6pack_bytes(rows, cols), dtype=torch.uint8, device="cuda")
    D.pack_q8_f6(dev(qs), dev(sc), packed, rows, cols)
    y = torch.full((n, rows), float("nan"), dtype=torch.float32, device="cuda")
    D.gemm_q8_f6p(packed, panel, y, rows, cols, n)
    return host(y)


@pytest.mark.parametrize("rows,cols,n", [(130, 256, 70), (33, 96, 5), (97, 1024, 131),
                                         (200, 320, 300)])
def test_q8_block_dots_are_exact(gpu_ready, orc, rows, cols, n):
    """Scale 1 on one block and 0 on the others: y is that block's exact dot
    sum_k xq * w, for every block, against brute force. The weights cover
    every int8 value including -128 (two fp6 digits: 8 * 15 + 8), the
    activations every |xq| up to 127."""
    rng = np.random.default_rng(rows + cols + n + 3)
    B = cols // 32
    xq = rng.integers(-127, 128, (n, cols), dtype=np.int8)
    xq[0, :32] = 127
    xq[-1, -32:] = -127
    qs = rng.integers(-128, 128, (rows, cols), dtype=np.int16).astype(np.int8)
    qs[0, :32] = -128
    qs[-1, -32:] = 127
    qs[1 % rows, :256 if cols >= 256 else cols] = np.arange(-128, 128, dtype=np.int16)[:min(cols, 256)].astype(np.int8)
    want = orc.block_dots_q8(qs, xq)
    for b in range(B):
        sw = np.zeros((rows, B), np.float32)
        sw[:, b] = 1.0
        xsc = np.zeros((n, B), np.float32)
        xsc[:, b] = 1.0
        y = gemm_q8_f6(qs, sw, xq, xsc, rows, cols, n)
        assert np.array_equal(y, want[:, :, b].astype(np.float32)), f"block {b}"


def test_q8_power_of_two_scales_are_exact(gpu_ready, orc):
    """Scales that are powers of two (both exponents ride in the MFMAs' E8M0
    scales, the mantissas are 1): every term exact; only the fp32 rounding of
    the running sum remains."""
    rows, cols, n = 64, 512, 96
    rng = np.random.default_rng(12)
    B = cols // 32
    xq = rng.integers(-127, 128, (n, cols), dtype=np.int8)
    qs = rng.integers(-127, 128, (rows, cols), dtype=np.int8)
    ex = rng.integers(-20, 10, (n, B))
    ew = rng.integers(-30, 30, (rows, B))
    xsc = np.ldexp(np.ones((n, B)), ex).astype(np.float32)
    sw = np.ldexp(np.ones((rows, B)), ew).astype(np.float32)
    d = orc.block_dots_q8(qs, xq).astype(np.float64)
    terms = d * np.ldexp(1.0, ex)[:, None, :] * np.ldexp(1.0, ew)[None, :, :]
    y = gemm_q8_f6(qs, sw, xq, xsc, rows, cols, n)
    assert np.max(np.abs(y - terms.sum(axis=2)) / np.abs(terms).sum(axis=2)) < 2 ** -20


@pytest.mark.parametrize("rows,cols,n,fp32_scales", [(4304, 1152, 1024, True),
                                                     (1152, 4320, 1024, True),
                                                     (1024, 1024, 1024, False),
                                                     (70, 96, 13, True), (128, 128, 40, False),
                                                     (97, 160, 129, True),
                                                     (2048, 4096, 256, False),
                                                     (300, 8192, 64, True)])
def test_q8_gemm_within_tolerance(gpu_ready, orc, rows, cols, n, fp32_scales):
    """Against the exact products (error / sum|terms| below 1e-5) and the CPU
    kernel's outputs (relative 1e-4, absolute 1e-5 near zero): GGUF-style
    fp16-exact scales, and weights quantized by lab_quantize_q8 (the vision
    encoder's BF16 -> Q8 path), whose fp32 scales use both mantissa pieces."""
    rng = np.random.default_rng(rows * 7 + cols + n)
    if fp32_scales:
        qs, sc = orc.quantize_q8((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
    else:
        # GGUF-style fp16 scales at the size of real weights (|w| near 0.02):
        # the synthetic scales / 16, still fp16 values. At the synthetic
        # size itself (|w| up to 3.8) outputs reach ~20, where two fp32 sums
        # in different orders differ by more than the 1e-5 absolute bar.
        qs, sc = synth.q8_weights(rng, rows, cols)
        sc = (sc / np.float32(16)).astype(np.float16).astype(np.float32)
    xs = synth.activations(rng, n, cols)
    xq, xsc = orc.quantize_q8(xs)
    ref = orc.gemm_q8(qs, sc, xs, n, threads=8, mode=1)
    y = gemm_q8_f6(qs, sc, xq, xsc, rows, cols, n)
    d = orc.block_dots_q8(qs, xq).astype(np.float64)
    s = (sc[None, :, :].astype(np.float32) * xsc[:, None, :]).astype(np.float32).astype(np.float64)
    exact, mag = (d * s).sum(axis=2), np.abs(d * s).sum(axis=2)
    assert np.all(np.abs(y - exact) <= 1e-5 * mag)
    ok, worst_rel, worst_abs = within_tolerance(y, ref)
    assert ok, (worst_rel, worst_abs)


# --------------------------- producers that write the panel of their output

def token_records(panel, n, cols):
    """The panel bytes of tokens 0..n-1 (their four 16-byte lane-record
    pieces and their C value per block), as one array per token."""
    p = host(panel).view(np.uint8)
    B = cols // 32
    out = []
    for t in range(n):
        g, r = divmod(t, 32)
        parts = []
        for b in range(B):
            rec = (g * B + b) * 2176
            for off in (r * 16, (32 + r) * 16, 1024 + r * 16, 1024 + (32 + r) * 16):
                parts.append(p[rec + off:rec + off + 16])
            c = 2048 + ((((r >> 2) & 1) * 16 + (r >> 3) * 4 + (r & 3)) * 4)
            parts.append(p[rec + c:rec + c + 4])
        out.append(np.concatenate(parts))
    return np.stack(out)


@pytest.mark.parametrize("n,cols", [(64, 6144), (13, 2048), (5, 96), (33, 1024)])
def test_swiglu_panel_equals_swiglu_then_quantizer(gpu_ready, n, cols):
    """dnx_swiglu_f6panel: h = SiLU(g) * u in place with swiglu's bits, and
    the panel dnx_quantize_q8_f6panel makes from h (padding tokens too)."""
    rng = np.random.default_rng(n + cols)
    g = (rng.standard_normal((n, cols)) * 2).astype(np.float32)
    u = rng.standard_normal((n, cols)).astype(np.float32)
    g1, g2, ud = dev(g), dev(g), dev(u)
    p1 = torch.full((D.f6_panel_bytes(n, cols),), 0x7f, dtype=torch.uint8, device="cuda")
    p2 = p1.clone()
    D.swiglu(g1, ud)
    D.quantize_q8_f6panel(g1, p1, n, cols)
    D.swiglu_f6panel(g2, ud, p2, n, cols)
    assert np.array_equal(bits(host(g2)), bits(host(g1)))
    assert np.array_equal(host(p2), host(p1))


@pytest.mark.parametrize("add", [False, True])
@pytest.mark.parametrize("n,cols", [(64, 2048), (13, 2048), (5, 4096), (33, 96), (256, 1024)])
def test_norm_panel_equals_norm_then_quantizer(gpu_ready, n, cols, add):
    """dnx_rms_norm_f6panel / dnx_add_rms_norm_f6panel: the norm's outputs
    (and the residual sum) with the unfused kernels' bits, and every live
    token's panel records as dnx_quantize_q8_f6panel makes them from the
    normed rows."""
    rng = np.random.default_rng(n * 3 + cols + add)
    x = rng.standard_normal((n, cols)).astype(np.float32)
    m = rng.standard_normal((n, cols)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    eps = 1e-6
    xa, xb, md, wd = dev(x), dev(x), dev(m), dev(w)
    o1 = torch.empty((n, cols), device="cuda")
    o2 = torch.empty((n, cols), device="cuda")
    p1 = torch.full((D.f6_panel_bytes(n, cols),), 0x7f, dtype=torch.uint8, device="cuda")
    p2 = p1.clone()
    if add:
        D.add_rms_norm(md, xa, wd, o1, n, cols, eps)
        D.add_rms_norm_f6panel(md, xb, wd, o2, p2, n, cols, eps)
        assert np.array_equal(bits(host(xb)), bits(host(xa)))
    else:
        D.rms_norm(xa, wd, o1, n, cols, eps)
        D.rms_norm_f6panel(xb, wd, o2, p2, n, cols, eps)
    D.quantize_q8_f6panel(o1, p1, n, cols)
    assert np.array_equal(bits(host(o2)), bits(host(o1)))
    assert np.array_equal(token_records(p2, n, cols), token_records(p1, n, cols))


@pytest.mark.parametrize("n,position,heads,kv_heads,hd,gated,window",
                         [(64, 256, 16, 8, 128, False, 0), (13, 600, 8, 2, 64, True, 0),
                          (37, 300, 8, 8, 128, False, 128), (64, 900, 32, 8, 128, True, 0)])
def test_attention_panel_equals_attention_then_quantizer(gpu_ready, n, position, heads,
                                                         kv_heads, hd, gated, window):
    """dnx_attention_f6panel on the split matrix-core path: out with
    dnx_attention's bits, and every live token's panel records as
    dnx_quantize_q8_f6panel makes them from out ([n][heads * hd])."""
    rng = np.random.default_rng(n + position + hd)
    cols, kv = heads * hd, kv_heads * hd
    q = dev(rng.standard_normal((n, cols)).astype(np.float32))
    keys = dev(rng.standard_normal((position + n, kv)).astype(np.float32))
    values = dev(rng.standard_normal((position + n, kv)).astype(np.float32))
    gate = dev(rng.standard_normal((n, heads)).astype(np.float32)) if gated else None
    o1 = torch.full((n, cols), np.nan, device="cuda")
    o2 = o1.clone()
    p1 = torch.full((D.f6_panel_bytes(n, cols),), 0x7f, dtype=torch.uint8, device="cuda")
    p2 = p1.clone()
    D.attention(q, keys, values, gate, o1, position, n, heads, kv_heads, hd, window)
    rc = D.attention_f6panel(q, keys, values, gate, o2, p2, position, n, heads, kv_heads, hd,
                             window)
    assert rc == 0
    D.quantize_q8_f6panel(o1, p1, n, cols)
    assert np.array_equal(bits(host(o2)), bits(host(o1)))
    assert np.array_equal(token_records(p2, n, cols), token_records(p1, n, cols))


@pytest.mark.parametrize("n,position,hd", [(8, 0, 128), (4, 500, 128), (16, 300, 32)])
def test_attention_panel_refused_off_the_split_path(gpu_ready, n, position, hd):
    """Where the attention does not run its split matrix-core path (a short
    context, fewer than 8 tokens, hd not 64 or 128), dnx_attention_f6panel
    returns DNX_EINVAL and launches nothing."""
    heads, kv_heads = 8, 4
    rng = np.random.default_rng(n + position)
    cols, kv = heads * hd, kv_heads * hd
    q = dev(rng.standard_normal((n, cols)).astype(np.float32))
    keys = dev(rng.standard_normal((position + n, kv)).astype(np.float32))
    values = dev(rng.standard_normal((position + n, kv)).astype(np.float32))
    out = torch.full((n, cols), 7.0, device="cuda")
    panel = torch.full((D.f6_panel_bytes(n, cols),), 0x7f, dtype=torch.uint8, device="cuda")
    rc = D.attention_f6panel(q, keys, values, None, out, panel, position, n, heads, kv_heads, hd)
    assert rc == -1
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
    assert bool((panel == 0x7f).all())
