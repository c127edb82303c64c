"""The CPU oracle pinned against the reference's own kernels (CPU only).

Every function of oracle/lab_oracle.c is checked against:
* the golden vectors in tests/golden/ (written by the compiled reference
  src/c/lab_native.c, see make_golden.py);
* the compiled reference itself (oracle/_ref) on fresh seeded inputs, when
  that library is present;
* closed forms: quantizer edge cases, exhaustive fp16 conversions,
  brute-force integer block dots, argmax ties and NaN, SiLU and GELU
  identities.
"""

import glob
import math
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("name", ["edges", "random"])
def test_quantize_q8_matches_golden(orc, name):
    d = np.load(os.path.join(GOLDEN, f"quantize_q8_{name}.npz"))
    qs, sc = orc.quantize_q8(d["x"])
    assert np.array_equal(qs, d["qs"])
    assert np.array_equal(bits(sc), bits(d["scales"]))


@pytest.mark.parametrize("name", ["quantize_q4", "quantize_q4_edges"])
def test_quantize_q4_matches_golden(orc, name):
    d = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    qs, sc = orc.quantize_q4(d["x"])
    assert np.array_equal(qs, d["qs"])
    assert np.array_equal(sc, d["scales"])


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "gemm_*.npz"))),
                         ids=lambda p: os.path.basename(p)[:-4])
@pytest.mark.parametrize("mode", [0, 1])
def test_gemm_matches_golden(orc, path, mode):
    d = np.load(path)
    q4 = os.path.basename(path).startswith("gemm_q4")
    n = d["xs"].shape[0]
    f = orc.gemm_q4 if q4 else orc.gemm_q8
    for threads in (1, 3):
        y = f(d["qs"], d["scales"], d["xs"], n, threads=threads, mode=mode)
        assert np.array_equal(bits(y), bits(d[f"y_mode{mode}"]))


def test_quantizer_closed_forms(orc):
    # scale 1 (amax 127): q = round half away from zero, in float.
    x = np.zeros((1, 32), np.float32)
    x[0, :7] = [127.0, -127.0, 0.49999997, 2.5, -2.5, 0.5, -0.5]
    qs, sc = orc.quantize_q8(x)
    assert sc[0, 0] == 1.0
    assert list(qs[0, :7]) == [127, -127, 1, 3, -3, 1, -1]
    # all-zero block: scale 0, q 0
    qs, sc = orc.quantize_q8(np.zeros((2, 64), np.float32))
    assert not qs.any() and not sc.any()
    # scale is amax / 127 correctly rounded; every |q| <= 127
    rng = np.random.default_rng(7)
    x = rng.standard_normal((64, 128)).astype(np.float32)
    qs, sc = orc.quantize_q8(x)
    amax = np.abs(x.reshape(64, 4, 32)).max(axis=2)
    assert np.array_equal(bits(sc), bits((amax / np.float32(127)).astype(np.float32)))
    assert np.abs(qs.astype(int)).max() <= 127
    # dequantized values within half a step of the input
    deq = qs.reshape(64, 4, 32).astype(np.float64) * sc[..., None]
    assert np.all(np.abs(deq - x.reshape(64, 4, 32)) <= sc[..., None] * 0.5 * (1 + 1e-6))


def test_padded_quantizer_is_the_padded_problem(orc):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 4304)).astype(np.float32)
    qs, sc = orc.quantize_q8_padded(x, 4320)
    xp = np.zeros((5, 4320), np.float32)
    xp[:, :4304] = x
    qs2, sc2 = orc.quantize_q8(xp)
    assert np.array_equal(qs, qs2) and np.array_equal(bits(sc), bits(sc2))
    assert not qs[:, 4304:].any()


def test_bf16_quantizer_is_widen_then_quantize(orc):
    from dianoia_amd.formats import widen_bf16
    from dianoia_amd.synth import bf16_rne
    rng = np.random.default_rng(4)
    w = bf16_rne(rng.standard_normal((7, 1152)).astype(np.float32) * np.float32(0.02))
    qs, sc = orc.quantize_q8_bf16(w)
    qs2, sc2 = orc.quantize_q8(widen_bf16(w))
    assert np.array_equal(qs, qs2) and np.array_equal(bits(sc), bits(sc2))


def test_q6k_dequantizer_against_ggml_packing(orc):
    """dequantizeQ6K (gguf.dart:220-254) on values packed by ggml's
    quantize_row_q6_K layout equals the definition d * sc * (q - 32)."""
    from q6k_util import expected_values, pack_q6k, random_blocks
    rng = np.random.default_rng(61)
    q, sc, d = random_blocks(rng, 64)
    # every 6-bit value in every position of one block, extreme scales
    q[8] = np.arange(256) % 64
    sc[8] = [-128, 127, -1, 1, 0, 5, -7, 64, -64, 100, -100, 3, 2, -2, 126, -127]
    got = orc.dequantize_q6k(pack_q6k(q, sc, d))
    want = expected_values(q, sc, d)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits(got[~nan]), bits(want[~nan]))


def test_q6k_adapter_is_dequantize_then_quantize(orc):
    from q6k_util import pack_q6k, random_blocks
    rows, cols = 5, 512
    q, sc, d = random_blocks(np.random.default_rng(62), rows * cols // 256)
    blocks = pack_q6k(q, sc, d)
    qs, s = orc.q6k_to_q8(blocks, rows, cols)
    q2, s2 = orc.quantize_q8(orc.dequantize_q6k(blocks).reshape(rows, cols))
    assert np.array_equal(qs, q2)
    assert np.array_equal(bits(s), bits(s2))


def test_half_conversions_exhaustive(orc):
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([orc.half_to_float(int(v)) for v in h], dtype=np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(bits(got)[finite], bits(want)[finite])
    assert np.all(np.isnan(got[~np.isfinite(want) & np.isnan(want)]))
    # float -> half round trip and RNE against numpy's conversion
    f = np.concatenate([want[finite], np.float32([1e-8, 6.1e-5, 65519.0, 65520.0, 1e6, -1e-9])])
    f = np.concatenate([f, (f * np.float32(1.0009765)).astype(np.float32)])
    got_h = np.array([orc.float_to_half(float(v)) for v in f], dtype=np.uint16)
    assert np.array_equal(got_h, f.astype(np.float16).view(np.uint16))


def test_block_dots_brute_force(orc):
    rng = np.random.default_rng(9)
    qs = rng.integers(-127, 128, (6, 96), dtype=np.int8)
    xq = rng.integers(-127, 128, (3, 96), dtype=np.int8)
    d = orc.block_dots_q8(qs, xq)
    want = np.einsum("rbk,tbk->trb", qs.reshape(6, 3, 32).astype(np.int64),
                     xq.reshape(3, 3, 32).astype(np.int64))
    assert np.array_equal(d, want)
    q4 = rng.integers(0, 256, (6, 48), dtype=np.uint8)
    w = np.empty((6, 96), np.int64)
    blocks = q4.reshape(6, 3, 16).astype(np.int64)
    w.reshape(6, 3, 32)[:, :, :16] = (blocks & 15) - 8
    w.reshape(6, 3, 32)[:, :, 16:] = (blocks >> 4) - 8
    d4 = orc.block_dots_q4(q4, xq)
    assert np.array_equal(d4, np.einsum("rbk,tbk->trb", w.reshape(6, 3, 32),
                                        xq.reshape(3, 3, 32).astype(np.int64)))


def test_mode1_products_against_exact_sums(orc):
    # y = sum_b s_b * d_b within fp32 rounding of the exact double sum
    rng = np.random.default_rng(11)
    w = (rng.random((9, 512)) - 0.5).astype(np.float32)
    xs = (rng.random((2, 512)) * 2 - 1).astype(np.float32)
    qs, sc = orc.quantize_q8(w)
    y = orc.gemm_q8(qs, sc, xs, 2, threads=1, mode=1)
    xq, xsc = orc.quantize_q8(xs)
    d = orc.block_dots_q8(qs, xq).astype(np.float64)
    exact = (d * sc[None].astype(np.float64) * xsc[:, None, :]).sum(axis=2)
    mag = (np.abs(d) * sc[None] * xsc[:, None, :]).sum(axis=2)
    assert np.all(np.abs(y - exact) <= 1e-6 * mag + 1e-30)


def test_argmax_closed_forms(orc):
    assert orc.argmax(np.float32([1, 3, 3, 2])) == 1            # first of a tie
    assert orc.argmax(np.float32([-0.0, 0.0])) == 0             # -0 == +0
    assert orc.argmax(np.float32([np.nan, 5, 7])) == 0          # NaN at 0 stays
    assert orc.argmax(np.float32([1, np.nan, 0.5])) == 0        # NaN never wins
    assert orc.argmax(np.float32([1, np.nan, 4])) == 2
    assert orc.argmax(np.float32([-np.inf, -1e38])) == 1
    rng = np.random.default_rng(5)
    v = rng.standard_normal(100001).astype(np.float32)
    assert orc.argmax(v) == int(np.argmax(v))


def test_silu_glue_closed_forms(orc):
    rng = np.random.default_rng(12)
    g = rng.standard_normal(4096).astype(np.float32) * 4
    u = rng.standard_normal(4096).astype(np.float32)
    h = orc.silu_mul(g, u)
    gd = g.astype(np.float64)
    silu = (gd / (1 + np.exp(-gd))).astype(np.float32)
    assert np.array_equal(bits(h), bits((silu * u).astype(np.float32)))
    assert orc.silu_mul(np.float32([0.0]), np.float32([3.0]))[0] == 0.0
    big = orc.silu_mul(np.float32([30.0]), np.float32([1.0]))[0]
    assert abs(big - 30.0) < 1e-5


def test_gelu_closed_forms(orc):
    x = np.linspace(-6, 6, 2001).astype(np.float32)
    y = orc.gelu(x).astype(np.float64)
    exact = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in x.astype(np.float64)])
    # A&S 7.1.26 has |error| <= 1.5e-7 in erf
    assert np.all(np.abs(y - exact) <= 0.5 * np.abs(x) * 1.6e-7 + 6e-8 * np.abs(exact) + 1e-30)
    assert orc.gelu(np.float32([0.0]))[0] == 0.0
    # gelu(x) - gelu(-x) = x (erf is odd)
    assert np.allclose(orc.gelu(x) - orc.gelu(-x), x, atol=2e-6)


@pytest.mark.skipif(not O.reference_available(), reason="oracle/_ref not built (no reference)")
@pytest.mark.parametrize("fmt", ["q8", "q4"])
def test_oracle_matches_compiled_reference(orc, fmt):
    ref = O.Reference()
    rng = np.random.default_rng(21)
    for rows, cols, n in [(37, 2048, 3), (130, 1152, 2), (8, 6144, 1), (64, 4320, 4)]:
        w = (rng.random((rows, cols), dtype=np.float32) - 0.5).astype(np.float32)
        xs = rng.standard_normal((n, cols), dtype=np.float32)
        if fmt == "q8":
            qs, sc = ref.quantize_q8(w)
            q2, s2 = orc.quantize_q8(w)
            assert np.array_equal(qs, q2) and np.array_equal(bits(sc), bits(s2))
            for mode in (0, 1):
                a = ref.gemm_q8(qs, sc, xs, n, threads=4, mode=mode)
                b = orc.gemm_q8(qs, sc, xs, n, threads=2, mode=mode)
                assert np.array_equal(bits(a), bits(b))
        else:
            qs, sc = ref.quantize_q4(w)
            q2, s2 = orc.quantize_q4(w)
            assert np.array_equal(qs, q2) and np.array_equal(sc, s2)
            for mode in (0, 1):
                a = ref.gemm_q4(qs, sc, xs, n, threads=4, mode=mode)
                b = orc.gemm_q4(qs, sc, xs, n, threads=2, mode=mode)
                assert np.array_equal(bits(a), bits(b))


# ---- layer steps (Metal shader semantics): closed forms and invariants

def test_rms_norm_closed_forms(orc):
    cols = 96
    x = np.stack([np.full(cols, 3.0, np.float32), np.full(cols, -0.5, np.float32),
                  np.random.default_rng(3).standard_normal(cols).astype(np.float32)])
    ones = np.ones(cols, np.float32)
    y = orc.rms_norm(x, ones, 0.0)
    assert np.allclose(y[0], 1.0, rtol=2e-7) and np.allclose(y[1], -1.0, rtol=2e-7)
    assert abs(np.sqrt(np.mean(y[2].astype(np.float64) ** 2)) - 1.0) < 1e-6  # unit RMS
    eps = np.float32(0.25)
    ye = orc.rms_norm(x[:1], ones, float(eps))
    assert np.allclose(ye, 3.0 / np.sqrt(9.0 + 0.25), rtol=2e-7)  # mean(x^2) + eps
    w = np.linspace(-2, 2, cols).astype(np.float32)
    assert np.array_equal(orc.rms_norm(x, 2 * w, 1e-6), 2 * orc.rms_norm(x, w, 1e-6))
    base = np.full_like(x, 0.5)
    acc = orc.rms_norm(x, w, 1e-6, out=base)
    assert np.array_equal(acc, base + orc.rms_norm(x, w, 1e-6))


def test_head_norm_rope_invariants(orc):
    heads, hd, n = 3, 16, 2
    rng = np.random.default_rng(4)
    x = rng.standard_normal((n, heads * hd)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    pair = hd // 2
    ident = np.concatenate([np.ones(pair), np.zeros(pair)]).astype(np.float32)
    ident = np.tile(ident, (n, 1))
    y = orc.head_norm_rope(x, heads * hd, w, ident, hd, heads, hd, n, 1e-6)
    normed = orc.rms_norm(x.reshape(n * heads, hd), w, 1e-6).reshape(n, heads * hd)
    assert np.array_equal(y, normed)  # cos 1, sin 0: the norm alone
    quarter = np.tile(np.concatenate([np.zeros(pair), np.ones(pair)]).astype(np.float32), (n, 1))
    z = orc.head_norm_rope(x, heads * hd, w, quarter, hd, heads, hd, n, 1e-6)
    nr = normed.reshape(n, heads, 2, pair)
    assert np.array_equal(z.reshape(n, heads, 2, pair)[:, :, 0], -nr[:, :, 1])  # j <- -(j + hd/2)
    assert np.array_equal(z.reshape(n, heads, 2, pair)[:, :, 1], nr[:, :, 0])
    ang = rng.uniform(0, 6.3, (n, pair))
    table = np.concatenate([np.cos(ang), np.sin(ang)], axis=1).astype(np.float32)
    r = orc.head_norm_rope(x, heads * hd, w, table, hd, heads, hd, n, 1e-6).reshape(n, heads, 2, pair)
    # a rotation keeps each pair's length
    assert np.allclose((r ** 2).sum(axis=2), (nr ** 2).sum(axis=2), rtol=1e-5)


def test_short_conv_closed_forms(orc):
    width, k, n = 5, 3, 6
    rng = np.random.default_rng(5)
    bcx = rng.standard_normal((n, 3, width)).astype(np.float32)
    weight = rng.standard_normal((width, k)).astype(np.float32)
    hist = rng.standard_normal((k - 1, width)).astype(np.float32)
    y, h2 = orc.short_conv(bcx, weight, hist, width, k, n)
    # z = B * X; a causal conv of [history; z] with the kernel reversed; y = C * conv
    z = (bcx[:, 0] * bcx[:, 2]).astype(np.float64)
    full = np.concatenate([hist.astype(np.float64), z])
    for ch in range(width):
        conv = np.convolve(full[:, ch], weight[ch, ::-1].astype(np.float64), mode="valid")
        assert np.allclose(y.reshape(n, width)[:, ch], bcx[:, 1, ch] * conv, rtol=1e-5, atol=1e-6)
    assert np.array_equal(h2, z[-(k - 1):].astype(np.float32))  # the last k - 1 z
    # two calls carrying the history equal one call
    y1, hmid = orc.short_conv(bcx[:2], weight, hist, width, k, 2)
    y2, hend = orc.short_conv(bcx[2:], weight, hmid, width, k, n - 2)
    assert np.array_equal(np.concatenate([y1, y2]), y) and np.array_equal(hend, h2)


def test_attention_closed_forms(orc):
    heads, kv, hd, pos, n = 4, 2, 8, 5, 2
    rng = np.random.default_rng(6)
    total = pos + n
    q = rng.standard_normal(n * heads * hd).astype(np.float32)
    vals = rng.standard_normal((total, kv * hd)).astype(np.float32)
    same = np.tile(rng.standard_normal(kv * hd).astype(np.float32), (total, 1))
    out = orc.attention(q, same, vals, None, pos, n, heads, kv, hd).reshape(n, heads, hd)
    for t in range(n):  # equal keys: the mean of the visible values, KV head h // 2
        for h in range(heads):
            want = vals[: pos + t + 1, (h // 2) * hd:(h // 2 + 1) * hd].astype(np.float64).mean(0)
            assert np.allclose(out[t, h], want, rtol=1e-5, atol=1e-6)
    keys = rng.standard_normal((total, kv * hd)).astype(np.float32)
    one = orc.attention(q, keys, vals, None, pos, n, heads, kv, hd, window=1).reshape(n, heads, hd)
    for t in range(n):  # window 1: the token's own value
        for h in range(heads):
            assert np.allclose(one[t, h], vals[pos + t, (h // 2) * hd:(h // 2 + 1) * hd], rtol=1e-6)
    gate = rng.standard_normal(n * heads).astype(np.float32)
    gated = orc.attention(q, keys, vals, gate, pos, n, heads, kv, hd).reshape(n, heads, hd)
    plain = orc.attention(q, keys, vals, None, pos, n, heads, kv, hd).reshape(n, heads, hd)
    sig = 1.0 / (1.0 + np.exp(-gate.astype(np.float64).reshape(n, heads, 1)))
    assert np.allclose(gated, plain * sig, rtol=1e-6, atol=1e-7)
    # a window of 3 ignores the keys and values before it
    k2, v2 = keys.copy(), vals.copy()
    k2[:pos + 1 - 3] = 100.0
    v2[:pos + 1 - 3] = -100.0
    a = orc.attention(q, keys, vals, None, pos, n, heads, kv, hd, window=3)
    b = orc.attention(q, k2, v2, None, pos, n, heads, kv, hd, window=3)
    assert np.array_equal(a, b)
    # two keys: weights in the ratio exp((q.k0 - q.k1) / sqrt(hd))
    qq = rng.standard_normal(kv * hd).astype(np.float32)[:hd]
    kk = rng.standard_normal((2, hd)).astype(np.float32)
    vv = rng.standard_normal((2, hd)).astype(np.float32)
    o = orc.attention(qq, kk, vv, None, 1, 1, 1, 1, hd)
    s = kk.astype(np.float64) @ qq.astype(np.float64) / np.sqrt(hd)
    p = np.exp(s - s.max()) / np.exp(s - s.max()).sum()
    assert np.allclose(o, p @ vv.astype(np.float64), rtol=1e-5, atol=1e-6)


def test_steer_closed_forms(orc):
    rng = np.random.default_rng(7)
    v = rng.standard_normal(64)
    v = (v / np.linalg.norm(v)).astype(np.float32)
    u = rng.standard_normal(64)
    u = (u - (u @ v) * v).astype(np.float32)  # orthogonal to v
    x = np.stack([u + 3.0 * v, u - 0.5 * v]).astype(np.float32)
    assert np.array_equal(orc.steer(x, v, 0, 1.0), x + v)
    removed = orc.steer(x, v, 1, 1.0)
    assert np.allclose(removed, np.stack([u, u]), atol=1e-5)
    half = orc.steer(x, v, 1, 0.5)
    assert np.allclose(half[0], u + 1.5 * v, atol=1e-5)


def test_gguf_split_q8_0_scale_widening(orc):
    # halfToDouble (native.dart:871-880) on hand-worked patterns, and every
    # non-NaN pattern against numpy's IEEE binary16 conversion.
    cases = {0x3C00: 1.0, 0xC000: -2.0, 0x0001: 2.0 ** -24, 0x03FF: 1023 * 2.0 ** -24,
             0x0400: 2.0 ** -14, 0x3555: 0.333251953125, 0x7BFF: 65504.0,
             0x7C00: math.inf, 0xFC00: -math.inf}
    pats = np.array(list(cases) + [0x8000, 0x7C01, 0xFE00, 0x7FFF], np.uint16)
    blocks = np.zeros((pats.size, 34), np.uint8)
    blocks[:, 0], blocks[:, 1] = pats & 0xFF, pats >> 8
    blocks[:, 2:] = np.arange(32, dtype=np.uint8) + 100
    qs, sc = orc.split_q8_0(blocks, pats.size)
    for i, want in enumerate(cases.values()):
        assert sc[i] == want
    assert sc[len(cases)] == 0 and math.copysign(1, sc[len(cases)]) < 0  # -0 kept
    assert np.all(sc[len(cases) + 1:].view(np.uint32) == 0x7FC00000)   # double.nan
    assert np.array_equal(qs.view(np.uint8).reshape(-1, 32), blocks[:, 2:])
    allp = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    allp = allp[~np.isnan(allp.view(np.float16))]
    b = np.zeros((allp.size, 34), np.uint8)
    b[:, 0], b[:, 1] = allp & 0xFF, allp >> 8
    _, sc = orc.split_q8_0(b, allp.size)
    assert np.array_equal(sc.view(np.uint32),
                          allp.view(np.float16).astype(np.float32).view(np.uint32))


def test_gguf_split_q4_0_is_a_byte_split(orc):
    rng = np.random.default_rng(4)
    blocks = rng.integers(0, 256, (5, 18), dtype=np.uint8)
    qs, d = orc.split_q4_0(blocks, 5)
    assert np.array_equal(qs.reshape(5, 16), blocks[:, 2:])
    assert np.array_equal(d, blocks[:, 0].astype(np.int64) + 256 * blocks[:, 1].astype(np.int64))
