"""Q6_K super-blocks for the adapter's tests.

`pack_q6k` packs known 6-bit values the way ggml's quantize_row_q6_K does,
the inverse of dequantize_row_q6_K that lib/src/gguf.dart:220-254 follows.
Per 128 values j..j+127 of a super-block and l < 32, with
q1..q4 = values l, l+32, l+64, l+96:
ql[l] = q1 & 15 | (q3 & 15) << 4, ql[l + 32] = q2 & 15 | (q4 & 15) << 4,
qh[l] = q1 >> 4 | (q2 >> 4) << 2 | (q3 >> 4) << 4 | (q4 >> 4) << 6, then
ql += 64, qh += 32; sc[i] scales values 16i..16i+15; the fp16 d comes last
(210 bytes). `expected_values` is the definition of each value,
d * sc * (q - 32), computed with numpy's own fp16 widening. Decoding packed
values and comparing with the definition pins the decoder's bit layout.
"""

import numpy as np


def pack_q6k(q, sc, d_bits):
    """q: [blocks][256] in 0..63; sc: int8 [blocks][16]; d_bits: uint16 [blocks]."""
    q = np.asarray(q, np.uint8).reshape(-1, 256)
    nb = q.shape[0]
    out = np.zeros((nb, 210), np.uint8)
    for h in (0, 1):
        v = q[:, 128 * h: 128 * h + 128]
        q1, q2, q3, q4 = v[:, 0:32], v[:, 32:64], v[:, 64:96], v[:, 96:128]
        out[:, 64 * h: 64 * h + 32] = (q1 & 15) | ((q3 & 15) << 4)
        out[:, 64 * h + 32: 64 * h + 64] = (q2 & 15) | ((q4 & 15) << 4)
        out[:, 128 + 32 * h: 160 + 32 * h] = ((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4)
                                              | ((q4 >> 4) << 6))
    out[:, 192:208] = np.asarray(sc, np.int8).reshape(nb, 16).view(np.uint8)
    d = np.asarray(d_bits, np.uint16).reshape(nb)
    out[:, 208] = (d & 0xFF).astype(np.uint8)
    out[:, 209] = (d >> 8).astype(np.uint8)
    return out


def expected_values(q, sc, d_bits):
    """d * sc[v // 16] * (q[v] - 32), exact in float64, rounded once to float32."""
    q = np.asarray(q, np.int64).reshape(-1, 256)
    d = np.asarray(d_bits, np.uint16).reshape(-1).view(np.float16).astype(np.float64)
    s = np.repeat(np.asarray(sc, np.int8).reshape(-1, 16).astype(np.float64), 16, axis=1)
    with np.errstate(invalid="ignore"):
        return (d[:, None] * s * (q - 32).astype(np.float64)).astype(np.float32).reshape(-1)


def random_blocks(rng, count, specials=True):
    """Random 6-bit values, int8 scales and fp16 d of realistic size; with
    `specials`, some d are 0, subnormal, negative, infinite or NaN."""
    q = rng.integers(0, 64, size=(count, 256), dtype=np.uint8)
    sc = rng.integers(-128, 128, size=(count, 16)).astype(np.int8)
    d = (np.abs(rng.standard_normal(count)) * 0.002).astype(np.float16).view(np.uint16)
    if specials and count >= 8:
        d[:8] = [0x0000, 0x8000, 0x0001, 0x03FF, 0xBC00, 0x7C00, 0x7E00, 0x7BFF]
    return q, sc, d
