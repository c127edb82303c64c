"""Host-side formats on the path (CPU): GGUF splits, BF16 widening, fp16."""

import numpy as np
import pytest

from dianoia_amd import ArgumentError
from dianoia_amd.formats import (QuantMatrix, float_to_half, half_to_float, join_q4_0,
                                 join_q8_0, split_q4_0, split_q8_0, widen_bf16)
from dianoia_amd.synth import bf16_rne


def test_split_q8_0_keeps_bytes_and_widens_d_exactly():
    # qwen3_gguf_test.dart:13-29: values (i - 20) / 16 quantized as Q8_0
    values = ((np.arange(64) - 20) / 16).astype(np.float32)
    d = np.abs(values.reshape(2, 32)).max(axis=1) / 127
    d_bits = d.astype(np.float16).view(np.uint16)
    qs = np.round(values.reshape(2, 32) / d_bits.view(np.float16).astype(np.float32)[:, None])
    qs = qs.astype(np.int8)
    blocks = join_q8_0(qs, d_bits)
    assert blocks.size == 2 * 34
    m = split_q8_0(blocks, 2, 32)
    assert m.format == "q8" and (m.rows, m.cols) == (1 * 2, 32)
    got_qs = m.qs_bytes.view(np.int8).reshape(2, 32)
    got_d = m.scale_bytes.view(np.float32)
    assert np.array_equal(got_qs, qs)
    assert np.array_equal(got_d, d_bits.view(np.float16).astype(np.float32))
    assert np.all(np.abs(got_qs * got_d[:, None] - values.reshape(2, 32)) <= 0.02)


def test_split_q8_0_matches_the_oracle_nan_included(orc):
    rng = np.random.default_rng(9)
    blocks = rng.integers(0, 256, (64, 34), dtype=np.uint8)
    blocks[:4, 0:2] = [[0x01, 0x7C], [0x00, 0xFE], [0x00, 0x80], [0x00, 0x7C]]
    m = split_q8_0(blocks, 2, 1024)
    qs, sc = orc.split_q8_0(blocks, 64)
    assert np.array_equal(m.qs_bytes.view(np.int8), qs)
    assert np.array_equal(m.scale_bytes.view(np.uint32), sc.view(np.uint32))


def test_split_q4_0_round_trip():
    rng = np.random.default_rng(0)
    qs = rng.integers(0, 256, (3, 64 // 2), dtype=np.uint8)
    d = rng.integers(0, 0x7BFF, (3, 2), dtype=np.uint16)
    m = split_q4_0(join_q4_0(qs, d), 3, 64)
    assert np.array_equal(m.qs_bytes.reshape(3, 32), qs)
    assert np.array_equal(m.scale_bytes.view(np.uint16).reshape(3, 2), d)


def test_split_rejects_bad_sizes():
    with pytest.raises(ArgumentError):
        split_q8_0(np.zeros(33, np.uint8), 1, 32)
    with pytest.raises(ArgumentError):
        split_q4_0(np.zeros(18, np.uint8), 1, 48)
    with pytest.raises(ArgumentError):
        QuantMatrix.q8(np.zeros((2, 40), np.int8), np.zeros(2, np.float32))


def test_widen_bf16_is_shift():
    b = np.array([0x0000, 0x8000, 0x3F80, 0xBF80, 0x7F80, 0x0001, 0x4049], np.uint16)
    w = widen_bf16(b)
    assert np.array_equal(w.view(np.uint32), b.astype(np.uint32) << 16)
    assert list(w[:4]) == [0.0, -0.0, 1.0, -1.0] and np.isinf(w[4])


def test_bf16_rne_rounds_to_nearest_even():
    x = np.float32([1.0, 1.00390625, 1.01171875, 1.0 + 2 ** -8 + 2 ** -20])
    # 1 + 2^-8 is a tie between bf16 1.0 and 1.0078125 -> even (1.0)
    assert list(widen_bf16(bf16_rne(x))) == [1.0, 1.0, 1.015625, 1.0078125]


def test_half_helpers_exhaustive():
    h = np.arange(65536, dtype=np.uint16)
    f = half_to_float(h)
    finite = np.isfinite(f)
    assert np.array_equal(float_to_half(f[finite]), h[finite])
