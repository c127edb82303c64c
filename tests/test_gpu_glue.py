"""The glue between the quantized products on the GPU against the C oracle,
bit for bit: the vision projector's exact-erf GELU (dnx_gelu,
lib/src/vision_encoder.dart:260-263, :496-509: Abramowitz-Stegun erf in
double, rounded once to float) at every start offset within a 16-byte line
and at counts around its four-values-per-thread passes, with the special
values the formula meets (signed zeros, subnormals, values whose
exponential underflows, infinities and NaN; NaN results compared as NaN)."""

import numpy as np
import pytest
import torch

from dianoia_amd import device as D
from gpu_util import bits, dev, host

pytestmark = pytest.mark.gpu

SPECIAL = np.array([0.0, -0.0, 1e-40, -1e-40, 1e-7, -1e-7, 0.5, -0.5, 3.0, -3.0, 10.0, -10.0,
                    40.0, -40.0, 1e30, -1e30, np.inf, -np.inf, np.nan], np.float32)


@pytest.mark.parametrize("count", [1, 2, 3, 4, 5, 7, 8, 1023, 4099, 1 << 20])
@pytest.mark.parametrize("offset", [0, 1, 2, 3])
def test_gelu_bit_exact_at_any_offset(gpu_ready, orc, count, offset):
    rng = np.random.default_rng(count * 4 + offset)
    x = (rng.standard_normal(count) * 2).astype(np.float32)
    x[:min(count, SPECIAL.size)] = SPECIAL[:min(count, SPECIAL.size)]
    pad = np.full(offset + count + 5, 7.0, np.float32)   # guard values around x
    pad[offset:offset + count] = x
    d = dev(pad)
    D.gelu(d[offset:offset + count])
    out = host(d)
    want = orc.gelu(x)
    got = out[offset:offset + count]
    # NaN results (from NaN and -inf) are compared as NaN: their payload
    # bits are the hardware's, not the formula's.
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits(got[~nan]), bits(want[~nan]))
    assert np.all(out[:offset] == 7.0) and np.all(out[offset + count:] == 7.0)
