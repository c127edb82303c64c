"""GPU quantizers against the reference's CPU quantizer, bit for bit."""

import os

import numpy as np
import pytest
import torch

from dianoia_amd import device as D
from gpu_util import bits, dev, host

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def gpu_quantize(x, cols_pad=None):
    rows, cols = x.shape
    cols_pad = cols if cols_pad is None else cols_pad
    qs = torch.zeros((rows, cols_pad), dtype=torch.int8, device="cuda")
    sc = torch.zeros((rows, cols_pad // 32), dtype=torch.float32, device="cuda")
    D.quantize_q8(dev(x), qs, sc, rows, cols, cols_pad)
    return host(qs), host(sc)


@pytest.mark.parametrize("name", ["edges", "random"])
def test_quantize_matches_golden(gpu_ready, name):
    d = np.load(os.path.join(GOLDEN, f"quantize_q8_{name}.npz"))
    qs, sc = gpu_quantize(d["x"])
    assert np.array_equal(qs, d["qs"])
    assert np.array_equal(bits(sc), bits(d["scales"]))


@pytest.mark.parametrize("rows,cols,pad", [(1, 1024, 1024), (512, 2048, 2048), (1024, 1152, 1152),
                                           (1024, 4304, 4320), (3, 33, 64), (7, 4, 32)])
def test_quantize_matches_oracle(gpu_ready, orc, rows, cols, pad):
    rng = np.random.default_rng(rows * 7 + cols)
    x = rng.standard_normal((rows, cols), dtype=np.float32)
    x[0, : min(cols, 5)] = [0.0, -0.0, 1e-40, -3e-39, 0.5][: min(cols, 5)]
    qs, sc = gpu_quantize(x, pad)
    q2, s2 = orc.quantize_q8_padded(x, pad)
    assert np.array_equal(qs, q2)
    assert np.array_equal(bits(sc), bits(s2))


@pytest.mark.parametrize("rows,cols", [(4304, 1152), (1152, 4304), (5, 37)])
def test_bf16_weight_quantizer(gpu_ready, orc, rows, cols):
    from dianoia_amd.synth import bf16_weights
    w = bf16_weights(np.random.default_rng(rows + cols), rows, cols)
    pad = (cols + 31) // 32 * 32
    qs = torch.zeros((rows, pad), dtype=torch.int8, device="cuda")
    sc = torch.zeros((rows, pad // 32), dtype=torch.float32, device="cuda")
    D.quantize_q8_bf16(dev(w), qs, sc, rows, cols, pad)
    q2, s2 = orc.quantize_q8_bf16(w, pad)
    assert np.array_equal(host(qs), q2)
    assert np.array_equal(bits(host(sc)), bits(s2))


def test_bf16_quantizer_through_the_abi(gpu_ready, orc):
    """GpuLinear.upload_bf16 -> lab_gpu_enc_quantize_q8_bf16 (C4's load path)."""
    from dianoia_amd.gpu import GpuLinear
    from dianoia_amd.synth import bf16_weights
    gpu = GpuLinear.start()
    try:
        w = bf16_weights(np.random.default_rng(44), 1152, 4304)
        gpu.upload_bf16("fc2", w, 1152, 4304)
        qs, sc = gpu.quantized("fc2")
        q2, s2 = orc.quantize_q8_bf16(w, 4320)
        assert qs.shape == (1152, 4320)
        assert np.array_equal(qs, q2)
        assert np.array_equal(bits(sc), bits(s2))
    finally:
        gpu.dispose()


def test_quantizer_rejects_bad_shapes(gpu_ready):
    x = torch.zeros(64, device="cuda")
    out = torch.zeros(64, dtype=torch.int8, device="cuda")
    sc = torch.zeros(2, device="cuda")
    with pytest.raises(RuntimeError):
        D.quantize_q8(x, out, sc, 1, 64, 48)  # cols_pad < cols
    with pytest.raises(RuntimeError):
        D.quantize_q8(x, out, sc, 1, 64, 63)  # not a multiple of 32
