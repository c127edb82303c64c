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


# Shapes of 64 K blocks or more take the block-per-lane kernel (2048 x 2048,
# 1024 x 4304 padded), the others the quad-per-lane one.
@pytest.mark.parametrize("rows,cols,pad", [(1, 1024, 1024), (512, 2048, 2048), (2048, 2048, 2048),
                                           (1024, 1152, 1152),
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


# ---- lab_quantize_q4 (lab_native.c:928-955)

def gpu_quantize_q4(x, bf16=False):
    rows, cols = x.shape
    qs = torch.zeros((rows, cols // 2), dtype=torch.uint8, device="cuda")
    sc = torch.zeros((rows, cols // 32), dtype=torch.int16, device="cuda")
    (D.quantize_q4_bf16 if bf16 else D.quantize_q4)(dev(x), qs, sc, rows, cols)
    return host(qs), host(sc).view(np.uint16)


@pytest.mark.parametrize("name", ["quantize_q4", "quantize_q4_edges"])
def test_quantize_q4_matches_golden(gpu_ready, name):
    d = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    qs, sc = gpu_quantize_q4(d["x"])
    assert np.array_equal(qs, d["qs"])
    assert np.array_equal(sc, d["scales"])


@pytest.mark.parametrize("rows,cols", [(1, 32), (6144, 2048), (2048, 6144), (37, 1152), (3, 96)])
def test_quantize_q4_matches_oracle(gpu_ready, orc, rows, cols):
    rng = np.random.default_rng(rows * 5 + cols)
    x = rng.standard_normal((rows, cols), dtype=np.float32)
    x *= (np.float32(10.0) ** rng.integers(-8, 9, size=(rows, 1))).astype(np.float32)
    # Small integers: many blocks whose largest magnitude appears with both
    # signs, where the first in column order decides d's sign.
    x[rows // 2:] = rng.integers(-4, 5, size=(rows - rows // 2, cols)).astype(np.float32)
    qs, sc = gpu_quantize_q4(x)
    q2, s2 = orc.quantize_q4(x)
    assert np.array_equal(qs, q2)
    assert np.array_equal(sc, s2)


@pytest.mark.parametrize("rows,cols", [(4304, 1152), (1152, 4320), (5, 64)])
def test_bf16_q4_weight_quantizer(gpu_ready, orc, rows, cols):
    from dianoia_amd.synth import bf16_weights
    w = bf16_weights(np.random.default_rng(rows + 3 * cols), rows, cols)
    widened = (w.astype(np.uint32) << 16).view(np.float32)
    qs, sc = gpu_quantize_q4(w, bf16=True)
    q2, s2 = orc.quantize_q4(widened)
    assert np.array_equal(qs, q2)
    assert np.array_equal(sc, s2)


@pytest.mark.parametrize("bf16", [False, True])
def test_q4_quantizer_through_the_abi(gpu_ready, orc, bf16):
    """GpuLinear.upload_f32 / upload_bf16 with fmt="q4" -> lab_gpu_enc_quantize_q4*,
    then a decode product on the quantized weights, bit-exact with the CPU."""
    from dianoia_amd.gpu import GpuLinear
    from dianoia_amd.synth import bf16_weights
    rows, cols = 300, 2048
    rng = np.random.default_rng(9)
    gpu = GpuLinear.start()
    try:
        if bf16:
            w = bf16_weights(rng, rows, cols)
            gpu.upload_bf16("w", w, rows, cols, fmt="q4")
            wf = (w.astype(np.uint32) << 16).view(np.float32)
        else:
            wf = rng.standard_normal((rows, cols), dtype=np.float32)
            gpu.upload_f32("w", wf, rows, cols, fmt="q4")
        qs, sc = gpu.quantized("w")
        q2, s2 = orc.quantize_q4(wf)
        assert np.array_equal(qs, q2)
        assert np.array_equal(sc, s2)
        xs = rng.standard_normal(cols, dtype=np.float32)
        ys = np.zeros(rows, np.float32)
        gpu.apply("w", xs, ys, 1)
        cpu = orc.gemm_q4(q2, s2, xs, 1, threads=4, mode=1).reshape(-1)
        assert np.array_equal(bits(ys), bits(cpu))
    finally:
        gpu.dispose()


def test_quantizers_generic_path(gpu_ready, orc):
    """Inputs the block-per-lane kernel does not take (a bf16 source at an odd
    element, int8 output not 16-byte aligned) run the generic kernel, with the
    same results."""
    from dianoia_amd.synth import bf16_weights
    rows, cols = 33, 256
    w = bf16_weights(np.random.default_rng(71), rows, cols + 1)
    src = dev(w.reshape(-1))[1:1 + rows * cols]          # 2-byte aligned
    widened = (w.reshape(-1)[1:1 + rows * cols].astype(np.uint32) << 16).view(np.float32)
    widened = widened.reshape(rows, cols)
    qs = torch.zeros((rows, cols // 2), dtype=torch.uint8, device="cuda")
    sc = torch.zeros((rows, cols // 32), dtype=torch.int16, device="cuda")
    D.quantize_q4_bf16(src, qs, sc, rows, cols)
    q2, s2 = orc.quantize_q4(widened)
    assert np.array_equal(host(qs), q2)
    assert np.array_equal(host(sc).view(np.uint16), s2)
    x = np.random.default_rng(72).standard_normal((rows, cols), dtype=np.float32)
    q8 = torch.zeros(rows * cols + 4, dtype=torch.int8, device="cuda")
    s8 = torch.zeros((rows, cols // 32), dtype=torch.float32, device="cuda")
    D.quantize_q8(dev(x), q8[4:], s8, rows, cols, cols)  # output 4-byte aligned only
    q3, s3 = orc.quantize_q8(x)
    assert np.array_equal(host(q8)[4:].reshape(rows, cols), q3)
    assert np.array_equal(bits(host(s8)), bits(s3))


def test_q4_quantizer_rejects_bad_shapes(gpu_ready):
    x = torch.zeros(96, device="cuda")
    qs = torch.zeros(48, dtype=torch.uint8, device="cuda")
    sc = torch.zeros(3, dtype=torch.int16, device="cuda")
    with pytest.raises(RuntimeError):
        D.quantize_q4(x, qs, sc, 1, 48)   # not a multiple of 32
    with pytest.raises(RuntimeError):
        D.quantize_q4(x, qs[1:], sc, 1, 32)  # qs not 4-byte aligned


# ---- the Q6_K -> Q8 embedding / LM-head adapter (gguf.dart:402-414)

def gpu_q6k_to_q8(blocks, rows, cols):
    qs = torch.zeros((rows, cols), dtype=torch.int8, device="cuda")
    sc = torch.zeros((rows, cols // 32), dtype=torch.float32, device="cuda")
    D.q6k_to_q8(dev(blocks), qs, sc, rows, cols)
    return host(qs), host(sc)


@pytest.mark.parametrize("rows,cols,raw", [(1, 256, False), (37, 2048, False), (4096, 2048, False),
                                           (64, 1024, True), (3, 4096, True),
                                           (2048, 2048, True), (300, 7168, True)])
def test_q6k_to_q8_matches_oracle(gpu_ready, orc, rows, cols, raw):
    from q6k_util import pack_q6k, random_blocks
    rng = np.random.default_rng(rows + cols + raw)
    nb = rows * cols // 256
    if raw:  # every byte pattern, fp16 d of any kind included
        blocks = rng.integers(0, 256, size=(nb, 210), dtype=np.uint8)
    else:
        blocks = pack_q6k(*random_blocks(rng, nb))
    qs, sc = gpu_q6k_to_q8(blocks, rows, cols)
    q2, s2 = orc.q6k_to_q8(blocks, rows, cols)
    assert np.array_equal(qs, q2)
    assert np.array_equal(bits(sc), bits(s2))


def test_q6k_adapter_through_the_abi(gpu_ready, orc):
    """GpuLinear.upload_q6k -> lab_gpu_enc_q6k_to_q8, then the LM head with the
    fused greedy argmax on the converted weights, bit-exact with the CPU."""
    from dianoia_amd.gpu import GpuLinear
    from q6k_util import pack_q6k, random_blocks
    rows, cols = 1000, 2048
    rng = np.random.default_rng(63)
    blocks = pack_q6k(*random_blocks(rng, rows * cols // 256, specials=False))
    gpu = GpuLinear.start()
    try:
        gpu.upload_q6k("head", blocks, rows, cols)
        qs, sc = gpu.quantized("head")
        q2, s2 = orc.q6k_to_q8(blocks, rows, cols)
        assert np.array_equal(qs, q2)
        assert np.array_equal(bits(sc), bits(s2))
        xs = rng.standard_normal(cols, dtype=np.float32)
        logits = np.zeros(rows, np.float32)
        token = gpu.apply_argmax("head", xs, logits)
        cpu = orc.gemm_q8(q2, s2, xs, 1, threads=4, mode=1).reshape(-1)
        assert np.array_equal(bits(logits), bits(cpu))
        assert token == orc.argmax(cpu)
    finally:
        gpu.dispose()


def test_q6k_adapter_rejects_bad_shapes(gpu_ready):
    blocks = torch.zeros(420, dtype=torch.uint8, device="cuda")
    qs = torch.zeros(512, dtype=torch.int8, device="cuda")
    sc = torch.zeros(16, device="cuda")
    with pytest.raises(RuntimeError):
        D.q6k_to_q8(blocks, qs, sc, 1, 480)  # not a multiple of 256


def test_quantizer_rejects_bad_shapes(gpu_ready):
    x = torch.zeros(64, device="cuda")
    out = torch.zeros(64, dtype=torch.int8, device="cuda")
    sc = torch.zeros(2, device="cuda")
    with pytest.raises(RuntimeError):
        D.quantize_q8(x, out, sc, 1, 64, 48)  # cols_pad < cols
    with pytest.raises(RuntimeError):
        D.quantize_q8(x, out, sc, 1, 64, 63)  # not a multiple of 32
