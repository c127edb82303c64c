"""The quantized products' other callers at their own shapes, through the
lab_gpu_* ABI (GpuLinear) and through dnx_matmul_* (the same product route
on device pointers), against the CPU kernels.

Shapes, from the reference:
* Audio encoder (Q4_0 GGUF matrices, audio_encoder.dart:197-205, shapes
  audio_gguf.dart:242-290): hidden 768 and FFN 1792 as the reference's
  real-checkpoint test pins them (test/audio_encoder_test.dart:221-222); the
  projector maps into the 2048-wide language model
  (docs/lfm3_audio_support.md:156). K/V projections are taken at the full
  width (the head counts are not pinned by the reference's tests). Token
  counts: one 80 ms streaming chunk (1 row), 4, about 1 s (13 rows) and a
  30 s clip (375 rows: frames / 8).
* Audio generator (Depthformer, audio_generation.dart:19-25): only the
  reference's own fixture dimensions exist in the reference
  (test/fixtures/audio/generation_oracle.json: width 32, FFN 64, 2 / 1
  heads of 16), at the 12 codebook rows of one frame.
* Vision encoder attention projections and projector (vision_encoder.dart:
  275-316, :369-403, :252-271): hidden 1024, head dim 64
  (test/vision_config_test.dart:18-26), projector 4096 -> 4096 -> 2048, Q8
  from load-time quantization, at 1024 and 4096 patches (the 1024-token
  budget's 4 patches per token) and 256 / 1024 image tokens.

Mode 1 (int8 inputs, the ABI's default): n <= 4 bit-exact, wider n within
north_star's bar. Mode 0 (float inputs, what the reference's encoders use on
the CPU): n <= 4 the exact float-input GEMV, bit-exact; wider n the bf16-MFMA
float GEMM, within the reference GPU test's bar (1e-4 + 1e-5 |cpu|,
gpu_linear_test.dart:44): both it and the CPU round each block's float sum,
in different orders.
"""

import numpy as np
import pytest
import torch

from dianoia_amd import device as D
from dianoia_amd.formats import QuantMatrix
from dianoia_amd.gpu import GpuLinear, set_int8_inputs
from gpu_util import bits, dev, host, within_tolerance

pytestmark = pytest.mark.gpu

AUDIO_ENCODER = [(1792, 768), (768, 1792), (2304, 768), (768, 768), (2048, 768), (2048, 2048)]
AUDIO_GENERATOR = [(32, 32), (16, 32), (64, 32), (32, 64)]
VISION = [(1024, 1024, 1024), (1024, 1024, 4096), (4096, 4096, 256), (4096, 4096, 1024),
          (2048, 4096, 256), (2048, 4096, 1024)]

CASES = ([("q4", r, c, n) for r, c in AUDIO_ENCODER for n in (1, 4, 13, 375)] +
         [("q4", r, c, n) for r, c in AUDIO_GENERATOR for n in (1, 12)] +
         [("q8", r, c, n) for r, c, n in VISION])


@pytest.fixture()
def gpu(gpu_ready):
    g = GpuLinear.start()
    assert g is not None
    yield g
    g.dispose()


def weights(orc, fmt, rng, rows, cols):
    w = ((rng.random(rows * cols) * 2 - 1) * 0.1).astype(np.float32).reshape(rows, cols)
    if fmt == "q4":
        qs, sc = orc.quantize_q4(w)
        return QuantMatrix.q4(qs, sc), qs, sc
    qs, sc = orc.quantize_q8(w)
    return QuantMatrix.q8(qs, sc), qs, sc


def cpu(orc, fmt, qs, sc, xs, n, mode):
    f = orc.gemm_q4 if fmt == "q4" else orc.gemm_q8
    return f(qs, sc, xs, n, threads=8, mode=mode).reshape(-1)


@pytest.mark.parametrize("fmt,rows,cols,n", CASES)
@pytest.mark.parametrize("int8", [True, False], ids=["mode1", "mode0"])
def test_callers_through_the_abi(gpu, orc, fmt, rows, cols, n, int8):
    print(f"callers {fmt} {rows}x{cols} n={n} int8={int8}", flush=True)
    rng = np.random.default_rng(rows * 7 + cols + n)
    m, qs, sc = weights(orc, fmt, rng, rows, cols)
    gpu.upload("w", m)
    xs = (rng.random(n * cols) * 2 - 1).astype(np.float32)
    y = np.zeros(n * rows, np.float32)
    previous = set_int8_inputs(int8)
    try:
        gpu.apply("w", xs, y, n)
    finally:
        set_int8_inputs(previous)
    ref = cpu(orc, fmt, qs, sc, xs, n, 1 if int8 else 0)
    if n <= 4:
        assert np.array_equal(bits(y), bits(ref))
    elif not int8:
        assert np.all(np.abs(y - ref) <= 1e-4 + 1e-5 * np.abs(ref))
    else:
        ok, rel, ab = within_tolerance(y, ref)
        assert ok, (rel, ab)


@pytest.mark.parametrize("fmt,rows,cols,n", [("q4", 768, 1792, 1), ("q4", 768, 1792, 375),
                                             ("q8", 1024, 1024, 4096), ("q4", 6144, 2048, 384),
                                             ("q4", 64, 20000, 3), ("q8", 2048, 4096, 7)])
def test_matmul_route_on_device_pointers(gpu_ready, orc, fmt, rows, cols, n):
    """dnx_matmul_* takes the ABI's route: the GEMV (n <= 4; bit-exact), the
    GEMM after the GEMV refuses a wide x (K = 20000 at n = 3), the int8
    GEMM, and the fp6 GEMM (Q4, 384 tokens x 6144 rows)."""
    rng = np.random.default_rng(rows + cols + n)
    _, qs, sc = weights(orc, fmt, rng, rows, cols)
    xs = (rng.random(n * cols) * 2 - 1).astype(np.float32)
    y = torch.full((n, rows), float("nan"), device="cuda")
    ws = D.matmul_workspace(cols, n)
    f = D.matmul_q4 if fmt == "q4" else D.matmul_q8
    f(dev(qs), dev(sc), dev(xs), y, rows, cols, n, True, ws)
    got = host(y).reshape(-1)
    ref = cpu(orc, fmt, qs, sc, xs, n, 1)
    if n <= 4 and cols <= 8192:
        assert np.array_equal(bits(got), bits(ref))
    else:
        ok, rel, ab = within_tolerance(got, ref)
        assert ok, (rel, ab)


def test_matmul_route_rejects_a_short_workspace(gpu_ready):
    z = torch.zeros(1 << 16, device="cuda")
    short = torch.empty(16, dtype=torch.uint8, device="cuda")
    with pytest.raises(RuntimeError):
        D.matmul_q8(z, z, z, z, 64, 64, 8, True, short)
