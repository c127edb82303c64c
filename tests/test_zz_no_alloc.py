"""The allocation-free fp6 GEMM entry point (dnx_gemm_q4_f6p_noalloc), called
through the C ABI, against the allocating one (dnx_gemm_q4_f6p) on two calls
in a row, the second smaller, both splitting K (so both use the fixed scratch
array for their partials): the same bits, and the CPU kernel's bar."""

import ctypes

import numpy as np
import pytest
import torch

from dianoia_amd import synth
from gpu_util import bits, dev, host, within_tolerance

pytestmark = pytest.mark.gpu

DNX_ESCRATCH = -4


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def test_noalloc_gemm_matches_allocating_entry(gpu_ready, orc):
    lib = gpu_ready
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    max_floats = int(lib.dnx_gemm_q4_f6p_noalloc_max_floats())
    assert max_floats > 0
    # rows x cols x n: 16 and 11 workgroup tiles, so K splits 8 and 4 ways.
    for rows, cols, n in ((1536, 4096, 64), (1000, 2048, 40)):
        print(f"noalloc gemm {rows}x{cols} n={n}", flush=True)
        rng = np.random.default_rng(rows + n)
        qs, sc = synth.q4_weights(rng, rows, cols)
        xs = synth.activations(rng, n, cols)
        panel = torch.empty(int(lib.dnx_f6_panel_bytes(n, cols)), dtype=torch.uint8,
                            device="cuda")
        xd = dev(xs)
        assert lib.dnx_quantize_q8_f6panel(_p(xd), _p(panel), n, cols, stream) == 0
        packed = torch.empty(int(lib.dnx_q4_f6pack_bytes(rows, cols)), dtype=torch.uint8,
                             device="cuda")
        qd, sd = dev(qs), dev(sc)
        assert lib.dnx_pack_q4_f6(_p(qd), _p(sd), _p(packed), rows, cols, stream) == 0
        y_free = torch.full((n, rows), float("nan"), device="cuda")
        y_alloc = torch.full((n, rows), float("nan"), device="cuda")
        rc = lib.dnx_gemm_q4_f6p_noalloc(_p(packed), _p(panel), _p(y_free), rows, cols, n, stream)
        assert rc == 0, rc
        assert lib.dnx_gemm_q4_f6p(_p(packed), _p(panel), _p(y_alloc), rows, cols, n,
                                   stream) == 0
        a, b = host(y_free), host(y_alloc)
        assert np.array_equal(bits(a), bits(b))
        ref = orc.gemm_q4(qs, sc, xs, n, threads=8, mode=1)
        ok, worst_rel, worst_abs = within_tolerance(a, ref)
        assert ok, (worst_rel, worst_abs)


def test_noalloc_gemm_allocates_nothing(gpu_ready):
    """The call's defining property: at a shape whose split partials (12.6 MB,
    2 K parts x 128 tokens x 12288 rows) are larger than any earlier call's
    in this file, device free memory is the same before and after (an
    allocating path would have grown its partials buffer by that much); its
    bits equal the allocating entry point's."""
    lib = gpu_ready
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rows, cols, n = 12288, 4096, 128     # 128 workgroup tiles: K splits 2 ways
    rng = np.random.default_rng(3)
    qs, sc = synth.q4_weights(rng, rows, cols)
    xs = synth.activations(rng, n, cols)
    panel = torch.empty(int(lib.dnx_f6_panel_bytes(n, cols)), dtype=torch.uint8, device="cuda")
    xd = dev(xs)
    assert lib.dnx_quantize_q8_f6panel(_p(xd), _p(panel), n, cols, stream) == 0
    packed = torch.empty(int(lib.dnx_q4_f6pack_bytes(rows, cols)), dtype=torch.uint8,
                         device="cuda")
    qd, sd = dev(qs), dev(sc)
    assert lib.dnx_pack_q4_f6(_p(qd), _p(sd), _p(packed), rows, cols, stream) == 0
    y_free = torch.full((n, rows), float("nan"), device="cuda")
    y_alloc = torch.full((n, rows), float("nan"), device="cuda")
    # warm-up at a small split shape (the per-device scratch address lookup)
    assert lib.dnx_gemm_q4_f6p_noalloc(_p(packed), _p(panel), _p(y_free), 96, cols, n,
                                       stream) == 0
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    rc = lib.dnx_gemm_q4_f6p_noalloc(_p(packed), _p(panel), _p(y_free), rows, cols, n, stream)
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    assert rc == 0, rc
    assert free0 - free1 < (4 << 20), (free0, free1)
    assert lib.dnx_gemm_q4_f6p(_p(packed), _p(panel), _p(y_alloc), rows, cols, n, stream) == 0
    torch.cuda.synchronize()
    assert np.array_equal(bits(host(y_free)), bits(host(y_alloc)))


def test_noalloc_gemm_rejects_bad_arguments(gpu_ready):
    """Shapes the GEMM does not take are refused before any launch, as by the
    allocating entry point; DNX_ESCRATCH is the code for partials beyond the
    array, which no accepted shape reaches with the current split policy."""
    lib = gpu_ready
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    buf = torch.empty(1 << 16, dtype=torch.uint8, device="cuda")
    y = torch.empty(1024, device="cuda")
    assert lib.dnx_gemm_q4_f6p_noalloc(_p(buf), _p(buf), _p(y), 32, 48, 1, stream) == -1
    assert lib.dnx_gemm_q4_f6p_noalloc(_p(buf), _p(buf), _p(y), 0, 64, 1, stream) == -1
    torch.cuda.synchronize()
