"""GGUF Q8_0 / Q4_0 blocks split into the engine's layout on the GPU
(splitQ8_0 / splitQ4_0, lib/src/gguf.dart:208-218, 270-282), bit for bit
against the oracle: every byte pattern (fp16 d of every kind, NaN
included), odd and even block counts (the values' 2 mod 4 alignment), a
buffer that ends with the last block, the 2^25-block segment boundary, and
through GpuLinear.upload_gguf to the products."""

import numpy as np
import pytest
import torch

from dianoia_amd import ArgumentError
from dianoia_amd import device as D
from gpu_util import bits, dev, host

pytestmark = pytest.mark.gpu

SIZES = {"q8_0": (34, 32, torch.int8, torch.float32), "q4_0": (18, 16, torch.uint8, torch.int16)}


def gpu_split(kind, blocks_dev, count):
    nb, nq, qdt, sdt = SIZES[kind]
    qs = torch.full((count * nq,), 0x55, dtype=torch.uint8, device="cuda").view(qdt)
    sc = torch.zeros(count, dtype=sdt, device="cuda")
    (D.split_q8_0 if kind == "q8_0" else D.split_q4_0)(blocks_dev, qs, sc, count)
    return qs, sc


def expect(orc, kind, blocks, count):
    return (orc.split_q8_0 if kind == "q8_0" else orc.split_q4_0)(blocks, count)


def same(kind, got_qs, got_sc, want_qs, want_sc):
    assert np.array_equal(np.asarray(got_qs).view(np.uint8), np.asarray(want_qs).view(np.uint8))
    if kind == "q8_0":
        assert np.array_equal(bits(got_sc), bits(want_sc))
    else:
        assert np.array_equal(np.asarray(got_sc).view(np.uint16), want_sc)


@pytest.mark.parametrize("kind", ["q8_0", "q4_0"])
@pytest.mark.parametrize("count", [1, 2, 3, 7, 1000, 65537])
def test_split_matches_oracle(gpu_ready, orc, kind, count):
    nb = SIZES[kind][0]
    rng = np.random.default_rng(count)
    blocks = rng.integers(0, 256, (count, nb), dtype=np.uint8)
    specials = [[0x01, 0x7C], [0x00, 0xFE], [0x00, 0x80], [0x00, 0x7C], [0x01, 0x00]]
    blocks[:min(count, 5), :2] = specials[:min(count, 5)]
    # The blocks' tensor is exactly count * nb bytes: the last block ends it.
    qs, sc = gpu_split(kind, dev(blocks.reshape(-1)), count)
    want_qs, want_sc = expect(orc, kind, blocks, count)
    same(kind, host(qs), host(sc), want_qs, want_sc)


@pytest.mark.parametrize("kind", ["q8_0", "q4_0"])
def test_split_across_the_segment_boundary(gpu_ready, orc, kind):
    """2^25 + 3 blocks: two launches, the second starting at block 2^25.
    Blocks near the boundary and at the end are checked against the oracle."""
    nb, nq = SIZES[kind][:2]
    count = (1 << 25) + 3
    gen = torch.Generator(device="cuda").manual_seed(17)
    blocks = torch.randint(0, 256, (count * nb,), dtype=torch.uint8, device="cuda",
                           generator=gen)
    qs, sc = gpu_split(kind, blocks, count)
    torch.cuda.synchronize()
    for lo, hi in [(0, 4), ((1 << 25) - 5, (1 << 25) + 3), (count - 4, count)]:
        b = blocks[lo * nb:hi * nb].cpu().numpy()
        want_qs, want_sc = expect(orc, kind, b, hi - lo)
        same(kind, qs[lo * nq:hi * nq].cpu().numpy(), sc[lo:hi].cpu().numpy(), want_qs, want_sc)
    del blocks, qs, sc
    torch.cuda.empty_cache()


def test_split_rejects_misaligned_pointers(gpu_ready):
    blocks = torch.zeros(34 * 4 + 16, dtype=torch.uint8, device="cuda")
    qs = torch.zeros(32 * 4 + 16, dtype=torch.uint8, device="cuda")
    sc = torch.zeros(8, device="cuda")
    with pytest.raises(RuntimeError):
        D.split_q8_0(blocks[2:], qs, sc, 4)        # blocks not 4-byte aligned
    with pytest.raises(RuntimeError):
        D.split_q8_0(blocks, qs[4:], sc, 4)        # values not 16-byte aligned


@pytest.mark.parametrize("kind,rows,cols,n", [("q8_0", 300, 256, 1), ("q4_0", 96, 512, 3),
                                              ("q8_0", 64, 128, 24)])
def test_upload_gguf_products(gpu_ready, orc, kind, rows, cols, n):
    from dianoia_amd.formats import join_q4_0, join_q8_0
    from dianoia_amd.gpu import GpuLinear
    from gpu_util import within_tolerance
    rng = np.random.default_rng(rows + n)
    w = (rng.random((rows, cols)) * 2 - 1).astype(np.float32)
    if kind == "q8_0":
        qs, sc = orc.quantize_q8(w)
        d = sc.astype(np.float16).view(np.uint16)   # a GGUF file holds fp16 d
        blocks = join_q8_0(qs, d)
    else:
        qs, d = orc.quantize_q4(w)
        blocks = join_q4_0(qs, d)
    gpu = GpuLinear.start()
    try:
        gpu.upload_gguf("w", blocks, rows, cols, kind)
        got_qs, got_sc = gpu.quantized("w")
        want_qs, want_sc = expect(orc, kind, blocks, rows * cols // 32)
        same(kind, got_qs.reshape(-1), got_sc.reshape(-1), want_qs, want_sc)
        xs = (rng.random(n * cols) * 2 - 1).astype(np.float32)
        y = np.zeros(n * rows, np.float32)
        gpu.apply("w", xs, y, n)
        if kind == "q8_0":
            cpu = orc.gemm_q8(want_qs.reshape(rows, cols), want_sc.reshape(rows, -1), xs, n,
                              threads=4, mode=1)
        else:
            cpu = orc.gemm_q4(want_qs.reshape(rows, cols // 2), want_sc.reshape(rows, -1), xs,
                              n, threads=4, mode=1)
        if n <= 4:
            assert np.array_equal(bits(y.reshape(n, rows)), bits(cpu))
        else:
            ok, rel, ab = within_tolerance(y.reshape(n, rows), cpu)
            assert ok, (rel, ab)
        with pytest.raises(ArgumentError):
            gpu.upload_gguf("bad", blocks[:-1], rows, cols, kind)
    finally:
        gpu.dispose()


def test_split_encoders_at_offsets(gpu_ready, orc):
    """lab_gpu_enc_split_q8_0 / _q4_0 on buffers at nonzero offsets, both in
    one command buffer, read back through the host views; a misaligned
    offset fails the command buffer."""
    import ctypes
    from dianoia_amd import _lib
    lib = _lib.load()
    assert lib.lab_gpu_init() == 1
    rng = np.random.default_rng(21)
    rows, cols = 5, 96
    count = rows * cols // 32
    b8 = rng.integers(0, 256, (count, 34), dtype=np.uint8)
    b4 = rng.integers(0, 256, (count, 18), dtype=np.uint8)
    handles = []

    def buf(nbytes):
        h = lib.lab_gpu_buffer(nbytes)
        assert h >= 0
        handles.append(h)
        return h

    def view(h, nbytes):
        return np.ctypeslib.as_array(
            ctypes.cast(lib.lab_gpu_contents(h), ctypes.POINTER(ctypes.c_uint8)), (nbytes,))

    try:
        src = buf(4096)
        dst = buf(8192)
        view(src, 4096)[64:64 + b8.size] = b8.reshape(-1)
        view(src, 4096)[2048:2048 + b4.size] = b4.reshape(-1)
        lib.lab_gpu_begin()
        lib.lab_gpu_enc_split_q8_0(src, 64, dst, 16, dst, 1024, rows, cols)
        lib.lab_gpu_enc_split_q4_0(src, 2048, dst, 2048, dst, 4000, rows, cols)
        assert lib.lab_gpu_commit(1) == 1
        out = view(dst, 8192)
        q8, s8 = orc.split_q8_0(b8, count)
        q4, d4 = orc.split_q4_0(b4, count)
        assert np.array_equal(out[16:16 + q8.size], q8.view(np.uint8))
        assert np.array_equal(out[1024:1024 + 4 * count].view(np.uint32), s8.view(np.uint32))
        assert np.array_equal(out[2048:2048 + q4.size], q4)
        assert np.array_equal(out[4000:4000 + 2 * count].view(np.uint16), d4)
        lib.lab_gpu_begin()
        lib.lab_gpu_enc_split_q8_0(src, 66, dst, 16, dst, 1024, rows, cols)   # not 4-aligned
        assert lib.lab_gpu_commit(1) == 0
    finally:
        for h in handles:
            lib.lab_gpu_release(h)
