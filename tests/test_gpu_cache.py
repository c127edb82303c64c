"""A weight cache (LFM3Q8C1) placed in HBM by GpuLinear.wrap_cache
(gpu.dart:938-979, ``_wrapWeights``) and multiplied through the lab_gpu_*
ABI: the products equal the CPU kernels' (bit-exact for n <= 4, within
the GEMM tolerance above), whether the cache is one buffer or many."""

import numpy as np
import pytest

from dianoia_amd import StateError
from dianoia_amd.formats import QuantMatrix
from dianoia_amd.gpu import GpuLinear, live_buffers
from dianoia_amd.q8_cache import Q8Cache
from gpu_util import bits, within_tolerance

pytestmark = pytest.mark.gpu

SHAPES = [("embed", "q8", 96, 64), ("attn.q", "q4", 64, 128), ("ffn.up", "q4", 160, 96),
          ("ffn.down", "q8", 64, 160), ("lm_head", "q8", 300, 64)]


@pytest.fixture()
def cache(tmp_path, orc):
    rng = np.random.default_rng(11)
    mats, raw = {}, {}
    for name, fmt, rows, cols in SHAPES:
        w = (rng.random((rows, cols)) * 2 - 1).astype(np.float32)
        if fmt == "q4":
            qs, sc = orc.quantize_q4(w)
            mats[name] = QuantMatrix.q4(qs, sc)
        else:
            qs, sc = orc.quantize_q8(w)
            mats[name] = QuantMatrix.q8(qs, sc)
        raw[name] = (fmt, qs, sc, rows, cols)
    path = str(tmp_path / "lfm3-q8.cache")
    Q8Cache.write(path, "key", mats)
    c = Q8Cache.open(path, "key")
    yield c, raw
    c.close()


def products_match(gpu, orc, raw, n):
    rng = np.random.default_rng(n)
    for name, (fmt, qs, sc, rows, cols) in raw.items():
        xs = (rng.random(n * cols) * 2 - 1).astype(np.float32)
        y = np.zeros(n * rows, np.float32)
        gpu.apply(name, xs, y, n)
        want = (orc.gemm_q4 if fmt == "q4" else orc.gemm_q8)(qs, sc, xs, n, threads=4, mode=1)
        if n <= 4:
            assert np.array_equal(bits(y.reshape(n, rows)), bits(want)), name
        else:
            ok, rel, ab = within_tolerance(y.reshape(n, rows), want)
            assert ok, (name, rel, ab)


@pytest.mark.parametrize("n", [1, 3, 20])
def test_one_segment(gpu_ready, orc, cache, n):
    c, raw = cache
    live = live_buffers()
    g = GpuLinear.start()
    try:
        where = g.wrap_cache(c)
        assert g.segments == 1 and len({h for h, _ in where.values()}) == 1
        assert all(start == 1 << 20 for _, start in where.values())  # page of the first matrix
        products_match(g, orc, raw, n)
    finally:
        g.dispose()
    assert live_buffers() == live


def test_segments_hold_whole_matrices(gpu_ready, orc, cache):
    c, raw = cache
    g = GpuLinear.start()
    try:
        # The first four matrices end 31680 bytes after the data region's
        # start; lm_head ends 53280 after it, and 36896 after its own page.
        where = g.wrap_cache(c, limit=37000)
        assert g.segments == 2
        assert where["embed"] == where["ffn.down"] and where["embed"] != where["lm_head"]
        for name, (h, start) in where.items():
            o = c.offsets(name, raw[name][3], raw[name][4])
            assert start % 16384 == 0 and start <= o["qs"] and o["end"] - start <= 37000
        products_match(g, orc, raw, 2)
        # Replacing a wrapped matrix keeps the shared segment alive.
        fmt, qs, sc, rows, cols = raw["embed"]
        g.upload("embed", QuantMatrix.q8(qs, sc))
        products_match(g, orc, raw, 1)
    finally:
        g.dispose()


def test_a_matrix_larger_than_the_limit_is_refused(gpu_ready, cache):
    c, _ = cache
    g = GpuLinear.start()
    try:
        with pytest.raises(StateError):
            g.wrap_cache(c, limit=8192)
    finally:
        g.dispose()


@pytest.mark.parametrize("nbytes", [(40 << 20) + 12345, (16 << 20), (3 << 20) + 7])
def test_wrap_copies_every_byte(gpu_ready, nbytes):
    """lab_gpu_wrap of a pageable region (large ones go through the pinned
    staging pieces): the HBM copy, read back through lab_gpu_contents, holds
    every byte."""
    import ctypes
    from dianoia_amd import _lib
    lib = _lib.load()
    assert lib.lab_gpu_init() == 1
    src = np.random.default_rng(nbytes % 1000).integers(0, 256, size=nbytes, dtype=np.uint8)
    h = lib.lab_gpu_wrap(src.ctypes.data, nbytes)
    assert h >= 0
    try:
        view = lib.lab_gpu_contents(h)
        assert view
        back = np.ctypeslib.as_array((ctypes.c_uint8 * nbytes).from_address(view))
        assert np.array_equal(back, src)
    finally:
        lib.lab_gpu_release(h)
