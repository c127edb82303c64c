"""The decoder's other layer steps on the GPU (lab_gpu_enc_rms_norm ..
lab_gpu_enc_steer, lib/src/gpu.dart:179-312, Metal semantics
src/metal/lab_metal.m:321-579) against the CPU oracle's restatement of the
shaders. Element-wise steps with no reduction (conv, add, copy, steer mode 0)
are bit-exact; reductions run in another order, so those steps are held to
fp32 rounding: relative 1e-5, absolute 1e-6."""

import ctypes

import numpy as np
import pytest
import torch

from dianoia_amd import _lib
from dianoia_amd import device as D
from dianoia_amd import synth
from gpu_util import bits, dev, host

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-6


def close(gpu, cpu, rtol=RTOL, atol=ATOL):
    gpu, cpu = np.asarray(gpu, np.float64), np.asarray(cpu, np.float64)
    err = np.abs(gpu - cpu)
    ok = err <= atol + rtol * np.abs(cpu)
    return bool(ok.all()), float(err.max(initial=0.0))


@pytest.mark.parametrize("rows,cols,acc", [(1, 2048, False), (7, 1024, True), (128, 4096, False),
                                           (3, 37, True), (2, 16384, True), (5, 6144, False),
                                           (1, 2052, True), (1, 20000, False), (512, 2048, True),
                                           (256, 2048, True)])
def test_rms_norm(gpu_ready, orc, rows, cols, acc):
    rng = np.random.default_rng(rows + cols)
    x = (rng.standard_normal((rows, cols)) * 3).astype(np.float32)
    w = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    base = rng.standard_normal((rows, cols)).astype(np.float32)
    out = dev(base if acc else np.zeros_like(x))
    D.rms_norm(dev(x), dev(w), out, rows, cols, 1e-5, accumulate=acc)
    want = orc.rms_norm(x, w, 1e-5, out=base if acc else None)
    ok, err = close(host(out), want)
    assert ok, err


@pytest.mark.parametrize("heads,hd,n,stride_pad", [(16, 128, 1, 0), (8, 64, 5, 64), (2, 256, 3, 0),
                                                   (4, 512, 2, 32)])
def test_head_norm_rope(gpu_ready, orc, heads, hd, n, stride_pad):
    rng = np.random.default_rng(heads * hd + n)
    stride = heads * hd + stride_pad
    x = rng.standard_normal((n, stride)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    pair = hd // 2
    ang = rng.uniform(0, 6.3, (n, pair))
    rope_stride = hd + 16
    table = np.zeros((n, rope_stride), np.float32)
    table[:, :pair], table[:, pair:hd] = np.cos(ang), np.sin(ang)
    xd = dev(x)
    D.head_norm_rope(xd, stride, dev(w), dev(table), rope_stride, heads, hd, n, 1e-6)
    want = orc.head_norm_rope(x, stride, w, table, rope_stride, heads, hd, n, 1e-6)
    got = host(xd)
    ok, err = close(got[:, :heads * hd], want[:, :heads * hd])
    assert ok, err
    assert np.array_equal(got[:, heads * hd:], x[:, heads * hd:])  # the padding is untouched


@pytest.mark.parametrize("width,k,n", [(6144, 3, 1), (2048, 4, 7), (300, 16, 3), (33, 2, 5),
                                       (2048, 3, 512), (300, 16, 100), (100, 16, 7), (64, 4, 3),
                                       (65, 1, 10), (2048, 4, 129), (130, 16, 14), (70, 16, 79)])
def test_short_conv_bit_exact(gpu_ready, orc, width, k, n):
    """y and the carried state bit for bit, across token tiles (n > 64), with
    fewer new tokens than state rows (old rows shift down), n = k - 1, k = 1
    (no state) and widths that leave a partial channel slab."""
    rng = np.random.default_rng(width + k + n)
    bcx = rng.standard_normal((n, 3, width)).astype(np.float32)
    weight = rng.standard_normal((width, k)).astype(np.float32)
    hist = rng.standard_normal((k - 1, width)).astype(np.float32)
    hd_ = dev(hist)
    y = torch.zeros(n * width, device="cuda")
    D.short_conv(dev(bcx), dev(weight), hd_, y, width, k, n)
    want_y, want_h = orc.short_conv(bcx, weight, hist, width, k, n)
    assert np.array_equal(bits(host(y)), bits(want_y))
    assert np.array_equal(bits(host(hd_)), bits(want_h))


@pytest.mark.parametrize("heads,kv,hd,pos,n,window,gated", [
    (16, 4, 128, 2047, 1, 0, False),   # decode at 2 K context, GQA 4:1
    (8, 8, 64, 100, 7, 0, True),       # prefill chunk, gated heads
    (4, 2, 256, 600, 3, 128, False),   # sliding window
    (2, 1, 32, 0, 5, 0, True),         # from position 0
    (8, 2, 64, 3000, 3, 1000, True),   # split keys: window, gate, 3 tokens
    (32, 8, 128, 300, 4, 0, False),    # split keys, the tokens' counts differ
    (1, 1, 16, 20000, 1, 0, False),    # beyond one workgroup's LDS: split
    (32, 4, 64, 2500, 1, 0, True),     # split keys, 8 query heads per KV head
    (12, 2, 128, 1500, 2, 0, False),   # split keys, 6 per KV head: pairs of heads
    (6, 2, 32, 900, 1, 300, False),    # split keys, 3 per KV head: one head each
    (32, 8, 128, 0, 512, 0, False),    # prefill on the matrix cores, keys split in two
    (16, 8, 64, 37, 100, 0, True),     # matrix cores, 2 heads per KV head, gated, ragged
    (8, 8, 128, 500, 40, 64, False),   # matrix cores, one head per KV head, window 64
    (12, 4, 64, 3000, 24, 0, False),   # matrix cores, a long context: many key splits
    (4, 1, 128, 10, 9, 0, True),       # matrix cores, the smallest chunk, 4 heads per KV
    (8, 2, 64, 0, 64, 0, False),       # matrix cores, hd 64 with 4 heads per KV head
    (16, 2, 64, 200, 300, 100, True),  # matrix cores, 8 per KV head, window, gate, ragged
])
def test_attention(gpu_ready, orc, heads, kv, hd, pos, n, window, gated):
    rng = np.random.default_rng(heads + hd + pos + n)
    total = pos + n
    q = rng.standard_normal(n * heads * hd).astype(np.float32)
    keys = rng.standard_normal((total, kv * hd)).astype(np.float32)
    values = rng.standard_normal((total, kv * hd)).astype(np.float32)
    gate = rng.standard_normal(n * heads).astype(np.float32) if gated else None
    out = torch.zeros(n * heads * hd, device="cuda")
    D.attention(dev(q), dev(keys), dev(values), dev(gate) if gated else None, out, pos, n, heads,
                kv, hd, window)
    want = orc.attention(q, keys, values, gate, pos, n, heads, kv, hd, window)
    ok, err = close(host(out), want)
    assert ok, err


def test_attention_limits(gpu_ready):
    lib = _lib.load()
    assert lib.dnx_attention_max_keys(128) >= 15000
    assert lib.dnx_attention_max_keys(96) == -1  # 256 % 96 != 0
    q = torch.zeros(128, device="cuda")
    with pytest.raises(RuntimeError):
        D.attention(q, q, q, None, q, 0, 1, 1, 1, 96)


def test_add_copy_steer(gpu_ready, orc):
    rng = np.random.default_rng(8)
    a = rng.standard_normal(100003).astype(np.float32)
    b = rng.standard_normal(100003).astype(np.float32)
    dst = dev(b)
    D.add(dev(a), dst, a.size)
    assert np.array_equal(bits(host(dst)), bits(b + a))
    D.copy(dev(a), dst, a.size)
    assert np.array_equal(bits(host(dst)), bits(a))
    x = rng.standard_normal((5, 2048)).astype(np.float32)
    v = rng.standard_normal(2048)
    v = (v / np.linalg.norm(v)).astype(np.float32)
    xd = dev(x)
    D.steer(xd, dev(v), 5, 2048, 0, 1.0)
    assert np.array_equal(bits(host(xd)), bits(orc.steer(x, v, 0, 1.0)))
    xd = dev(x)
    D.steer(xd, dev(v), 5, 2048, 1, 0.75)
    ok, err = close(host(xd), orc.steer(x, v, 1, 0.75), atol=1e-5)
    assert ok, err


class Bufs:
    """lab_gpu_* buffers with host views (the ABI's staged coherence)."""

    def __init__(self):
        self.lib = _lib.load()
        assert self.lib.lab_gpu_init() == 1
        self.handles = []

    def new(self, arr):
        arr = np.ascontiguousarray(arr, np.float32).reshape(-1)
        h = self.lib.lab_gpu_buffer(max(arr.nbytes, 4))
        assert h >= 0
        self.handles.append(h)
        self.view(h, arr.size)[:] = arr
        return h

    def view(self, h, count):
        p = self.lib.lab_gpu_contents(h)
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_float)), (count,))

    def close(self):
        for h in self.handles:
            self.lib.lab_gpu_release(h)


def test_layer_steps_through_the_abi(gpu_ready, orc):
    """One command buffer with every layer step, read back through the
    host views, against the oracle (and bit-exact where the step is)."""
    rng = np.random.default_rng(9)
    B = Bufs()
    try:
        lib = B.lib
        rows, cols = 3, 256
        x = rng.standard_normal((rows, cols)).astype(np.float32)
        w = rng.uniform(0.5, 1.5, cols).astype(np.float32)
        hx, hw, hout = B.new(x), B.new(w), B.new(np.zeros_like(x))
        heads, hd, n = 4, 64, 2
        xr = rng.standard_normal((n, heads * hd)).astype(np.float32)
        wr = rng.uniform(0.5, 1.5, hd).astype(np.float32)
        ang = rng.uniform(0, 6.3, (n, hd // 2))
        table = np.concatenate([np.cos(ang), np.sin(ang)], axis=1).astype(np.float32)
        hxr, hwr, htab = B.new(xr), B.new(wr), B.new(table)
        width, k, tn = 96, 3, 4
        bcx = rng.standard_normal((tn, 3, width)).astype(np.float32)
        cw = rng.standard_normal((width, k)).astype(np.float32)
        hist = rng.standard_normal((k - 1, width)).astype(np.float32)
        hb, hcw, hh, hy = B.new(bcx), B.new(cw), B.new(hist), B.new(np.zeros(tn * width))
        ah, akv, ahd, apos, an = 4, 2, 32, 9, 2
        q = rng.standard_normal(an * ah * ahd).astype(np.float32)
        keys = rng.standard_normal((apos + an, akv * ahd)).astype(np.float32)
        vals = rng.standard_normal((apos + an, akv * ahd)).astype(np.float32)
        gate = rng.standard_normal(an * ah).astype(np.float32)
        hq, hk, hv, hg = B.new(q), B.new(keys), B.new(vals), B.new(gate)
        hao = B.new(np.zeros(an * ah * ahd))
        src = rng.standard_normal(1000).astype(np.float32)
        dst = rng.standard_normal(1000).astype(np.float32)
        hs, hd_, hc = B.new(src), B.new(dst), B.new(np.zeros(1000))
        sv = rng.standard_normal(cols)
        sv = (sv / np.linalg.norm(sv)).astype(np.float32)
        hsx, hsv = B.new(x), B.new(sv)

        lib.lab_gpu_begin()
        lib.lab_gpu_enc_rms_norm(hx, 0, hw, 0, hout, 0, rows, cols, 1e-5, 0)
        lib.lab_gpu_enc_head_norm_rope(hxr, 0, heads * hd, hwr, 0, htab, 0, hd, heads, hd, n, 1e-6)
        lib.lab_gpu_enc_conv(hb, hcw, 0, hh, hy, width, k, tn)
        lib.lab_gpu_enc_attention(hq, hk, hv, hg, hao, apos, an, ah, akv, ahd, 0)
        lib.lab_gpu_enc_add(hs, 0, hd_, 0, 1000)
        lib.lab_gpu_enc_copy(hs, 4 * 10, hc, 0, 990)
        lib.lab_gpu_enc_steer(hsx, 0, hsv, 0, rows, cols, 1, 1.0)
        assert lib.lab_gpu_commit(1) == 1

        ok, err = close(B.view(hout, rows * cols), orc.rms_norm(x, w, 1e-5).reshape(-1))
        assert ok, ("rms_norm", err)
        want = orc.head_norm_rope(xr, heads * hd, wr, table, hd, heads, hd, n, 1e-6)
        ok, err = close(B.view(hxr, n * heads * hd), want.reshape(-1))
        assert ok, ("head_norm_rope", err)
        wy, wh = orc.short_conv(bcx, cw, hist, width, k, tn)
        assert np.array_equal(bits(B.view(hy, tn * width)), bits(wy))
        assert np.array_equal(bits(B.view(hh, (k - 1) * width)), bits(wh.reshape(-1)))
        wa = orc.attention(q, keys, vals, gate, apos, an, ah, akv, ahd)
        ok, err = close(B.view(hao, an * ah * ahd), wa)
        assert ok, ("attention", err)
        assert np.array_equal(bits(B.view(hd_, 1000)), bits(dst + src))
        assert np.array_equal(bits(B.view(hc, 990)), bits(src[10:]))
        ok, err = close(B.view(hsx, rows * cols), orc.steer(x, sv, 1, 1.0).reshape(-1), atol=1e-5)
        assert ok, ("steer", err)

        # An invalid command fails the buffer instead of reading out of bounds.
        lib.lab_gpu_begin()
        lib.lab_gpu_enc_attention(hq, hk, hv, -1, hao, apos + 100, an, ah, akv, ahd, 0)
        assert lib.lab_gpu_commit(1) == 0
    finally:
        B.close()


def _profile(lib):
    """(ms, counts) per kind since the last call (lab_gpu_profile clears)."""
    ms = (ctypes.c_double * 21)()
    counts = (ctypes.c_int64 * 21)()
    assert lib.lab_gpu_profile(ms, counts, 21) == 21
    return list(ms), list(counts)


def _byte_buffer(B, raw):
    """A lab_gpu buffer holding `raw` (uint8) through its host view."""
    h = B.lib.lab_gpu_buffer(raw.nbytes)
    assert h >= 0
    B.handles.append(h)
    p = B.lib.lab_gpu_contents(h)
    view = np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_uint8)), (raw.nbytes,))
    view[:] = raw
    return h


def _run_sequence(build, split):
    """Records the commands build(B, lib) encodes, in one command buffer or
    one per command (split), with profiling on; returns the host views it
    names and the profile."""
    B = Bufs()
    lib = B.lib
    try:
        cmds, views = build(B, lib)
        _profile(lib)
        lib.lab_gpu_set_profiling(1)
        if split:
            for c in cmds:
                lib.lab_gpu_begin()
                c()
                assert lib.lab_gpu_commit(1) == 1
        else:
            lib.lab_gpu_begin()
            for c in cmds:
                c()
            assert lib.lab_gpu_commit(1) == 1
        lib.lab_gpu_set_profiling(0)
        prof = _profile(lib)
        return [B.view(h, n).copy() for h, n in views], prof
    finally:
        B.close()


RMS_NORM, HEAD_NORM_ROPE = 4, 5


def test_norm_fusion_declines_weights_in_the_norm_output_buffer(gpu_ready):
    """An RMSNorm whose output buffer also holds the weights of the matmul
    that reads it (disjoint regions): the commit runs the norm on its own
    (its kind gets time of its own) and leaves what one command per commit
    leaves, bit for bit."""
    rng = np.random.default_rng(31)
    rows, cols = 64, 256
    qs, sc = synth.q4_weights(rng, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    w = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    qs_off, sc_off = 4096, 4096 + qs.nbytes
    raw = np.zeros(sc_off + sc.nbytes, np.uint8)
    raw[qs_off:qs_off + qs.nbytes] = qs.reshape(-1)
    raw[sc_off:] = sc.reshape(-1).view(np.uint8)

    def build(B, lib):
        hx, hw, hy = B.new(x), B.new(w), B.new(np.zeros(rows))
        hp = _byte_buffer(B, raw)
        cmds = [lambda: lib.lab_gpu_enc_rms_norm(hx, 0, hw, 0, hp, 0, 1, cols, 1e-6, 0),
                lambda: lib.lab_gpu_enc_matmul_q4(hp, qs_off, sc_off, hp, 0, hy, 0, rows, cols, 1)]
        return cmds, [(hy, rows), (hp, cols)]

    (y1, n1), (ms1, _) = _run_sequence(build, split=False)
    (y2, n2), (ms2, _) = _run_sequence(build, split=True)
    assert np.array_equal(bits(y1), bits(y2)) and np.array_equal(bits(n1), bits(n2))
    assert ms1[RMS_NORM] > 0 and ms2[RMS_NORM] > 0


@pytest.mark.parametrize("shared", ["q_norm_weights", "rope_table"])
def test_rope_attention_fusion_declines_out_sharing_a_buffer(gpu_ready, shared):
    """A decode token's q/k head norms + RoPE and its attention, where the
    attention's out buffer also holds (past out's own bytes) the q norm's
    weights or the rope table: the commit does not fold the norms into the
    attention (the head norm kind gets time of its own) and leaves out, q and
    the key row as one command per commit does, bit for bit. (A gate in out's
    buffer would overlap out itself: both sit at offset 0.)"""
    rng = np.random.default_rng(37)
    heads, kv, hd, pos = 4, 2, 64, 200
    kvd = kv * hd
    q = rng.standard_normal(heads * hd).astype(np.float32)
    keys = rng.standard_normal((pos + 1) * kvd).astype(np.float32)
    vals = rng.standard_normal((pos + 1) * kvd).astype(np.float32)
    qw = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    kw = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    ang = rng.uniform(0, 6.3, hd // 2)
    rope = np.concatenate([np.cos(ang), np.sin(ang)]).astype(np.float32)
    gate = rng.standard_normal(heads).astype(np.float32)
    tail = {"q_norm_weights": qw, "rope_table": rope}[shared]
    out_floats = heads * hd

    def build(B, lib):
        hq, hk, hv = B.new(q), B.new(keys), B.new(vals)
        hout = B.new(np.concatenate([np.zeros(out_floats, np.float32), tail]))
        tail_off = out_floats * 4
        hqw = hout if shared == "q_norm_weights" else B.new(qw)
        qw_off = tail_off if shared == "q_norm_weights" else 0
        hkw = B.new(kw)
        hrope = hout if shared == "rope_table" else B.new(rope)
        rope_off = tail_off if shared == "rope_table" else 0
        hg = B.new(gate)
        cmds = [lambda: lib.lab_gpu_enc_head_norm_rope(hq, 0, heads * hd, hqw, qw_off, hrope,
                                                       rope_off, hd, heads, hd, 1, 1e-6),
                lambda: lib.lab_gpu_enc_head_norm_rope(hk, pos * kvd * 4, kvd, hkw, 0, hrope,
                                                       rope_off, hd, kv, hd, 1, 1e-6),
                lambda: lib.lab_gpu_enc_attention(hq, hk, hv, hg, hout, pos, 1, heads, kv, hd, 0)]
        return cmds, [(hout, out_floats), (hq, heads * hd), (hk, (pos + 1) * kvd)]

    (o1, q1, k1), (ms1, _) = _run_sequence(build, split=False)
    (o2, q2, k2), (ms2, _) = _run_sequence(build, split=True)
    assert np.array_equal(bits(o1), bits(o2))
    assert np.array_equal(bits(q1), bits(q2)) and np.array_equal(bits(k1), bits(k2))
    assert ms1[HEAD_NORM_ROPE] > 0


@pytest.mark.parametrize("rows,cols", [(1, 2048), (3, 6144), (256, 1024), (1, 4), (2, 16384)])
def test_add_rms_norm_fused(gpu_ready, orc, rows, cols):
    """The residual add and the following norm in one launch: x and out bit
    for bit what dnx_add then dnx_rms_norm leave, and out within the norm's
    bar of the oracle."""
    rng = np.random.default_rng(rows * 7 + cols)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    m = rng.standard_normal((rows, cols)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    x1, out1 = dev(x), torch.empty((rows, cols), device="cuda")
    D.add(dev(m), x1, rows * cols)
    D.rms_norm(x1, dev(w), out1, rows, cols, 1e-6)
    x2, out2 = dev(x), torch.empty((rows, cols), device="cuda")
    D.add_rms_norm(dev(m), x2, dev(w), out2, rows, cols, 1e-6)
    assert np.array_equal(bits(host(x2)), bits(host(x1)))
    assert np.array_equal(bits(host(out2)), bits(host(out1)))
    ok, err = close(host(out2), orc.rms_norm(x + m, w, 1e-6))
    assert ok, err


def test_add_rms_norm_rejects(gpu_ready):
    z = torch.zeros(1 << 16, device="cuda")
    with pytest.raises(RuntimeError):
        D.add_rms_norm(z, z[4096:], z, z[8192:], 257, 8, 1e-6)   # more rows than it holds in registers
    with pytest.raises(RuntimeError):
        D.add_rms_norm(z, z[4096:], z, z[8192:], 1, 6, 1e-6)     # cols not a multiple of 4
    with pytest.raises(RuntimeError):
        D.add_rms_norm(z, z[4097:], z, z[8192:], 1, 8, 1e-6)     # x not 16-byte aligned


@pytest.mark.parametrize("h0,h1,hd,n", [(16, 8, 128, 1), (32, 8, 64, 3), (2, 1, 256, 2)])
def test_head_norm_rope_pair(gpu_ready, h0, h1, hd, n):
    """q and k heads in one launch: bit-identical to the two calls."""
    rng = np.random.default_rng(h0 * hd + n)
    s0, s1 = h0 * hd + 32, h1 * hd
    q = rng.standard_normal((n, s0)).astype(np.float32)
    k = rng.standard_normal((n, s1)).astype(np.float32)
    w0 = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    w1 = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    pair = hd // 2
    ang = rng.uniform(0, 6.3, (n, pair))
    rs = hd + 16
    table = np.zeros((n, rs), np.float32)
    table[:, :pair], table[:, pair:hd] = np.cos(ang), np.sin(ang)
    qa, ka = dev(q), dev(k)
    D.head_norm_rope(qa, s0, dev(w0), dev(table), rs, h0, hd, n, 1e-6)
    D.head_norm_rope(ka, s1, dev(w1), dev(table), rs, h1, hd, n, 1e-6)
    qb, kb = dev(q), dev(k)
    D.head_norm_rope2(qb, s0, dev(w0), h0, kb, s1, dev(w1), h1, dev(table), rs, hd, n, 1e-6)
    assert np.array_equal(bits(host(qb)), bits(host(qa)))
    assert np.array_equal(bits(host(kb)), bits(host(ka)))


@pytest.mark.parametrize("heads,kv,hd,pos,window,gated", [(16, 8, 128, 4095, 0, False),
                                                          (32, 8, 128, 700, 0, True),
                                                          (8, 8, 64, 300, 0, False),
                                                          (16, 2, 64, 1000, 256, True),
                                                          (4, 1, 128, 64, 0, False),
                                                          (8, 4, 256, 300, 0, False),
                                                          (16, 8, 32, 500, 0, True)])
def test_attention_rope_equals_norms_then_attention(gpu_ready, heads, kv, hd, pos, window, gated):
    """dnx_attention_rope (the q and k head norms + RoPE folded into a decode
    token's split-key attention) against dnx_head_norm_rope on q and on the
    token's key row, then dnx_attention: out, q and the key row bit for bit;
    every other key row untouched. Head sizes 32 to 256 (hd 256: two rotary
    pairs per lane; hd 32: a 256-key split)."""
    rng = np.random.default_rng(heads * 7 + pos)
    kvd = kv * hd
    q0 = rng.standard_normal(heads * hd).astype(np.float32)
    keys0 = rng.standard_normal((pos + 1) * kvd).astype(np.float32)
    vals = dev(rng.standard_normal((pos + 1) * kvd).astype(np.float32))
    qw = dev(rng.uniform(0.5, 1.5, hd).astype(np.float32))
    kw = dev(rng.uniform(0.5, 1.5, hd).astype(np.float32))
    ang = rng.uniform(0, 6.3, hd // 2)
    rope = dev(np.concatenate([np.cos(ang), np.sin(ang)]).astype(np.float32))
    gate = dev(rng.standard_normal(heads).astype(np.float32)) if gated else None
    eps = 1e-6
    q_ref, k_ref = dev(q0), dev(keys0)
    out_ref = torch.empty(heads * hd, device="cuda")
    D.head_norm_rope(q_ref, heads * hd, qw, rope, hd, heads, hd, 1, eps)
    D.head_norm_rope(k_ref[pos * kvd:], kvd, kw, rope, hd, kv, hd, 1, eps)
    D.attention(q_ref, k_ref, vals, gate, out_ref, pos, 1, heads, kv, hd, window)
    q, k = dev(q0), dev(keys0)
    out = torch.full((heads * hd,), float("nan"), device="cuda")
    D.attention_rope(q, k, vals, gate, out, pos, heads, kv, hd, window, qw, kw, rope, eps)
    assert np.array_equal(bits(host(out)), bits(host(out_ref)))
    assert np.array_equal(bits(host(q)), bits(host(q_ref)))
    assert np.array_equal(bits(host(k)), bits(host(k_ref)))


def test_attention_rope_refuses_short_or_unsplit(gpu_ready):
    hd, heads, kv = 128, 16, 8
    z = torch.zeros(64 * kv * hd, device="cuda")
    w = torch.ones(hd, device="cuda")
    out = torch.zeros(heads * hd, device="cuda")
    q = torch.zeros(heads * hd, device="cuda")
    with pytest.raises(RuntimeError):   # 10 keys: one split, not the split-key path
        D.attention_rope(q, z, z, None, out, 9, heads, kv, hd, 0, w, w, w, 1e-6)
    z2 = torch.zeros(201 * 4 * 128, device="cuda")
    q2 = torch.zeros(12 * 128, device="cuda")
    out2 = torch.zeros(12 * 128, device="cuda")
    with pytest.raises(RuntimeError):   # three query heads per KV head: no single workgroup
        D.attention_rope(q2, z2, z2, None, out2, 200, 12, 4, 128, 0, w, w, w, 1e-6)
