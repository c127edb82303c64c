"""GpuLinear through the lab_gpu_* ABI: the reference's gpu_linear_test.dart
cases (test/gpu_linear_test.dart:26-102), compared with the CPU kernels in
mode 1 (int8 inputs, the default) and, with float inputs, in mode 0 (what the
reference's own test compares against), plus the configurations' end-to-end
chains."""

import numpy as np
import pytest

from dianoia_amd import ArgumentError, StateError, synth
from dianoia_amd.formats import QuantMatrix
from dianoia_amd.gpu import GpuLinear, live_buffers, set_int8_inputs
from gpu_util import bits, within_tolerance

pytestmark = pytest.mark.gpu


@pytest.fixture()
def gpu(gpu_ready):
    g = GpuLinear.start()
    assert g is not None
    yield g
    g.dispose()


def values(rng, count):
    return (rng.random(count) * 2 - 1).astype(np.float32)


def quantized(orc, fmt, w, rows, cols):
    w = w.reshape(rows, cols)
    if fmt == "q4":
        qs, sc = orc.quantize_q4(w)
        return QuantMatrix.q4(qs, sc), qs, sc
    qs, sc = orc.quantize_q8(w)
    return QuantMatrix.q8(qs, sc), qs, sc


def cpu_mode1(orc, fmt, qs, sc, xs, n):
    return (orc.gemm_q4 if fmt == "q4" else orc.gemm_q8)(qs, sc, xs, n, threads=4, mode=1)


def check(gpu_y, cpu_y, n):
    if n <= 4:
        assert np.array_equal(bits(gpu_y), bits(cpu_y))  # GEMV: same float order
    else:
        ok, rel, ab = within_tolerance(gpu_y, cpu_y)
        assert ok, (rel, ab)


@pytest.mark.parametrize("fmt,rows,cols,n", [("q4", 64, 64, 1), ("q4", 70, 96, 13),
                                             ("q8", 36, 64, 9), ("q8", 128, 128, 40),
                                             ("q8", 36, 64, 3), ("q4", 70, 96, 4)])
def test_matches_the_cpu_kernels(gpu, orc, fmt, rows, cols, n):
    rng = np.random.default_rng(5)
    m, qs, sc = quantized(orc, fmt, values(rng, rows * cols), rows, cols)
    gpu.upload("m", m)
    xs = values(rng, n * cols)
    on_gpu = np.zeros(n * rows, np.float32)
    gpu.apply("m", xs, on_gpu, n)
    check(on_gpu.reshape(n, rows), cpu_mode1(orc, fmt, qs, sc, xs, n), n)


def test_grows_its_buffers_and_keeps_earlier_matrices(gpu, orc):
    rng = np.random.default_rng(6)
    small, sq, ss = quantized(orc, "q4", values(rng, 32 * 32), 32, 32)
    large, lq, ls = quantized(orc, "q4", values(rng, 64 * 256), 64, 256)
    gpu.upload("small", small)
    gpu.upload("large", large)
    for name, (q, s), rows, cols, n in [("small", (sq, ss), 32, 32, 3),
                                        ("large", (lq, ls), 64, 256, 50),
                                        ("small", (sq, ss), 32, 32, 7)]:
        xs = values(rng, n * cols)
        on_gpu = np.zeros(n * rows, np.float32)
        gpu.apply(name, xs, on_gpu, n)
        check(on_gpu.reshape(n, rows), cpu_mode1(orc, "q4", q, s, xs, n), n)


def test_rejects_unknown_matrices_and_short_lists(gpu, orc):
    m, _, _ = quantized(orc, "q4", values(np.random.default_rng(1), 32 * 32), 32, 32)
    gpu.upload("m", m)
    with pytest.raises(ArgumentError):
        gpu.apply("missing", np.zeros(32, np.float32), np.zeros(32, np.float32), 1)
    with pytest.raises(ArgumentError):
        gpu.apply("m", np.zeros(32, np.float32), np.zeros(32, np.float32), 2)


def test_frees_its_buffers_once_and_then_refuses_work(gpu_ready, orc):
    live = live_buffers()
    other = GpuLinear.start()
    rng = np.random.default_rng(2)
    m, _, _ = quantized(orc, "q8", values(rng, 32 * 32), 32, 32)
    other.upload("m", m)
    other.apply("m", values(rng, 32), np.zeros(32, np.float32), 1)
    assert live_buffers() == live + 3
    other.dispose()
    other.dispose()
    assert live_buffers() == live
    with pytest.raises(StateError):
        other.apply("m", values(rng, 32), np.zeros(32, np.float32), 1)


def test_config0_q8_gemv(gpu, orc):
    qs, sc, x = synth.config0()
    gpu.upload("w", QuantMatrix.q8(qs, sc))
    y = np.zeros(3072, np.float32)
    gpu.apply("w", x, y, 1)
    assert np.array_equal(bits(y), bits(orc.gemm_q8(qs, sc, x, 1, threads=8, mode=1)[0]))


def test_config1_mlp(gpu, orc):
    """Config 1 through the ABI: gate/up GEMVs, SiLU glue, down GEMV.
    Stage-wise: the down product is checked bit-exactly on the GPU's own glue
    output; the glue itself against the CPU glue (double SiLU) to 1 ulp."""
    (gq, gs), (uq, us), (dq, ds), x = synth.config1()
    for name, (q, s) in (("gate", (gq, gs)), ("up", (uq, us)), ("down", (dq, ds))):
        gpu.upload(name, QuantMatrix.q4(q, s))
    y = np.zeros(2048, np.float32)
    gpu.mlp("gate", "up", "down", x, y, 1)
    g = orc.gemm_q4(gq, gs, x, 1, threads=8, mode=1)
    u = orc.gemm_q4(uq, us, x, 1, threads=8, mode=1)
    g_gpu = np.zeros(6144, np.float32)
    u_gpu = np.zeros(6144, np.float32)
    gpu.apply("gate", x, g_gpu, 1)
    gpu.apply("up", x, u_gpu, 1)
    assert np.array_equal(bits(g_gpu), bits(g[0])) and np.array_equal(bits(u_gpu), bits(u[0]))
    # The ABI fuses gate, up and the glue into one kernel (peephole at
    # commit); u must still hold the up products the unfused chain leaves.
    assert np.array_equal(bits(gpu._aux["u"].view(count=6144)), bits(u[0]))
    h = orc.silu_mul(g, u)
    # down product of the CPU glue output, bit-exact against the GPU's chain
    ref = orc.gemm_q4(dq, ds, h, 1, threads=8, mode=1)[0]
    diff_ulp = np.abs(bits(y).astype(np.int64) - bits(ref).astype(np.int64))
    # identical glue -> identical output; report the rare 1-ulp SiLU flip
    assert np.mean(diff_ulp == 0) > 0.99, np.mean(diff_ulp == 0)
    ok, rel, ab = within_tolerance(y, ref)
    assert ok, (rel, ab)


@pytest.mark.parametrize("fmt,rows,cols,n", [("q4", 512, 4096, 2), ("q4", 512, 4096, 3),
                                             ("q4", 512, 4096, 4), ("q8", 256, 10240, 4),
                                             ("q8", 256, 10240, 3), ("q4", 64, 1024, 4)])
def test_mlp_short_prompts_wide_hidden(gpu, orc, fmt, rows, cols, n):
    """The MLP of a 2-4 token prompt tail: where x is too wide for the fused
    gate/up kernel's LDS (Q4 from about 3400 columns at n = 3..4, Q8 from
    about 9400) the commit runs the two GEMVs and the glue unfused, with the
    same bits; where it fits, the fused kernel's result is the same. The up
    products are compared bit for bit, y to the north-star bar (the glue's
    SiLU can differ from the CPU's by 1 ulp)."""
    rng = np.random.default_rng(rows + cols + n)
    mats = {}
    for name, (r, c) in (("gate", (rows, cols)), ("up", (rows, cols)), ("down", (cols, rows))):
        m, qs, sc = quantized(orc, fmt, values(rng, r * c) * 0.1, r, c)
        gpu.upload(name, m)
        mats[name] = (qs, sc)
    x = values(rng, n * cols)
    y = np.zeros(n * cols, np.float32)
    gpu.mlp("gate", "up", "down", x, y, n)
    g = cpu_mode1(orc, fmt, *mats["gate"], x, n)
    u = cpu_mode1(orc, fmt, *mats["up"], x, n)
    assert np.array_equal(bits(gpu._aux["u"].view(count=n * rows)), bits(u.reshape(-1)))
    h = orc.silu_mul(g, u)
    ref = cpu_mode1(orc, fmt, *mats["down"], h, n).reshape(-1)
    ok, rel, ab = within_tolerance(y, ref)
    assert ok, (rel, ab)


def test_config2_lm_head_argmax(gpu, orc):
    qs, sc, x = synth.config2()
    gpu.upload("head", QuantMatrix.q8(qs, sc))
    logits = np.zeros(151936, np.float32)
    token = gpu.apply_argmax("head", x, logits)
    ref = orc.gemm_q8(qs, sc, x, 1, threads=8, mode=1)[0]
    assert np.array_equal(bits(logits), bits(ref))
    assert token == orc.argmax(ref)


def test_config3_prefill_gemm(gpu, orc):
    qs, sc, xs = synth.config3()
    gpu.upload("w", QuantMatrix.q4(qs, sc))
    y = np.zeros(512 * 6144, np.float32)
    gpu.apply("w", xs, y, 512)
    ref = orc.gemm_q4(qs, sc, xs, 512, threads=8, mode=1)
    ok, rel, ab = within_tolerance(y.reshape(512, 6144), ref)
    assert ok, (rel, ab)


def test_config4_vision_pair(gpu, orc):
    """BF16 -> Q8 on the GPU (bit-exact), then fc1 -> GELU -> fc2 at M=1024.
    fc2's K of 4304 runs zero-padded to 4320; fc1 gets 16 zero rows so its
    output is already padded."""
    fc1, fc2, x = synth.config4()
    gpu.upload_bf16("fc1", fc1, 4304, 1152, rows_pad=4320)
    gpu.upload_bf16("fc2", fc2, 1152, 4304)
    q1, s1 = orc.quantize_q8_bf16(fc1)
    q2, s2 = orc.quantize_q8_bf16(fc2, 4320)
    g1, h1 = gpu.quantized("fc1")
    g2, h2 = gpu.quantized("fc2")
    assert np.array_equal(g1[:4304], q1) and np.array_equal(bits(h1[:4304]), bits(s1))
    assert not g1[4304:].any() and not h1[4304:].any()
    assert np.array_equal(g2, q2) and np.array_equal(bits(h2), bits(s2))
    # Stage-wise, as the glue's parity is: each stage's CPU reference takes
    # the GPU's own input to that stage (a 1-ulp difference upstream can move
    # a value across a Q8 rounding boundary of the next input quantizer).
    y = np.zeros(1024 * 1152, np.float32)
    h = np.zeros(1024 * 4320, np.float32)
    gpu.gelu_pair("fc1", "fc2", x, y, 1024, intermediate=h)
    h = h.reshape(1024, 4320)
    a = np.zeros(1024 * 4320, np.float32)
    gpu.apply("fc1", x, a, 1024)
    a = a.reshape(1024, 4320)
    ok, rel, ab = within_tolerance(a[:, :4304], orc.gemm_q8(q1, s1, x, 1024, threads=8, mode=1))
    assert ok, ("fc1", rel, ab)
    assert not a[:, 4304:].any()
    assert np.array_equal(bits(h), bits(orc.gelu(a)))          # GELU stage, bit-exact
    ref = orc.gemm_q8(q2, s2, h, 1024, threads=8, mode=1)       # fc2 stage
    ok, rel, ab = within_tolerance(y.reshape(1024, 1152), ref)
    assert ok, ("fc2", rel, ab)


def test_profile_and_device_queries(gpu, orc):
    import ctypes
    from dianoia_amd import _lib
    lib = _lib.load()
    name = ctypes.create_string_buffer(256)
    lib.lab_gpu_device_name(name, 256)
    assert b"gfx950" in name.value
    assert lib.lab_gpu_max_buffer_length() > (1 << 30)
    lib.lab_gpu_set_profiling(1)
    m, _, _ = quantized(orc, "q8", values(np.random.default_rng(0), 64 * 64), 64, 64)
    gpu.upload("p", m)
    gpu.apply("p", np.ones(64, np.float32), np.zeros(64, np.float32), 1)
    lib.lab_gpu_set_profiling(0)
    ms = (ctypes.c_double * 21)()
    counts = (ctypes.c_int64 * 21)()
    assert lib.lab_gpu_profile(ms, counts, 18) == 21
    assert counts[13] == 1 and ms[13] > 0  # gemv_q8_i8
    assert lib.lab_gpu_last_ms() > 0


def test_invalid_dispatch_fails_its_commit(gpu_ready):
    from dianoia_amd import _lib
    lib = _lib.load()
    h = lib.lab_gpu_buffer(1024)
    try:
        lib.lab_gpu_begin()
        lib.lab_gpu_enc_matmul_q8(h, 0, 512, h, 0, h, 0, 64, 96, 1)  # qs past the end
        assert lib.lab_gpu_commit(1) == 0
        lib.lab_gpu_begin()
        assert lib.lab_gpu_commit(1) == 1
    finally:
        lib.lab_gpu_release(h)


# ------------------------------------------------------------ float inputs

@pytest.fixture()
def float_inputs(gpu_ready):
    was = set_int8_inputs(False)
    yield
    set_int8_inputs(was)


def cpu_mode0(orc, fmt, qs, sc, xs, n):
    return (orc.gemm_q4 if fmt == "q4" else orc.gemm_q8)(qs, sc, xs, n, threads=4, mode=0)


@pytest.mark.parametrize("fmt,rows,cols,n", [("q4", 64, 64, 1), ("q4", 70, 96, 13),
                                             ("q8", 36, 64, 9), ("q8", 128, 128, 40)])
def test_float_inputs_match_the_cpu_kernels(float_inputs, gpu, orc, fmt, rows, cols, n):
    """The reference test as written: GPU vs CPU with float inputs, within
    1e-4 + 1e-5 |cpu| (gpu_linear_test.dart:44); for n <= 4 (the exact
    float-input GEMV) also bit-exact."""
    rng = np.random.default_rng(5)
    m, qs, sc = quantized(orc, fmt, values(rng, rows * cols), rows, cols)
    gpu.upload("m", m)
    xs = values(rng, n * cols)
    on_gpu = np.zeros(n * rows, np.float32)
    gpu.apply("m", xs, on_gpu, n)
    cpu = cpu_mode0(orc, fmt, qs, sc, xs, n).reshape(-1)
    assert np.all(np.abs(on_gpu - cpu) <= 1e-4 + 1e-5 * np.abs(cpu))
    if n <= 4:
        assert np.array_equal(bits(on_gpu), bits(cpu))


@pytest.mark.parametrize("fmt,n", [("q8", 1), ("q4", 3), ("q8", 9)])
def test_float_inputs_wider_than_the_gemv(float_inputs, gpu, orc, fmt, n):
    """x rows of 40960 floats: more than the exact float GEMV's LDS holds
    (one token's fp32 x fits up to about 35000 columns), so the route falls
    back to the bf16-MFMA float GEMM, any width; its outputs meet the
    reference GPU test's bar against CPU mode 0 and the reference kernels'
    own bar (error / sum|terms| < 1e-5) against the exact products."""
    from test_gpu_gemm_float import exact_mode0
    rows, cols = 48, 40960
    rng = np.random.default_rng(7 + n)
    m, qs, sc = quantized(orc, fmt, values(rng, rows * cols), rows, cols)
    gpu.upload("wide", m)
    xs = values(rng, n * cols)
    on_gpu = np.zeros(n * rows, np.float32)
    gpu.apply("wide", xs, on_gpu, n)
    cpu = cpu_mode0(orc, fmt, qs, sc, xs, n).reshape(-1)
    assert np.all(np.abs(on_gpu - cpu) <= 1e-4 + 1e-5 * np.abs(cpu))
    exact, mag = exact_mode0(fmt, qs, sc, xs.reshape(n, cols))
    assert np.all(np.abs(on_gpu.reshape(n, rows).astype(np.float64) - exact) <= 1e-5 * mag)


def test_float_inputs_grow_buffers_and_keep_matrices(float_inputs, gpu, orc):
    rng = np.random.default_rng(6)
    small, sq, ss = quantized(orc, "q4", values(rng, 32 * 32), 32, 32)
    large, lq, ls = quantized(orc, "q4", values(rng, 64 * 256), 64, 256)
    gpu.upload("small", small)
    gpu.upload("large", large)
    for name, (q, s), rows, cols, n in [("small", (sq, ss), 32, 32, 3),
                                        ("large", (lq, ls), 64, 256, 50),
                                        ("small", (sq, ss), 32, 32, 7)]:
        xs = values(rng, n * cols)
        on_gpu = np.zeros(n * rows, np.float32)
        gpu.apply(name, xs, on_gpu, n)
        want = cpu_mode0(orc, "q4", q, s, xs, n).reshape(-1)
        if n <= 4:
            assert np.array_equal(bits(on_gpu), bits(want))
        else:  # the float GEMM: the reference GPU test's bar
            assert np.all(np.abs(on_gpu - want) <= 1e-4 + 1e-5 * np.abs(want))


def test_float_inputs_mlp_and_lm_head(float_inputs, gpu, orc):
    """With float inputs the MLP and the LM head run unfused (the fused
    kernels take int8 inputs); gate, up and the logits are mode-0 exact, the
    token is argmaxToken of them."""
    (gq, gs), (uq, us), (dq, ds), x = synth.config1()
    for name, (q, s) in (("gate", (gq, gs)), ("up", (uq, us)), ("down", (dq, ds))):
        gpu.upload(name, QuantMatrix.q4(q, s))
    y = np.zeros(2048, np.float32)
    gpu.mlp("gate", "up", "down", x, y, 1)
    g = orc.gemm_q4(gq, gs, x, 1, threads=8, mode=0)
    u = orc.gemm_q4(uq, us, x, 1, threads=8, mode=0)
    assert np.array_equal(bits(gpu._aux["u"].view(count=6144)), bits(u[0]))
    h = orc.silu_mul(g, u)
    ref = orc.gemm_q4(dq, ds, h, 1, threads=8, mode=0)[0]
    ok, rel, ab = within_tolerance(y, ref)  # the glue may differ by 1 ulp (double exp)
    assert ok, (rel, ab)
    rng = np.random.default_rng(9)
    qs, sc = synth.q8_weights(rng, 5000, 512)
    gpu.upload("head", QuantMatrix.q8(qs, sc))
    xs = synth.activations(rng, 1, 512)
    logits = np.zeros(5000, np.float32)
    token = gpu.apply_argmax("head", xs[0], logits)
    want = orc.gemm_q8(qs, sc, xs, 1, threads=8, mode=0)[0]
    assert np.array_equal(bits(logits), bits(want))
    assert token == orc.argmax(want)


def test_input_mode_switch_returns_previous(gpu_ready):
    was = set_int8_inputs(False)
    try:
        assert set_int8_inputs(True) is False
        assert set_int8_inputs(True) is True
    finally:
        set_int8_inputs(was)


def test_q8_batch_with_x_at_any_float_offset(gpu, orc):
    """The Q8 batch route on prepacked operands (1152 x 1152 at 1024 tokens)
    reads x 16 bytes at a time; lab_gpu_enc_matmul_q8 takes x at any float
    offset. At offsets 1..3 floats the command takes the int8 route, at 0
    and 4 the prepacked one: all within the bar of the CPU kernel."""
    rows, cols, n = 1152, 1152, 1024
    rng = np.random.default_rng(31)
    qs, sc = orc.quantize_q8((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
    xs = synth.activations(rng, n, cols)
    gpu.upload("w", QuantMatrix.q8(qs, sc))
    lib, w = gpu._lib, gpu._matrix("w")
    x = gpu._aux_buffer("x_off8", n * cols + 4)
    y = gpu._aux_buffer("y_off8", n * rows)
    ref = orc.gemm_q8(qs, sc, xs, n, threads=8, mode=1)
    for off in (1, 2, 3, 0, 4):
        v = x.view(count=n * cols + 4)
        v[:] = np.nan
        v[off:off + n * cols] = xs.reshape(-1)
        y.view(count=n * rows)[:] = np.nan
        lib.lab_gpu_begin()
        w.encode(lib, x.handle, y.handle, 0, n, x_offset=off * 4)
        gpu._finish()
        out = y.view(count=n * rows).reshape(n, rows).copy()
        ok, rel, ab = within_tolerance(out, ref)
        assert ok, (off, rel, ab)


@pytest.mark.parametrize("rows,cols,n", [(768, 768, 13), (768, 768, 375), (4096, 1024, 320)])
def test_q4_prefill_with_x_at_any_float_offset(gpu, orc, rows, cols, n):
    """The Q4 prefill routes with fp6 kernels (the chunk GEMM on the prepack
    for 5..512 tokens, the tiled fp6 GEMM for 320+ tokens on 4096+ rows)
    read x 16 bytes at a time; lab_gpu_enc_matmul_q4 takes x at any float
    offset. At offsets 1..3 floats the command takes the int8 route, at 0
    and 4 the fp6 route: all within the bar of the CPU kernel."""
    rng = np.random.default_rng(rows + n)
    qs, sc = synth.q4_weights(rng, rows, cols)
    xs = synth.activations(rng, n, cols)
    gpu.upload("w", QuantMatrix.q4(qs, sc))
    lib, w = gpu._lib, gpu._matrix("w")
    x = gpu._aux_buffer("x_off", n * cols + 4)
    y = gpu._aux_buffer("y_off", n * rows)
    ref = orc.gemm_q4(qs, sc, xs, n, threads=8, mode=1)
    for off in (1, 2, 3, 0, 4):
        v = x.view(count=n * cols + 4)
        v[:] = np.nan
        v[off:off + n * cols] = xs.reshape(-1)
        y.view(count=n * rows)[:] = np.nan
        lib.lab_gpu_begin()
        w.encode(lib, x.handle, y.handle, 0, n, x_offset=off * 4)
        gpu._finish()
        out = y.view(count=n * rows).reshape(n, rows).copy()
        ok, rel, ab = within_tolerance(out, ref)
        assert ok, (off, rel, ab)


@pytest.mark.parametrize("n", [13, 320])
def test_q4_prefill_follows_gpu_writes_into_the_weights(gpu, orc, n):
    """The Q4 prefill routes run on a prepacked copy of the weights made at
    their first use (13 tokens: the chunk GEMM; 320 on 4096 rows: the tiled
    fp6 GEMM). A GPU command that writes other weights into the same region
    (lab_gpu_enc_quantize_q4 again, from other fp32 values) makes the next
    prefill use them, and writing the first weights back returns to those:
    each product against the CPU kernel on the weights of the moment."""
    rows, cols = 4096, 1024
    rng = np.random.default_rng(17 + n)
    ws = [(rng.standard_normal((rows, cols)) * 0.02).astype(np.float32) for _ in range(2)]
    gpu.upload_f32("w", ws[0], rows, cols, fmt="q4")
    lib, m = gpu._lib, gpu._matrix("w")
    src = gpu._aux_buffer("w_src", rows * cols)
    xs = synth.activations(rng, n, cols)
    for step, k in enumerate((0, 1, 0)):
        if step > 0:   # weights k into the same region, on the GPU
            src.view(count=rows * cols)[:] = ws[k].reshape(-1)
            lib.lab_gpu_begin()
            lib.lab_gpu_enc_quantize_q4(src.handle, 0, m.buffer, m.qs, m.buffer, m.scales,
                                        rows, cols)
            gpu._finish()
        y = np.zeros(n * rows, np.float32)
        gpu.apply("w", xs, y, n)
        qs, sc = orc.quantize_q4(ws[k])
        ok, rel, ab = within_tolerance(y.reshape(n, rows), orc.gemm_q4(qs, sc, xs, n, threads=8,
                                                                         mode=1))
        assert ok, (k, rel, ab)


def test_q8_batch_follows_gpu_writes_into_the_weights(gpu, orc):
    """A Q8 batch of 256+ tokens (1024 x 1024 at 4096 tokens) runs on
    a prepacked copy of the weights made at its first use (the int8 GEMM on
    prepacked operands). A GPU command that writes other weights into the
    same region (lab_gpu_enc_quantize_q8 again) makes the next product use
    them, and writing the first weights back returns to those: each product
    against the CPU kernel on the weights of the moment."""
    from dianoia_amd import device as D
    rows, cols, n = 1024, 1024, 4096
    assert D.gemm_q8_i8p_tile(rows, cols, n) is not None
    rng = np.random.default_rng(23)
    ws = [(rng.standard_normal((rows, cols)) * 0.02).astype(np.float32) for _ in range(2)]
    gpu.upload_f32("w", ws[0], rows, cols, fmt="q8")
    lib, m = gpu._lib, gpu._matrix("w")
    src = gpu._aux_buffer("w_src", rows * cols)
    xs = synth.activations(rng, n, cols)
    for step, k in enumerate((0, 1, 0)):
        if step > 0:   # weights k into the same region, on the GPU
            src.view(count=rows * cols)[:] = ws[k].reshape(-1)
            lib.lab_gpu_begin()
            lib.lab_gpu_enc_quantize_q8(src.handle, 0, m.buffer, m.qs, m.buffer, m.scales,
                                        rows, cols, cols)
            gpu._finish()
        y = np.zeros(n * rows, np.float32)
        gpu.apply("w", xs, y, n)
        qs, sc = orc.quantize_q8(ws[k])
        ok, rel, ab = within_tolerance(y.reshape(n, rows), orc.gemm_q8(qs, sc, xs, n, threads=8,
                                                                         mode=1))
        assert ok, (k, rel, ab)


def test_q8_batch_and_q4_chunk_of_one_x_keep_their_own_panels(gpu, orc):
    """One x read in one command buffer by a Q8 batch (the int8 panel) and
    then by Q4 prefill matmuls (the fp6 panel), then Q8 again: each route
    quantizes x into its own panel format (the workspace's panel is keyed
    by format as well as by x), every product against the CPU kernel."""
    rng = np.random.default_rng(29)
    n, cols = 256, 4096
    q8r, q4r = 4096, 1024
    q8qs, q8sc = synth.q8_weights(rng, q8r, cols)
    q8sc = (q8sc / np.float32(16)).astype(np.float16).astype(np.float32)
    q4qs, q4sc = synth.q4_weights(rng, q4r, cols)
    gpu.upload("a", QuantMatrix.q8(q8qs, q8sc))
    gpu.upload("b", QuantMatrix.q4(q4qs, q4sc))
    lib = gpu._lib
    x = gpu._aux_buffer("x_fmt", n * cols)
    ya = gpu._aux_buffer("y_a", n * q8r)
    yb = gpu._aux_buffer("y_b", n * q4r)
    ya2 = gpu._aux_buffer("y_a2", n * q8r)
    xs = synth.activations(rng, n, cols)
    x.view(count=n * cols)[:] = xs.reshape(-1)
    ref8 = orc.gemm_q8(q8qs, q8sc, xs, n, threads=8, mode=1)
    ref4 = orc.gemm_q4(q4qs, q4sc, xs, n, threads=8, mode=1)
    for rep in range(2):   # the first pass also makes the prepacks
        lib.lab_gpu_begin()
        gpu._matrix("a").encode(lib, x.handle, ya.handle, 0, n)
        gpu._matrix("b").encode(lib, x.handle, yb.handle, 0, n)
        gpu._matrix("a").encode(lib, x.handle, ya2.handle, 0, n)
        gpu._finish()
        for name, y, ref, rows in (("a", ya, ref8, q8r), ("b", yb, ref4, q4r),
                                   ("a2", ya2, ref8, q8r)):
            ok, rel, ab = within_tolerance(y.view(count=n * rows).reshape(n, rows), ref)
            assert ok, (rep, name, rel, ab)


def test_q4_prefill_matmuls_of_one_x_share_its_panel(gpu, orc):
    """Prepacked Q4 prefill matmuls that read the same x in one command
    buffer (a chunk's q, k, v or gate, up) quantize x once and share the
    panel. A command that writes x in between (a copy into it) makes the
    next matmul quantize the new x, and so does a host write between
    commits: every product against the CPU kernel on the x of its moment,
    and the profile counts one activation quantize per distinct x."""
    import ctypes
    rng = np.random.default_rng(41)
    n, cols = 13, 1024
    shapes = {"a": 768, "b": 1536, "c": 512}
    mats = {}
    for name, rows in shapes.items():
        qs, sc = synth.q4_weights(rng, rows, cols)
        gpu.upload(name, QuantMatrix.q4(qs, sc))
        mats[name] = (qs, sc)
    lib = gpu._lib
    x = gpu._aux_buffer("x_share", n * cols)
    x2 = gpu._aux_buffer("x_other", n * cols)
    ys = {name: gpu._aux_buffer("y_" + name, n * rows) for name, rows in shapes.items()}
    xa = synth.activations(rng, n, cols)
    xb = synth.activations(rng, n, cols)

    def check(name, xs):
        rows = shapes[name]
        qs, sc = mats[name]
        out = ys[name].view(count=n * rows).reshape(n, rows)
        ok, rel, ab = within_tolerance(out, orc.gemm_q4(qs, sc, xs, n, threads=8, mode=1))
        assert ok, (name, rel, ab)

    ms = (ctypes.c_double * 21)()
    counts = (ctypes.c_int64 * 21)()
    quantize = 10
    for rep in range(2):   # the first pass also makes the prepacks
        x.view(count=n * cols)[:] = xa.reshape(-1)
        x2.view(count=n * cols)[:] = xb.reshape(-1)
        lib.lab_gpu_profile(ms, counts, 21)
        lib.lab_gpu_set_profiling(1)
        lib.lab_gpu_begin()
        gpu._matrix("a").encode(lib, x.handle, ys["a"].handle, 0, n)
        gpu._matrix("b").encode(lib, x.handle, ys["b"].handle, 0, n)
        lib.lab_gpu_enc_copy(x2.handle, 0, x.handle, 0, n * cols)
        gpu._matrix("c").encode(lib, x.handle, ys["c"].handle, 0, n)
        gpu._finish()
        lib.lab_gpu_set_profiling(0)
        lib.lab_gpu_profile(ms, counts, 21)
        check("a", xa)
        check("b", xa)
        check("c", xb)
        assert counts[quantize] == 2, list(counts)
    # A host write between commits: the panel is made again.
    x.view(count=n * cols)[:] = xa.reshape(-1)
    lib.lab_gpu_begin()
    gpu._matrix("c").encode(lib, x.handle, ys["c"].handle, 0, n)
    gpu._finish()
    check("c", xa)


def test_q4_prefill_inputs_from_norm_add_norm_and_swiglu_bring_their_panel(gpu, orc):
    """An RMSNorm, a residual add + RMSNorm or a SwiGLU whose output is the x
    of the prefill matmul right after it (a chunk's q/k/v, gate/up and down
    projections) writes x's activation panel too, and the matmul uses it:
    one command buffer gives the same bits as each command committed on its
    own, and the profile counts one activation quantize per x. A matmul of
    another x after the producer quantizes its own."""
    import ctypes
    rng = np.random.default_rng(43)
    n, cols, rows = 13, 1024, 768
    qs, sc = synth.q4_weights(rng, rows, cols)
    gpu.upload("a", QuantMatrix.q4(qs, sc))
    qs2, sc2 = synth.q4_weights(rng, cols, rows)
    gpu.upload("d", QuantMatrix.q4(qs2, sc2))
    lib = gpu._lib
    count = n * cols
    bufs = {k: gpu._aux_buffer("pp_" + k, count) for k in ("x", "m", "h", "o", "g", "u")}
    w = gpu._aux_buffer("pp_w", cols)
    ys = {k: gpu._aux_buffer("pp_y" + k, n * cols) for k in ("1", "2", "3", "4")}
    inputs = {k: synth.activations(rng, n, cols).reshape(-1) for k in ("x", "m", "o")}
    gu = (rng.standard_normal((2, n * rows)) * 2).astype(np.float32)
    w.view(count=cols)[:] = (1 + rng.standard_normal(cols) * 0.1).astype(np.float32)

    def encode():
        h = bufs
        yield lambda: lib.lab_gpu_enc_rms_norm(h["x"].handle, 0, w.handle, 0, h["h"].handle, 0,
                                               n, cols, 1e-6, 0)
        yield lambda: gpu._matrix("a").encode(lib, h["h"].handle, ys["1"].handle, 0, n)
        yield lambda: lib.lab_gpu_enc_add(h["m"].handle, 0, h["x"].handle, 0, count)
        yield lambda: lib.lab_gpu_enc_rms_norm(h["x"].handle, 0, w.handle, 0, h["h"].handle, 0,
                                               n, cols, 1e-6, 0)
        yield lambda: gpu._matrix("a").encode(lib, h["h"].handle, ys["2"].handle, 0, n)
        yield lambda: lib.lab_gpu_enc_swiglu(h["g"].handle, h["u"].handle, n * rows)
        yield lambda: gpu._matrix("d").encode(lib, h["g"].handle, ys["3"].handle, 0, n)
        yield lambda: lib.lab_gpu_enc_rms_norm(h["x"].handle, 0, w.handle, 0, h["h"].handle, 0,
                                               n, cols, 1e-6, 0)
        yield lambda: gpu._matrix("a").encode(lib, h["o"].handle, ys["4"].handle, 0, n)

    def run(together):
        for k, v in inputs.items():
            bufs[k].view(count=count)[:] = v
        bufs["g"].view(count=n * rows)[:] = gu[0]
        bufs["u"].view(count=n * rows)[:] = gu[1]
        for y in ys.values():
            y.view(count=n * cols)[:] = np.nan
        if together:
            lib.lab_gpu_begin()
            for enc in encode():
                enc()
            gpu._finish()
        else:
            for enc in encode():
                lib.lab_gpu_begin()
                enc()
                gpu._finish()
        return {k: y.view(count=n * cols).copy() for k, y in ys.items()}

    ms = (ctypes.c_double * 21)()
    counts = (ctypes.c_int64 * 21)()
    quantize = 10
    run(True)   # makes the prepacks
    apart = run(False)
    lib.lab_gpu_profile(ms, counts, 21)
    lib.lab_gpu_set_profiling(1)
    together = run(True)
    lib.lab_gpu_set_profiling(0)
    lib.lab_gpu_profile(ms, counts, 21)
    for k in ys:
        assert np.array_equal(bits(apart[k]), bits(together[k])), k
    assert counts[quantize] == 4, list(counts)
    # Against the CPU kernels on the inputs of each matmul.
    x1 = orc.rms_norm(inputs["x"].reshape(n, cols), w.view(count=cols).copy(), 1e-6)
    ok, rel, ab = within_tolerance(together["1"][:n * rows].reshape(n, rows),
                                   orc.gemm_q4(qs, sc, x1, n, threads=8, mode=1))
    assert ok, (rel, ab)


@pytest.mark.parametrize("n", [200, 300])
def test_q4_prefill_after_a_norm_with_or_without_its_panel(gpu, orc, n):
    """An RMSNorm of up to 256 rows writes the next prefill matmul's panel;
    one of more rows cannot (its kernel holds a row per workgroup only up
    to 256 rows), so the matmul quantizes its input itself: either way one
    command buffer gives the bits of one command per commit, within the bar
    of the CPU kernels."""
    rng = np.random.default_rng(47 + n)
    cols, rows = 1024, 768
    qs, sc = synth.q4_weights(rng, rows, cols)
    gpu.upload("a", QuantMatrix.q4(qs, sc))
    lib = gpu._lib
    x = gpu._aux_buffer("pf_x", n * cols)
    h = gpu._aux_buffer("pf_h", n * cols)
    w = gpu._aux_buffer("pf_w", cols)
    y = gpu._aux_buffer("pf_y", n * rows)
    xs = synth.activations(rng, n, cols)
    wv = (1 + rng.standard_normal(cols) * 0.1).astype(np.float32)
    w.view(count=cols)[:] = wv

    def run(together):
        x.view(count=n * cols)[:] = xs.reshape(-1)
        y.view(count=n * rows)[:] = np.nan
        cmds = [lambda: lib.lab_gpu_enc_rms_norm(x.handle, 0, w.handle, 0, h.handle, 0, n, cols,
                                                 1e-6, 0),
                lambda: gpu._matrix("a").encode(lib, h.handle, y.handle, 0, n)]
        if together:
            lib.lab_gpu_begin()
            for c in cmds:
                c()
            gpu._finish()
        else:
            for c in cmds:
                lib.lab_gpu_begin()
                c()
                gpu._finish()
        return y.view(count=n * rows).copy()

    run(True)   # makes the prepack
    apart, together = run(False), run(True)
    assert np.array_equal(bits(apart), bits(together))
    hn = orc.rms_norm(xs, wv, 1e-6)
    ok, rel, ab = within_tolerance(together.reshape(n, rows),
                                   orc.gemm_q4(qs, sc, hn, n, threads=8, mode=1))
    assert ok, (rel, ab)
