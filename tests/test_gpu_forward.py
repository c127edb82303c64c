"""A whole decoder pass through the lab_gpu_* ABI, encoded command for
command as the reference's GpuForward.forward does (lib/src/gpu.dart:
1036-1239), on random weights (dianoia_amd/forward.py).

* One command buffer per pass (the reference's) against one command buffer
  per command: the same bits for logits, KV rows and conv histories, so the
  commit's fusions and its host-view staging change nothing.
* Every command of a pass against the CPU oracle, on the inputs the host
  views hold before it (the stage-wise check the reference's own tests do).
* Host writes between command buffers reach the GPU: a restored state
  (gpu.dart:1003-1021) reproduces a pass bit for bit, and garbage written
  into KV rows changes the next token's logits.
* With host-write tracking on, a decode step uploads only what the host
  wrote (the token's embedding and RoPE row), not the KV history.
"""

import os
import subprocess
import tempfile
import sys

import numpy as np
import pytest

from dianoia_amd import forward as F
from gpu_util import bits

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def qwen3_small():
    return F.ForwardConfig(hidden=256, intermediate=512, heads=4, kv_heads=2, head_dim=64,
                           vocab=997, layer_types=[F.FULL, F.FULL], eps=1e-6)


CONFIGS = {"lfm3": F.lfm3_small, "qwen3": qwen3_small}
# (n, position) chunks of a sequence: a 6-token prefill (quantize + GEMM),
# decode steps (exact GEMVs, the gate/up fusion), a 3-token chunk.
PLAN = [(6, 0), (1, 6), (1, 7), (3, 8), (1, 11)]


def embeddings(cfg, position, n):
    rng = np.random.default_rng(1000 + position)
    return (rng.standard_normal(n * cfg.hidden) * 0.5).astype(np.float32)


def run(fwd, plan):
    """Runs the chunks; returns per chunk (logits, histories + KV rows)."""
    out = []
    for n, pos in plan:
        fwd.residual[:n * fwd.config.hidden] = embeddings(fwd.config, pos, n)
        fwd.forward(n, pos)
        out.append((fwd.logits.copy(), [b.copy() for b in fwd.state_blocks(pos + n)]))
    return out


def same(a, b):
    return np.array_equal(bits(a), bits(b))


@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_one_command_buffer_equals_one_per_command(gpu_ready, name):
    cfg = CONFIGS[name]()
    fused = F.GpuForward(cfg, max_seq=16, max_chunk=8, seed=3)
    split = F.GpuForward(cfg, max_seq=16, max_chunk=8, seed=3)
    split.split_commits = True
    try:
        a, b = run(fused, PLAN), run(split, PLAN)
        for (la, sa), (lb, sb), chunk in zip(a, b, PLAN):
            assert same(la, lb), f"logits differ after chunk {chunk}"
            assert all(same(x, y) for x, y in zip(sa, sb)), f"state differs after chunk {chunk}"
            assert np.isfinite(la).all()
    finally:
        fused.dispose()
        split.dispose()


def run_meanwhile(fwd, plan, work):
    """run() with every chunk committed without waiting and `work` run on the
    host while the GPU computes (GpuForward.forward(meanwhile:))."""
    out = []
    for n, pos in plan:
        fwd.residual[:n * fwd.config.hidden] = embeddings(fwd.config, pos, n)
        fwd.forward(n, pos, meanwhile=work)
        out.append((fwd.logits.copy(), [b.copy() for b in fwd.state_blocks(pos + n)]))
    return out


@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_forward_meanwhile_equals_waiting_commit(gpu_ready, name):
    """forward(meanwhile=...) (lab_gpu_commit(0), host work, lab_gpu_wait)
    leaves the logits, KV rows and conv histories of a waiting commit bit for
    bit, and runs the host work once per pass (forward_meanwhile_test.dart:
    23-47). The work computes on the host while the copy-backs of the pass
    are still landing in the pinned views."""
    cfg = CONFIGS[name]()
    plain = F.GpuForward(cfg, max_seq=16, max_chunk=8, seed=3)
    overlap = F.GpuForward(cfg, max_seq=16, max_chunk=8, seed=3)
    runs = []

    def work():
        rng = np.random.default_rng(len(runs))
        a = rng.standard_normal((256, 256))
        runs.append(float(np.linalg.norm(a @ a.T)))

    try:
        a, b = run(plain, PLAN), run_meanwhile(overlap, PLAN, work)
        assert len(runs) == len(PLAN)
        for (la, sa), (lb, sb), chunk in zip(a, b, PLAN):
            assert same(la, lb), f"logits differ after chunk {chunk}"
            assert all(same(x, y) for x, y in zip(sa, sb)), f"state differs after chunk {chunk}"
    finally:
        plain.dispose()
        overlap.dispose()


def test_forward_meanwhile_error_comes_after_the_pass(gpu_ready):
    """An error raised by the host work propagates after the pass has waited
    for the GPU (gpu.dart:1226-1233); the pass's results stand in its
    buffers and the next step continues from them. As in GpuForward, the
    raise skips the copy into ``logits`` (TextModel defers the error past
    that copy, model.dart:753-784, which forward_meanwhile_test.dart:57-66
    checks one level up): the logits buffer's view holds the pass's."""
    cfg = qwen3_small()
    plain = F.GpuForward(cfg, max_seq=16, max_chunk=8, seed=3)
    failing = F.GpuForward(cfg, max_seq=16, max_chunk=8, seed=3)

    def boom():
        raise ValueError("meanwhile")

    try:
        want = run(plain, PLAN)
        n, pos = PLAN[0]
        failing.residual[:n * cfg.hidden] = embeddings(cfg, pos, n)
        with pytest.raises(ValueError, match="meanwhile"):
            failing.forward(n, pos, meanwhile=boom)
        assert same(failing._logits.view, want[0][0])
        rest = run(failing, PLAN[1:])
        for (la, sa), (lb, sb) in zip(want[1:], rest):
            assert same(la, lb) and all(same(x, y) for x, y in zip(sa, sb))
    finally:
        plain.dispose()
        failing.dispose()


def test_decode_step_fuses_norms_and_adds(gpu_ready):
    """A one-token step dispatches no standalone RMSNorm or residual add:
    each RMSNorm runs in the prologue of the GEMV that reads it and each add
    in the epilogue of the GEMV whose output it adds (the commit's fusions,
    checked for their bits by the test above); the same step one command per
    commit runs them all. The profile still counts each of them once (with
    no time of its own when fused)."""
    import ctypes
    from dianoia_amd import _lib
    lib = _lib.load()
    cfg = qwen3_small()
    ms = (ctypes.c_double * 21)()

    def profiled_step(fwd):
        fwd.residual[:6 * cfg.hidden] = embeddings(cfg, 0, 6)
        fwd.forward(6, 0)
        lib.lab_gpu_profile(ms, (ctypes.c_int64 * 21)(), 21)  # clear the counts
        lib.lab_gpu_set_profiling(1)
        fwd.residual[:cfg.hidden] = embeddings(cfg, 6, 1)
        fwd.forward(1, 6)
        lib.lab_gpu_set_profiling(0)
        counts = (ctypes.c_int64 * 21)()
        assert lib.lab_gpu_profile(ms, counts, 21) == 21
        return list(counts), list(ms)

    fused = F.GpuForward(cfg, max_seq=16, max_chunk=8, seed=3)
    split = F.GpuForward(cfg, max_seq=16, max_chunk=8, seed=3)
    split.split_commits = True
    try:
        (a, a_ms), (b, b_ms) = profiled_step(fused), profiled_step(split)
    finally:
        fused.dispose()
        split.dispose()
    rms_norm, add, gemv_q8, gemv_q4 = 4, 17, 13, 14
    layers = len(cfg.layer_types)
    assert b[rms_norm] == 2 * layers + 1 and b[add] == 2 * layers, b
    assert b[gemv_q8] + b[gemv_q4] > 0, b
    # A fused launch counts every command it ran under that command's kind
    # (its time goes to its main kernel's kind), so the counts per kind are
    # those of one launch per command.
    assert a == b, (a, b)
    assert a_ms[rms_norm] == 0 and a_ms[add] == 0, a_ms
    assert b_ms[rms_norm] > 0 and b_ms[add] > 0, b_ms


class StageCheck:
    """checker for GpuForward.split_commits: each command against the oracle
    on the host views before it. Matmuls (n <= 4, exact GEMV) and the conv,
    add and copy are bit-exact; reductions run in another order (RMSNorm,
    norm + RoPE, attention: 1e-5 relative + 1e-6 absolute); the SiLU glue
    within 2 ulp of the oracle's double-precision result."""

    def __init__(self, orc, fwd):
        self.orc, self.fwd = orc, fwd
        self.buf = {b.handle: b for b in fwd._buffers}
        mats = [fwd._lm_head]
        for l in fwd._layers:
            mats += [m for m in (l.w1, l.w3, l.w2, l.in_proj, l.out_proj, l.q, l.k, l.v, l.gate, l.o)
                     if m is not None]
        self.mat = {m.buffer: m for m in mats}
        self.kinds = {}

    def view(self, handle, offset_bytes, count):
        v = self.buf[handle].view
        return v[offset_bytes // 4: offset_bytes // 4 + count].copy()

    def __call__(self, kind, args, fwd):
        self.kinds[kind] = self.kinds.get(kind, 0) + 1
        orc, cfg = self.orc, fwd.config
        if kind == "matmul":
            w, _, _, x, x_off, y, y_off, rows, cols, n = args
            m = self.mat[w]
            xs = self.view(x, x_off, n * cols).reshape(n, cols)
            qs, sc = m.qs_scales()
            want = (orc.gemm_q4 if m.q4 else orc.gemm_q8)(qs, sc, xs, n, threads=4, mode=1)

            def after():
                got = self.view(y, y_off, n * rows).reshape(n, rows)
                if n <= 4:
                    assert same(got, want), f"matmul {rows}x{cols} n={n} not bit-exact"
                else:
                    err = np.abs(got.astype(np.float64) - want)
                    assert np.all((err <= 1e-4 * np.abs(want)) | (err <= 1e-5)), "GEMM outside 1e-4"
            return after
        if kind == "rms_norm":
            x, x_off, w, w_off, out, out_off, rows, cols, eps, acc = args
            xs = self.view(x, x_off, rows * cols).reshape(rows, cols)
            ws = self.view(w, w_off, cols)
            base = self.view(out, out_off, rows * cols).reshape(rows, cols) if acc else None
            want = orc.rms_norm(xs, ws, eps, out=base)
            return lambda: self.close(self.view(out, out_off, rows * cols), want, kind)
        if kind == "head_norm_rope":
            x, x_off, stride, w, w_off, rope, rope_off, rope_stride, heads, hd, n, eps = args
            count = (n - 1) * stride + heads * hd
            xs = np.zeros(n * stride, np.float32)
            xs[:count] = self.view(x, x_off, count)
            table = np.zeros(n * rope_stride, np.float32)
            table[:(n - 1) * rope_stride + hd] = self.view(rope, rope_off, (n - 1) * rope_stride + hd)
            want = orc.head_norm_rope(xs.reshape(n, stride), stride, self.view(w, w_off, hd),
                                      table.reshape(n, rope_stride), rope_stride, heads, hd, n,
                                      eps).reshape(-1)[:count]
            return lambda: self.close(self.view(x, x_off, count), want, kind)
        if kind == "conv":
            bcx, weight, w_off, history, y, width, k, n = args
            want_y, want_h = orc.short_conv(self.view(bcx, 0, n * 3 * width),
                                            self.view(weight, w_off, width * k),
                                            self.view(history, 0, (k - 1) * width), width, k, n)

            def after():
                assert same(self.view(y, 0, n * width), want_y), "conv output"
                assert same(self.view(history, 0, (k - 1) * width), want_h.reshape(-1)), "history"
            return after
        if kind == "attention":
            q, keys, values, gate, out, position, n, heads, kv, hd, window = args
            rows = (position + n) * kv * hd
            want = orc.attention(self.view(q, 0, n * heads * hd), self.view(keys, 0, rows),
                                 self.view(values, 0, rows),
                                 None if gate < 0 else self.view(gate, 0, n * heads),
                                 position, n, heads, kv, hd, window)
            return lambda: self.close(self.view(out, 0, n * heads * hd), want, kind)
        if kind == "swiglu":
            g, u, count = args
            want = orc.silu_mul(self.view(g, 0, count), self.view(u, 0, count))

            def after():
                got = self.view(g, 0, count)
                ulp = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32))
                assert ulp.max() <= 2, "SiLU glue"
            return after
        if kind in ("add", "copy"):
            src, src_off, dst, dst_off, count = args
            s = self.view(src, src_off, count)
            want = s + self.view(dst, dst_off, count) if kind == "add" else s
            return lambda: self.close(self.view(dst, dst_off, count), want, kind, exact=True)
        raise AssertionError(f"unchecked command {kind}")

    @staticmethod
    def close(got, want, kind, exact=False):
        if exact:
            assert same(np.reshape(got, -1), np.reshape(want, -1)), kind
            return
        got = np.asarray(got, np.float64).reshape(-1)
        want = np.asarray(want, np.float64).reshape(-1)
        err = np.abs(got - want)
        assert np.all(err <= 1e-6 + 1e-5 * np.abs(want)), f"{kind}: max err {err.max()}"


@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_every_command_of_a_pass_against_the_oracle(gpu_ready, orc, name):
    cfg = CONFIGS[name]()
    fwd = F.GpuForward(cfg, max_seq=16, max_chunk=8, seed=5)
    fwd.split_commits = True
    check = StageCheck(orc, fwd)
    fwd.checker = check
    try:
        run(fwd, [(3, 0), (1, 3), (1, 4)])
    finally:
        fwd.dispose()
    want = {"matmul", "rms_norm", "head_norm_rope", "attention", "swiglu"}
    if name == "lfm3":
        want |= {"conv"}
    else:
        want |= {"add"}
    assert want <= set(check.kinds), check.kinds


@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_host_writes_between_commits_reach_the_gpu(gpu_ready, name):
    cfg = CONFIGS[name]()
    fwd = F.GpuForward(cfg, max_seq=16, max_chunk=8, seed=7)
    try:
        run(fwd, [(3, 0), (1, 3)])
        saved = [b.copy() for b in fwd.state_blocks(4)]
        first = run(fwd, [(1, 4), (1, 5)])
        # Restore the state at position 4 through the host views (histories
        # changed since; KV rows 0..3 are rewritten with their own values).
        for view, value in zip(fwd.state_blocks(4), saved):
            view[:] = value
        again = run(fwd, [(1, 4), (1, 5)])
        for (la, _), (lb, _) in zip(first, again):
            assert same(la, lb), "a restored state does not reproduce the pass"
        # Garbage in one attention layer's keys changes the next token ...
        blocks = fwd.state_blocks(4)
        keys = blocks[len(blocks) - 2]
        keep = keys.copy()
        keys[:] = np.random.default_rng(1).standard_normal(keys.size).astype(np.float32) * 4
        for view, value in zip(fwd.state_blocks(4)[:-2], saved[:-2]):
            view[:] = value
        changed = run(fwd, [(1, 4)])[0][0]
        assert not same(changed, first[0][0]), "a host write to the KV rows did not reach the GPU"
        # ... and writing the rows back restores it.
        keys[:] = keep
        for view, value in zip(fwd.state_blocks(4), saved):
            view[:] = value
        assert same(run(fwd, [(1, 4)])[0][0], first[0][0])
        # reset() clears the histories for a new sequence, through the views.
        fwd.reset()
        assert all((fwd.history(i) == 0).all() for i, l in enumerate(fwd._layers) if l.kind == F.CONV)
    finally:
        fwd.dispose()


def test_decode_step_uploads_only_host_writes(gpu_ready):
    """Tracking on (the default): a decode step at position 40 uploads the
    token's embedding and RoPE row (and nothing the host did not write),
    far less than the 40 rows of keys and values the attention layers read."""
    assert F.tracking_writes(), "host-write tracking should be on by default"
    cfg = qwen3_small()
    fwd = F.GpuForward(cfg, max_seq=64, max_chunk=8, seed=9)
    try:
        run(fwd, [(8, 0), (8, 8), (8, 16), (8, 24), (8, 32)])
        up0, down0 = F.transfer_bytes()
        run(fwd, [(1, 40)])
        up1, down1 = F.transfer_bytes()
        run(fwd, [(1, 41)])
        up2, _ = F.transfer_bytes()
    finally:
        fwd.dispose()
    kv_history = 2 * 41 * cfg.kv_dim * 4 * cfg.layers
    page = os.sysconf("SC_PAGESIZE")
    # The embedding (hidden floats) and the RoPE row (2 * hd floats), each
    # rounded up to whole pages.
    budget = 2 * page * (1 + (cfg.hidden * 4 + 2 * cfg.head_dim * 4) // page)
    for up in (up1 - up0, up2 - up1):
        assert up <= budget, f"decode step uploaded {up} bytes (KV history {kv_history})"
    assert down1 - down0 >= cfg.vocab * 4  # the logits come back


def test_tracking_off_uploads_the_history_and_agrees(gpu_ready):
    """DIANOIA_GPU_TRACK_WRITES=0 (a child process: the switch is read at
    lab_gpu_init): every read region is uploaded, including the KV history,
    and the logits are the same bits as with tracking."""
    script = os.path.join(ROOT, "tests", "forward_child.py")
    cfg = qwen3_small()
    fwd = F.GpuForward(cfg, max_seq=64, max_chunk=8, seed=9)
    try:
        run(fwd, [(8, 0), (8, 8), (1, 16)])
        want = fwd.logits.copy()
        up0, _ = F.transfer_bytes()
        run(fwd, [(1, 17)])
        up_tracked = F.transfer_bytes()[0] - up0
        want17 = fwd.logits.copy()
    finally:
        fwd.dispose()
    env = dict(os.environ, DIANOIA_GPU_TRACK_WRITES="0")
    with tempfile.TemporaryDirectory() as out_dir:
        r = subprocess.run([sys.executable, script, "plain", out_dir], env=env,
                           capture_output=True, text=True, timeout=300)
        assert r.returncode == 0, r.stderr[-2000:]
        out = dict(np.load(os.path.join(out_dir, "forward_child.npz")))
    assert int(out["tracking"]) == 0
    assert same(out["logits16"], want) and same(out["logits17"], want17)
    assert int(out["up17"]) >= up_tracked + 2 * 17 * cfg.kv_dim * 4 * cfg.layers


def test_replaced_segv_handler_turns_tracking_off(gpu_ready):
    """A SIGSEGV handler installed after lab_gpu_init (here the default
    action, in a child process) is noticed by the next lab_gpu_contents,
    which turns host-write tracking off and unprotects every page before
    the host writes through its views again: the pass then runs to the
    same logits as with tracking (a write to a still protected page would
    have ended the child)."""
    script = os.path.join(ROOT, "tests", "forward_child.py")
    cfg = qwen3_small()
    fwd = F.GpuForward(cfg, max_seq=64, max_chunk=8, seed=9)
    try:
        run(fwd, [(8, 0), (8, 8), (1, 16)])
        want = fwd.logits.copy()
    finally:
        fwd.dispose()
    with tempfile.TemporaryDirectory() as out_dir:
        r = subprocess.run([sys.executable, script, "replace-handler", out_dir],
                           capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, (r.returncode, r.stderr[-2000:])
        out = dict(np.load(os.path.join(out_dir, "forward_child_handler.npz")))
    assert int(out["before"]) == 1 and int(out["after"]) == 0
    assert same(out["logits16"], want)


# Head sizes of the split-key attention with the head norms folded in: its
# keys per split are 32 at hd 256, 128 at hd 64, 256 at hd 32, so each plan
# decodes past one split.
LONG_CONTEXT = {256: 40, 64: 160, 32: 264}


@pytest.mark.parametrize("hd", sorted(LONG_CONTEXT))
def test_long_context_decode_folds_head_norms(gpu_ready, hd):
    """Decode steps past one key split take the split-key attention, where
    the commit folds the q and k head norms into it: one command buffer per
    pass against one per command, bit for bit (logits and KV rows), and the
    folded step dispatches no standalone head norm (the profile counts the
    folded norms under their kind with no time). Head sizes 256 and 32 run
    the fold's generic lane layout, 64 its 16-lane one."""
    import ctypes
    from dianoia_amd import _lib
    lib = _lib.load()
    cfg = F.ForwardConfig(hidden=256, intermediate=512, heads=4, kv_heads=2, head_dim=hd,
                          vocab=997, layer_types=[F.FULL, F.FULL], eps=1e-6)
    start = LONG_CONTEXT[hd]
    plan = [(8, p) for p in range(0, start, 8)] + [(1, start), (1, start + 1)]
    fused = F.GpuForward(cfg, max_seq=start + 32, max_chunk=8, seed=5)
    split = F.GpuForward(cfg, max_seq=start + 32, max_chunk=8, seed=5)
    split.split_commits = True
    try:
        a = run(fused, plan[:-1])
        b = run(split, plan[:-1])
        for (la, sa), (lb, sb), chunk in zip(a, b, plan):
            assert same(la, lb), f"logits differ after chunk {chunk}"
            assert all(same(x, y) for x, y in zip(sa, sb)), f"state differs after chunk {chunk}"
        ms = (ctypes.c_double * 21)()
        lib.lab_gpu_profile(ms, (ctypes.c_int64 * 21)(), 21)
        lib.lab_gpu_set_profiling(1)
        la = run(fused, plan[-1:])
        lib.lab_gpu_set_profiling(0)
        counts = (ctypes.c_int64 * 21)()
        lib.lab_gpu_profile(ms, counts, 21)
        lb = run(split, plan[-1:])
        assert same(la[0][0], lb[0][0])
        head_norm_rope, attention = 5, 7
        layers = len(cfg.layer_types)
        # The folded head norms are counted under their own kind (q and k per
        # layer) with no time of their own: no standalone launch.
        assert counts[head_norm_rope] == 2 * layers and ms[head_norm_rope] == 0, list(counts)
        assert counts[attention] == layers and ms[attention] > 0, list(counts)
    finally:
        fused.dispose()
        split.dispose()
