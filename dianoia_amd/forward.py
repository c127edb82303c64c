"""Host-side mirror of the reference's GpuForward (lib/src/gpu.dart:700-1262)
over the lab_gpu_* C ABI: a decode / prefill pass of the LFM3 or Qwen3
decoder encoded command for command as ``GpuForward.forward`` encodes it
(gpu.dart:1036-1239), on random weights of a chosen shape.

It is a driver for the tests and the bench, which measure the drop-in
boundary under a real decoder's command stream: the per-token PCIe traffic
of the staged host views, the fusions ``lab_gpu_commit`` applies, and that
host writes between command buffers (a new token's embedding, a restored
conv history or KV rows, gpu.dart:1003-1021) reach the GPU.

Layout as in the reference:
  * every matrix in its own wrapped buffer (``lab_gpu_wrap``), Q4 body and
    a Q8 LM head (the reference's q4Body cache, gpu.dart:902-907);
  * the small float tensors (norm weights, conv kernels, q/k norms) packed
    into one buffer at 16-byte aligned offsets (gpu.dart:836-899);
  * activations of ``max_chunk`` rows, per-layer conv histories of
    (k - 1) x hidden floats, per-layer key and value caches of
    ``max_seq`` x kv_dim floats (gpu.dart:871-887, 909-928);
  * per token a RoPE row [full cos, full sin, sliding cos, sliding sin] of
    hd / 2 floats each (gpu.dart:1052-1062).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from .errors import ArgumentError, StateError

CONV, FULL, SLIDING = "conv", "full_attention", "sliding_attention"


@dataclass
class ForwardConfig:
    """The subset of TextModelConfig (lib/src/config.dart:28-250) the pass uses."""

    hidden: int
    intermediate: int
    heads: int
    kv_heads: int
    head_dim: int
    vocab: int
    layer_types: list = field(default_factory=list)
    conv_kernel: int = 3
    sliding_window: int = 0
    eps: float = 1e-5
    sandwich: bool = False
    gate: bool = False
    full_theta: float = 1e6
    sliding_theta: float = 1e4

    @property
    def kv_dim(self) -> int:
        return self.kv_heads * self.head_dim

    @property
    def layers(self) -> int:
        return len(self.layer_types)


def qwen3_1_7b() -> ForwardConfig:
    """Qwen3-1.7B's decoder (the shapes of configs 1 and 2): 28 full-attention
    layers, hidden 2048, SwiGLU 6144, 16 query / 8 KV heads of 128, vocabulary
    151936; QK-norm, no output gate, no sandwich norms (config.dart:190-235)."""
    return ForwardConfig(hidden=2048, intermediate=6144, heads=16, kv_heads=8, head_dim=128,
                         vocab=151936, layer_types=[FULL] * 28, eps=1e-6, full_theta=1e6,
                         sliding_theta=1e6)


def lfm3_small() -> ForwardConfig:
    """A small LFM3-shaped decoder exercising every layer step: gated short
    convolutions, full and sliding attention with the per-head output gate,
    sandwich norms (config.dart:140-188)."""
    return ForwardConfig(hidden=256, intermediate=768, heads=4, kv_heads=2, head_dim=64,
                         vocab=1000, layer_types=[CONV, FULL, CONV, SLIDING, CONV],
                         conv_kernel=3, sliding_window=3, eps=1e-5, sandwich=True, gate=True)


def _rope_row(theta: float, hd: int, position: int) -> tuple[np.ndarray, np.ndarray]:
    """cos and sin of the hd / 2 rotation angles of one position."""
    pair = hd // 2
    inv = theta ** (-np.arange(pair, dtype=np.float64) * 2.0 / hd)
    ang = position * inv
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


class _Buffer:
    """A lab_gpu_buffer of float32 values and its host view (gpu.dart _Buffer)."""

    def __init__(self, lib, floats: int):
        self.lib = lib
        self.floats = max(1, floats)
        self.handle = int(lib.lab_gpu_buffer(self.floats * 4))
        if self.handle < 0:
            raise StateError(f"GPU buffer of {self.floats * 4} bytes failed")

    @property
    def view(self) -> np.ndarray:
        ptr = self.lib.lab_gpu_contents(self.handle)
        if not ptr:
            raise StateError("lab_gpu_contents returned NULL")
        raw = (ctypes.c_float * self.floats).from_address(ptr)
        return np.frombuffer(raw, dtype=np.float32, count=self.floats)


@dataclass
class _Matrix:
    q4: bool
    buffer: int
    qs: int
    scales: int
    rows: int
    cols: int
    host: np.ndarray  # the wrapped bytes (kept for oracle checks)

    def qs_scales(self):
        """The matrix in the engine layout: (qs, scales) as the CPU kernels take them."""
        if self.q4:
            qs = self.host[self.qs:self.qs + self.rows * self.cols // 2].reshape(self.rows, -1)
            sc = self.host[self.scales:self.scales + self.rows * (self.cols // 32) * 2].view(np.uint16)
            return qs, sc.reshape(self.rows, -1)
        qs = self.host[self.qs:self.qs + self.rows * self.cols].view(np.int8).reshape(self.rows, -1)
        sc = self.host[self.scales:self.scales + self.rows * (self.cols // 32) * 4].view(np.float32)
        return qs, sc.reshape(self.rows, -1)


@dataclass
class _Layer:
    kind: str
    operator_norm: int
    post_operator_norm: int | None
    ffn_norm: int
    post_ffn_norm: int | None
    w1: _Matrix
    w3: _Matrix
    w2: _Matrix
    in_proj: _Matrix | None = None
    out_proj: _Matrix | None = None
    conv_kernel: int = -1
    history: _Buffer | None = None
    q: _Matrix | None = None
    k: _Matrix | None = None
    v: _Matrix | None = None
    gate: _Matrix | None = None
    o: _Matrix | None = None
    q_norm: int = -1
    k_norm: int = -1
    keys: _Buffer | None = None
    values: _Buffer | None = None


class GpuForward:
    """GpuForward (gpu.dart:700-1262) on random weights of ``config``.

    ``split_commits``: each recorded command runs in a command buffer of its
    own (committed and waited at once), so no fusion applies and every
    command's inputs and outputs pass through the host views; ``checker``
    (with split commits) is called as checker(kind, args, self) before each
    command's commit and returns a callable run after it.
    """

    def __init__(self, config: ForwardConfig, max_seq: int, max_chunk: int, seed: int = 0,
                 head_q8: bool = True):
        lib = _lib.load()
        if lib.lab_gpu_init() != 1:
            raise StateError("no GPU")
        self.lib = lib
        self.config = config
        self.max_seq = max_seq
        self.max_chunk = max_chunk
        self.split_commits = False
        self.checker = None
        self._owned: list[int] = []
        self._buffers: list[_Buffer] = []
        self._disposed = False
        rng = np.random.default_rng(seed)
        c = config
        h, hd = c.hidden, c.head_dim

        small: list[np.ndarray] = []
        at = [0]

        def place(values: np.ndarray) -> int:
            offset = at[0] * 4
            small.append(values.astype(np.float32))
            at[0] += (len(values) + 3) // 4 * 4
            return offset

        def norm_weight(n: int) -> np.ndarray:
            return rng.uniform(0.8, 1.2, n).astype(np.float32)

        self._layers: list[_Layer] = []
        for kind in c.layer_types:
            layer = _Layer(
                kind=kind,
                operator_norm=place(norm_weight(h)),
                post_operator_norm=place(norm_weight(h)) if c.sandwich else None,
                ffn_norm=place(norm_weight(h)),
                post_ffn_norm=place(norm_weight(h)) if c.sandwich else None,
                w1=self._matrix(rng, c.intermediate, h),
                w3=self._matrix(rng, c.intermediate, h),
                w2=self._matrix(rng, h, c.intermediate),
            )
            if kind == CONV:
                layer.in_proj = self._matrix(rng, 3 * h, h)
                layer.out_proj = self._matrix(rng, h, h)
                layer.conv_kernel = place(rng.uniform(-0.6, 0.6, h * c.conv_kernel))
                layer.history = self._new((c.conv_kernel - 1) * h)
            else:
                layer.q = self._matrix(rng, c.heads * hd, h)
                layer.k = self._matrix(rng, c.kv_dim, h)
                layer.v = self._matrix(rng, c.kv_dim, h)
                layer.gate = self._matrix(rng, c.heads, h) if c.gate else None
                layer.o = self._matrix(rng, h, c.heads * hd)
                layer.q_norm = place(norm_weight(hd))
                layer.k_norm = place(norm_weight(hd))
                layer.keys = self._new(max_seq * c.kv_dim)
                layer.values = self._new(max_seq * c.kv_dim)
            self._layers.append(layer)
        self._final_norm = place(norm_weight(h))
        self._small = self._new(at[0])
        view = self._small.view
        pos = 0
        for values in small:
            view[pos:pos + len(values)] = values
            pos += (len(values) + 3) // 4 * 4
        self._lm_head = self._matrix(rng, c.vocab, h, q4=not head_q8)

        rows = max_chunk
        heads = c.heads * hd
        self._x = self._new(rows * h)
        self._a = self._new(rows * h)
        self._m = self._new(rows * h)
        self._bcx = self._new(rows * 3 * h)
        self._y = self._new(rows * h)
        self._q = self._new(rows * heads)
        self._gate = self._new(rows * c.heads)
        self._attn_out = self._new(rows * heads)
        self._g = self._new(rows * c.intermediate)
        self._u = self._new(rows * c.intermediate)
        self._normed = self._new(h)
        self._logits = self._new(c.vocab)
        self._rope = self._new(rows * 2 * hd)
        self._capture = self._new((c.layers + 1) * rows * h)
        self.logits = np.zeros(c.vocab, np.float32)

    # ------------------------------------------------------------ weights

    def _new(self, floats: int) -> _Buffer:
        b = _Buffer(self.lib, floats)
        self._buffers.append(b)
        return b

    def _matrix(self, rng, rows: int, cols: int, q4: bool = True) -> _Matrix:
        """A random Q4 (nibbles 0..15, fp16 scales |N(0,1)| * 0.02) or Q8
        (int8 in [-127, 127], fp32 scales |N(0,1)| * 0.01) matrix, wrapped."""
        blocks = cols // 32
        if q4:
            qs = np.frombuffer(rng.bytes(rows * cols // 2), np.uint8)
            sc = (np.abs(rng.standard_normal(rows * blocks, np.float32)) * 0.02).astype(np.float16)
        else:
            # Uniform bytes with -128 moved to -127 (Q8 values lie in [-127, 127]).
            qs = np.frombuffer(rng.bytes(rows * cols), np.uint8).copy()
            qs[qs == 0x80] = 0x81
            sc = np.abs(rng.standard_normal(rows * blocks, np.float32)) * np.float32(0.01)
        sc = sc.view(np.uint8)
        scales_at = (len(qs) + 63) // 64 * 64
        host = np.zeros(scales_at + len(sc), np.uint8)
        host[:len(qs)] = qs
        host[scales_at:] = sc
        handle = int(self.lib.lab_gpu_wrap(host.ctypes.data, host.nbytes))
        if handle < 0:
            raise StateError("wrapping a weight matrix failed")
        self._owned.append(handle)
        return _Matrix(q4, handle, 0, scales_at, rows, cols, host)

    # ------------------------------------------------------------ views

    @property
    def residual(self) -> np.ndarray:
        """The residual stream entering the next forward: write embeddings here."""
        return self._x.view

    def history(self, i: int) -> np.ndarray:
        c = self.config
        return self._layers[i].history.view[:(c.conv_kernel - 1) * c.hidden]

    def state_blocks(self, position: int) -> list[np.ndarray]:
        """GpuForward.stateBlocks (gpu.dart:1003-1017): conv histories, then
        each attention layer's key and value rows before ``position``."""
        rows = position * self.config.kv_dim
        out = [self.history(i) for i, l in enumerate(self._layers) if l.kind == CONV]
        for l in self._layers:
            if l.kind != CONV:
                out += [l.keys.view[:rows], l.values.view[:rows]]
        return out

    def reset(self) -> None:
        """gpu.dart:980-990: conv histories cleared for a new sequence."""
        for i, l in enumerate(self._layers):
            if l.kind == CONV:
                self.history(i)[:] = 0.0

    def captured(self, slot: int, n: int) -> np.ndarray:
        rows = self.max_chunk * self.config.hidden
        return self._capture.view[slot * rows: slot * rows + n * self.config.hidden]

    # ------------------------------------------------------------ the pass

    def _run(self, kind: str, fn, *args) -> None:
        """Records one command; with split commits, runs it alone."""
        if not self.split_commits:
            fn(*args)
            return
        after = self.checker(kind, args, self) if self.checker else None
        self.lib.lab_gpu_begin()
        fn(*args)
        if self.lib.lab_gpu_commit(1) != 1:
            raise StateError(f"GPU command buffer failed ({kind})")
        if after is not None:
            after()

    def forward(self, n: int, position: int, with_logits: bool = True,
                capture: bool = False, meanwhile=None) -> None:
        """GpuForward.forward (gpu.dart:1036-1239): n tokens at positions
        position.. whose embeddings are in ``residual``.

        With ``meanwhile`` the command buffer is committed without waiting
        (lab_gpu_commit(0)), ``meanwhile`` runs on the host while the GPU
        computes, and the pass then waits (lab_gpu_wait), also when
        ``meanwhile`` raises, whose error then propagates
        (gpu.dart:1223-1233). It must not use the GPU or the buffers of the
        pass."""
        if self._disposed:
            raise StateError("the GPU forward pass is disposed")
        if n < 1 or n > self.max_chunk:
            raise ArgumentError(f"chunk of {n} tokens")
        if position + n > self.max_seq:
            raise StateError("position exceeds maxSeq")
        lib, c = self.lib, self.config
        h, hd, eps = c.hidden, c.head_dim, c.eps
        pair = hd // 2
        rope = self._rope.view
        for t in range(n):
            fc, fs = _rope_row(c.full_theta, hd, position + t)
            sc, ss = _rope_row(c.sliding_theta, hd, position + t)
            at = t * 4 * pair
            rope[at:at + pair] = fc
            rope[at + pair:at + 2 * pair] = fs
            rope[at + 2 * pair:at + 3 * pair] = sc
            rope[at + 3 * pair:at + 4 * pair] = ss

        def matmul(w: _Matrix, x: _Buffer, y: int, y_offset: int = 0) -> None:
            f = lib.lab_gpu_enc_matmul_q4 if w.q4 else lib.lab_gpu_enc_matmul_q8
            self._run("matmul", f, w.buffer, w.qs, w.scales, x.handle, 0, y, y_offset, w.rows,
                      w.cols, n)

        def norm(x: _Buffer, w: int, out: _Buffer, accumulate: bool = False) -> None:
            self._run("rms_norm", lib.lab_gpu_enc_rms_norm, x.handle, 0, self._small.handle, w,
                      out.handle, 0, n, h, eps, 1 if accumulate else 0)

        def residual(w: int | None) -> None:
            if w is not None:
                norm(self._m, w, self._x, accumulate=True)
            else:
                self._run("add", lib.lab_gpu_enc_add, self._m.handle, 0, self._x.handle, 0, n * h)

        def snapshot(slot: int) -> None:
            self._run("copy", lib.lab_gpu_enc_copy, self._x.handle, 0, self._capture.handle,
                      slot * self.max_chunk * h * 4, n * h)

        def head_norm_rope(x: int, x_offset: int, x_stride: int, w: int, heads: int,
                           rope_offset: int) -> None:
            self._run("head_norm_rope", lib.lab_gpu_enc_head_norm_rope, x, x_offset, x_stride,
                      self._small.handle, w, self._rope.handle, rope_offset, 4 * pair, heads, hd,
                      n, eps)

        if not self.split_commits:
            lib.lab_gpu_begin()
        if capture:
            snapshot(0)
        for i, l in enumerate(self._layers):
            norm(self._x, l.operator_norm, self._a)
            if l.kind == CONV:
                matmul(l.in_proj, self._a, self._bcx.handle)
                self._run("conv", lib.lab_gpu_enc_conv, self._bcx.handle, self._small.handle,
                          l.conv_kernel, l.history.handle, self._y.handle, h, c.conv_kernel, n)
                matmul(l.out_proj, self._y, self._m.handle)
            else:
                rows = position * c.kv_dim * 4
                rope_offset = (2 * pair if l.kind == SLIDING else 0) * 4
                matmul(l.q, self._a, self._q.handle)
                matmul(l.k, self._a, l.keys.handle, rows)
                matmul(l.v, self._a, l.values.handle, rows)
                if l.gate is not None:
                    matmul(l.gate, self._a, self._gate.handle)
                head_norm_rope(self._q.handle, 0, c.heads * hd, l.q_norm, c.heads, rope_offset)
                head_norm_rope(l.keys.handle, rows, c.kv_dim, l.k_norm, c.kv_heads, rope_offset)
                self._run("attention", lib.lab_gpu_enc_attention, self._q.handle, l.keys.handle,
                          l.values.handle, -1 if l.gate is None else self._gate.handle,
                          self._attn_out.handle, position, n, c.heads, c.kv_heads, hd,
                          c.sliding_window if l.kind == SLIDING else 0)
                matmul(l.o, self._attn_out, self._m.handle)
            residual(l.post_operator_norm)
            norm(self._x, l.ffn_norm, self._a)
            matmul(l.w1, self._a, self._g.handle)
            matmul(l.w3, self._a, self._u.handle)
            self._run("swiglu", lib.lab_gpu_enc_swiglu, self._g.handle, self._u.handle,
                      n * c.intermediate)
            matmul(l.w2, self._g, self._m.handle)
            residual(l.post_ffn_norm)
            if capture:
                snapshot(i + 1)
        if with_logits:
            self._run("rms_norm", lib.lab_gpu_enc_rms_norm, self._x.handle, (n - 1) * h * 4,
                      self._small.handle, self._final_norm, self._normed.handle, 0, 1, h, eps, 0)
            w = self._lm_head
            f = lib.lab_gpu_enc_matmul_q4 if w.q4 else lib.lab_gpu_enc_matmul_q8
            self._run("matmul", f, w.buffer, w.qs, w.scales, self._normed.handle, 0,
                      self._logits.handle, 0, w.rows, w.cols, 1)
        if self.split_commits:
            if meanwhile is not None:
                meanwhile()
        elif meanwhile is None:
            if lib.lab_gpu_commit(1) != 1:
                raise StateError("GPU command buffer failed")
        else:
            if lib.lab_gpu_commit(0) != 1:
                raise StateError("GPU command buffer failed")
            try:
                meanwhile()
            finally:
                if lib.lab_gpu_wait() != 1:
                    raise StateError("GPU command buffer failed")
        if with_logits:
            self.logits[:] = self._logits.view

    def last_ms(self) -> float:
        return float(self.lib.lab_gpu_last_ms())

    def dispose(self) -> None:
        if self._disposed:
            return
        self._disposed = True
        for b in self._buffers:
            self.lib.lab_gpu_release(b.handle)
        for hnd in self._owned:
            self.lib.lab_gpu_release(hnd)
        self._buffers.clear()
        self._owned.clear()


def transfer_bytes() -> tuple[int, int]:
    """Bytes copied host -> HBM and HBM -> host by the library so far."""
    lib = _lib.load()
    up, down = ctypes.c_int64(), ctypes.c_int64()
    lib.lab_gpu_transfer_bytes(ctypes.byref(up), ctypes.byref(down))
    return up.value, down.value


def tracking_writes() -> bool:
    return bool(_lib.load().lab_gpu_tracking_writes())
