"""ctypes bindings of the CPU oracle. TEST INFRASTRUCTURE ONLY.

Loads ``oracle/liblab_oracle.so`` (the scalar restatement in lab_oracle.c)
and, where it was built, ``oracle/_ref/liblab_native.so`` (the reference's
own ``src/c/lab_native.c``). Only tests/, ``__graft_entry__.smoke()`` and
bench.py's ``cpu_baseline`` leg may import this module: it is the checker
and the CPU baseline, never the product path.

Both libraries export the reference's argument order
(``lab_gemm_q8(qs, scales, xs, xq, xsc, ys, rows, cols, n, threads, mode)``,
``src/c/lab_native.c:553-555``), so one wrapper class serves both.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liblab_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "liblab_native.so")

_i64 = ctypes.c_int64
_p = ctypes.c_void_p


def build(force: bool = False) -> None:
    """Builds liblab_oracle.so (and _ref when the reference is mounted)."""
    if force or not os.path.exists(ORACLE_SO):
        subprocess.run(["make", "-C", HERE, "all"], check=True, capture_output=True)


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "arrays handed to C must be contiguous"
    return ctypes.c_void_p(a.ctypes.data)


class _Kernels:
    """The lab_* product and quantizer entry points of one library."""

    def __init__(self, path: str, prefix: str):
        self.path = path
        self.lib = ctypes.CDLL(path)
        self.prefix = prefix
        for name in ("quantize_q8", "quantize_q4"):
            f = getattr(self.lib, prefix + name)
            f.argtypes = [_p, _p, _p, _i64, _i64]
            f.restype = None
        for name in ("gemm_q8", "gemm_q4"):
            f = getattr(self.lib, prefix + name)
            f.argtypes = [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64]
            f.restype = None

    def quantize_q8(self, x: np.ndarray):
        x = np.ascontiguousarray(x, dtype=np.float32)
        rows, cols = x.shape
        qs = np.zeros((rows, cols), np.int8)
        scales = np.zeros((rows, cols // 32), np.float32)
        getattr(self.lib, self.prefix + "quantize_q8")(_ptr(x), _ptr(qs), _ptr(scales), rows, cols)
        return qs, scales

    def quantize_q4(self, w: np.ndarray):
        w = np.ascontiguousarray(w, dtype=np.float32)
        rows, cols = w.shape
        qs = np.zeros((rows, cols // 2), np.uint8)
        scales = np.zeros((rows, cols // 32), np.uint16)
        getattr(self.lib, self.prefix + "quantize_q4")(_ptr(w), _ptr(qs), _ptr(scales), rows, cols)
        return qs, scales

    def _gemm(self, name, qs, scales, xs, n, threads, mode, rows, cols):
        xs = np.ascontiguousarray(xs, dtype=np.float32).reshape(n, cols)
        xq = np.zeros(n * cols, np.int8)
        xsc = np.zeros(n * cols // 32 + 1, np.float32)
        ys = np.zeros((n, rows), np.float32)
        getattr(self.lib, self.prefix + name)(
            _ptr(qs), _ptr(scales), _ptr(xs), _ptr(xq), _ptr(xsc), _ptr(ys),
            rows, cols, n, threads, mode)
        return ys

    def gemm_q8(self, qs, scales, xs, n=None, threads=1, mode=1):
        qs = np.ascontiguousarray(qs, dtype=np.int8)
        scales = np.ascontiguousarray(scales, dtype=np.float32)
        rows, cols = qs.shape
        n = xs.size // cols if n is None else n
        return self._gemm("gemm_q8", qs, scales, xs, n, threads, mode, rows, cols)

    def gemm_q4(self, qs, scales, xs, n=None, threads=1, mode=1):
        qs = np.ascontiguousarray(qs, dtype=np.uint8)
        scales = np.ascontiguousarray(scales, dtype=np.uint16)
        rows, cols = qs.shape[0], qs.shape[1] * 2
        n = xs.size // cols if n is None else n
        return self._gemm("gemm_q4", qs, scales, xs, n, threads, mode, rows, cols)


class Oracle(_Kernels):
    """The restatement, plus the helpers the reference has no C form of."""

    def __init__(self, path: str = ORACLE_SO):
        build()
        super().__init__(path, "orc_")
        L = self.lib
        L.orc_half_to_float.argtypes = [ctypes.c_uint16]
        L.orc_half_to_float.restype = ctypes.c_float
        L.orc_float_to_half.argtypes = [ctypes.c_float]
        L.orc_float_to_half.restype = ctypes.c_uint16
        for name in ("orc_quantize_q8_bf16", "orc_quantize_q8_padded"):
            getattr(L, name).argtypes = [_p, _p, _p, _i64, _i64, _i64]
            getattr(L, name).restype = None
        for name in ("orc_block_dots_q8", "orc_block_dots_q4"):
            getattr(L, name).argtypes = [_p, _p, _p, _i64, _i64, _i64]
            getattr(L, name).restype = None
        L.orc_dequantize_q6k.argtypes = [_p, _p, _i64]
        L.orc_dequantize_q6k.restype = None
        L.orc_q6k_to_q8.argtypes = [_p, _p, _p, _i64, _i64]
        L.orc_q6k_to_q8.restype = None
        f32 = ctypes.c_float
        L.orc_rms_norm.argtypes = [_p, _p, _p, _i64, _i64, f32, ctypes.c_int]
        L.orc_head_norm_rope.argtypes = [_p, _i64, _p, _p, _i64, _i64, _i64, _i64, f32]
        L.orc_short_conv.argtypes = [_p, _p, _p, _p, _i64, _i64, _i64]
        L.orc_attention.argtypes = [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64]
        L.orc_steer.argtypes = [_p, _p, _i64, _i64, _i64, f32]
        for name in ("orc_rms_norm", "orc_head_norm_rope", "orc_short_conv", "orc_attention",
                     "orc_steer"):
            getattr(L, name).restype = None
        L.orc_argmax.argtypes = [_p, _i64]
        L.orc_argmax.restype = _i64
        L.orc_silu_mul.argtypes = [_p, _p, _i64]
        L.orc_silu_mul.restype = None
        L.orc_gelu.argtypes = [_p, _i64]
        L.orc_gelu.restype = None

    def half_to_float(self, h: int) -> float:
        return self.lib.orc_half_to_float(h)

    def float_to_half(self, f: float) -> int:
        return self.lib.orc_float_to_half(f)

    def quantize_q8_padded(self, x: np.ndarray, cols_pad: int):
        x = np.ascontiguousarray(x, dtype=np.float32)
        rows, cols = x.shape
        qs = np.zeros((rows, cols_pad), np.int8)
        scales = np.zeros((rows, cols_pad // 32), np.float32)
        self.lib.orc_quantize_q8_padded(_ptr(x), _ptr(qs), _ptr(scales), rows, cols, cols_pad)
        return qs, scales

    def quantize_q8_bf16(self, w: np.ndarray, cols_pad: int | None = None):
        w = np.ascontiguousarray(w, dtype=np.uint16)
        rows, cols = w.shape
        cols_pad = (cols + 31) // 32 * 32 if cols_pad is None else cols_pad
        qs = np.zeros((rows, cols_pad), np.int8)
        scales = np.zeros((rows, cols_pad // 32), np.float32)
        self.lib.orc_quantize_q8_bf16(_ptr(w), _ptr(qs), _ptr(scales), rows, cols, cols_pad)
        return qs, scales

    def dequantize_q6k(self, blocks: np.ndarray) -> np.ndarray:
        """Q6_K super-blocks (210 B each) -> float32 values (256 each)."""
        blocks = np.ascontiguousarray(blocks, np.uint8).reshape(-1)
        count = blocks.size // 210
        out = np.zeros(count * 256, np.float32)
        self.lib.orc_dequantize_q6k(_ptr(blocks), _ptr(out), count)
        return out

    def q6k_to_q8(self, blocks: np.ndarray, rows: int, cols: int):
        """The Q6_K -> Q8 adapter: dequantize, then lab_quantize_q8."""
        blocks = np.ascontiguousarray(blocks, np.uint8).reshape(-1)
        assert cols % 256 == 0 and blocks.size == rows * cols // 256 * 210
        qs = np.zeros((rows, cols), np.int8)
        scales = np.zeros((rows, cols // 32), np.float32)
        self.lib.orc_q6k_to_q8(_ptr(blocks), _ptr(qs), _ptr(scales), rows, cols)
        return qs, scales

    # ---- layer steps (Metal shader semantics, sums in double). Every array
    # handed to C is bound to a name first, so it outlives the call.

    def split_q8_0(self, blocks: np.ndarray, count: int):
        """GGUF Q8_0 blocks -> (int8 values [count * 32], fp32 scales [count]):
        splitQ8_0, lib/src/gguf.dart:270-282. Block b is 34 bytes: the fp16 d
        (little-endian) at 34b, the values at 34b + 2. d is widened as
        halfToDouble (lib/src/native.dart:871-880) then stored as a float:
        sign * mantissa * 2^-24 (subnormal), +-inf, double.nan (0x7FC00000
        for every NaN pattern), else sign * (1 + m / 1024) * 2^(e - 15)."""
        b = np.asarray(blocks, dtype=np.uint8).reshape(count, 34)
        bits = b[:, 0].astype(np.int64) | (b[:, 1].astype(np.int64) << 8)
        sign = np.where(bits & 0x8000, -1.0, 1.0)
        e, m = (bits >> 10) & 0x1F, bits & 0x3FF
        with np.errstate(invalid="ignore"):
            d = np.where(e == 0, sign * m * 2.0 ** -24,
                         np.where(e == 31, np.where(m == 0, sign * np.inf, np.nan),
                                  sign * (1 + m / 1024) * np.exp2(e - 15.0)))
        scales = d.astype(np.float32)
        scales[np.isnan(scales)] = np.uint32(0x7FC00000).view(np.float32)
        return b[:, 2:].copy().view(np.int8).reshape(-1), scales

    def split_q4_0(self, blocks: np.ndarray, count: int):
        """GGUF Q4_0 blocks -> (nibble bytes [count * 16], fp16 bits [count]):
        splitQ4_0, lib/src/gguf.dart:208-218 (bytes copied as they are)."""
        b = np.asarray(blocks, dtype=np.uint8).reshape(count, 18)
        d = (b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8))
        return b[:, 2:].copy().reshape(-1), d

    def rms_norm(self, x, w, eps, out=None):
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        rows, cols = x.shape
        acc = out is not None
        y = np.array(out, np.float32, order="C") if acc else np.zeros_like(x)
        self.lib.orc_rms_norm(_ptr(x), _ptr(w), _ptr(y), rows, cols, eps, 1 if acc else 0)
        return y

    def head_norm_rope(self, x, x_stride, w, rope, rope_stride, heads, hd, n, eps):
        x = np.array(x, np.float32, order="C")
        w = np.ascontiguousarray(w, np.float32)
        rope = np.ascontiguousarray(rope, np.float32)
        self.lib.orc_head_norm_rope(_ptr(x), x_stride, _ptr(w), _ptr(rope), rope_stride, heads,
                                    hd, n, eps)
        return x

    def short_conv(self, bcx, weight, history, width, k, n):
        bcx = np.ascontiguousarray(bcx, np.float32)
        weight = np.ascontiguousarray(weight, np.float32)
        history = np.array(history, np.float32, order="C")
        y = np.zeros(n * width, np.float32)
        self.lib.orc_short_conv(_ptr(bcx), _ptr(weight), _ptr(history), _ptr(y), width, k, n)
        return y, history

    def attention(self, q, keys, values, gate, position, n, heads, kv_heads, hd, window=0):
        q = np.ascontiguousarray(q, np.float32)
        keys = np.ascontiguousarray(keys, np.float32)
        values = np.ascontiguousarray(values, np.float32)
        g = None if gate is None else np.ascontiguousarray(gate, np.float32)
        out = np.zeros(n * heads * hd, np.float32)
        self.lib.orc_attention(_ptr(q), _ptr(keys), _ptr(values), None if g is None else _ptr(g),
                               _ptr(out), position, n, heads, kv_heads, hd, window)
        return out

    def steer(self, x, v, mode, scale):
        x = np.array(x, np.float32, order="C")
        v = np.ascontiguousarray(v, np.float32)
        rows, cols = x.shape
        self.lib.orc_steer(_ptr(x), _ptr(v), rows, cols, mode, scale)
        return x

    def block_dots_q8(self, qs, xq):
        qs = np.ascontiguousarray(qs, np.int8)
        rows, cols = qs.shape
        xq = np.ascontiguousarray(xq, np.int8).reshape(-1, cols)
        d = np.zeros((xq.shape[0], rows, cols // 32), np.int32)
        self.lib.orc_block_dots_q8(_ptr(qs), _ptr(xq), _ptr(d), rows, cols, xq.shape[0])
        return d

    def block_dots_q4(self, qs, xq):
        qs = np.ascontiguousarray(qs, np.uint8)
        rows, cols = qs.shape[0], qs.shape[1] * 2
        xq = np.ascontiguousarray(xq, np.int8).reshape(-1, cols)
        d = np.zeros((xq.shape[0], rows, cols // 32), np.int32)
        self.lib.orc_block_dots_q4(_ptr(qs), _ptr(xq), _ptr(d), rows, cols, xq.shape[0])
        return d

    def argmax(self, logits: np.ndarray) -> int:
        logits = np.ascontiguousarray(logits, np.float32)
        return int(self.lib.orc_argmax(_ptr(logits), logits.size))

    def silu_mul(self, g: np.ndarray, u: np.ndarray) -> np.ndarray:
        out = np.array(g, dtype=np.float32, copy=True)
        u = np.ascontiguousarray(u, np.float32)
        self.lib.orc_silu_mul(_ptr(out), _ptr(u), out.size)
        return out

    def gelu(self, x: np.ndarray) -> np.ndarray:
        out = np.array(x, dtype=np.float32, copy=True)
        self.lib.orc_gelu(_ptr(out), out.size)
        return out


class Reference(_Kernels):
    """The reference's lab_native.c, compiled in oracle/_ref by oracle/Makefile."""

    def __init__(self, path: str = REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        super().__init__(path, "lab_")


def reference_available() -> bool:
    return os.path.exists(REF_SO)


_oracle: Oracle | None = None


def get() -> Oracle:
    global _oracle
    if _oracle is None:
        _oracle = Oracle()
    return _oracle
