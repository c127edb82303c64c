"""Host-side mirror of the reference's GpuLinear, over the lab_gpu_* C ABI.

``GpuLinear`` follows ``lib/src/gpu.dart:1279-1368`` of the reference: the
same methods (start / upload / apply / dispose / names), argument meaning and
errors (``ArgumentError`` for unknown names and short lists, ``StateError``
after dispose or when a command buffer fails). Each call goes through the
C ABI exactly as Dart's ``@Native`` bindings would, so these tests exercise
the drop-in boundary itself.

Beyond the reference's class it offers the rest of this tier's path on the
same buffers: GPU load-time quantization of BF16 weights (``upload_bf16``),
the greedy LM-head token (``apply_argmax``), the MLP pair with its SiLU
glue (``mlp``) and the vision projector pair with its GELU (``gelu_pair``).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from .errors import ArgumentError, StateError
from .formats import QuantMatrix
from .q8_cache import Q8Cache


class _Buffer:
    """A lab_gpu_buffer of float32 values and its host view (gpu.dart _Buffer)."""

    def __init__(self, lib, floats: int):
        self.lib = lib
        nbytes = max(4, floats * 4)
        self.handle = lib.lab_gpu_buffer(nbytes)
        if self.handle < 0:
            raise StateError(f"GPU buffer of {nbytes} bytes failed")
        self.length = floats
        self.nbytes = nbytes

    def view(self, dtype=np.float32, count: int | None = None, offset: int = 0) -> np.ndarray:
        ptr = self.lib.lab_gpu_contents(self.handle)
        if not ptr:
            raise StateError("lab_gpu_contents returned NULL")
        itemsize = np.dtype(dtype).itemsize
        count = (self.nbytes - offset) // itemsize if count is None else count
        raw = (ctypes.c_char * (offset + count * itemsize)).from_address(ptr)
        return np.frombuffer(raw, dtype=dtype, count=count, offset=offset)


@dataclass
class _Matrix:
    """A Q8 or Q4 matrix: its buffer and byte offsets (gpu.dart:326-353)."""

    q4: bool
    buffer: int
    qs: int
    scales: int
    rows: int
    cols: int
    in_cols: int  # columns the caller's inputs have (cols may be padded)
    owns: bool = True  # False: a segment of a wrapped cache, shared and kept

    def encode(self, lib, x: int, y: int, y_offset: int, n: int, x_offset: int = 0) -> None:
        f = lib.lab_gpu_enc_matmul_q4 if self.q4 else lib.lab_gpu_enc_matmul_q8
        f(self.buffer, self.qs, self.scales, x, x_offset, y, y_offset, self.rows, self.cols, n)


def set_int8_inputs(on: bool) -> bool:
    """Input mode of the matmuls recorded from now on (process-wide); returns
    the previous one. True: x quantized per block (lab_gemm_* mode 1, the
    Vulkan layer's path); False: float inputs (mode 0, the Metal layer's)."""
    lib = _lib.load()
    return bool(lib.lab_gpu_set_int8_inputs(1 if on else 0))


def live_buffers() -> int:
    """GpuForward.liveBuffers (gpu.dart): buffers not yet released."""
    return int(_lib.load().lab_gpu_live_buffers())


class GpuLinear:
    """Products of quantized matrices on the GPU (gpu.dart:1270-1368)."""

    def __init__(self, lib):
        self._lib = lib
        self._matrices: dict[str, _Matrix] = {}
        self._owned: list[int] = []
        self._x: _Buffer | None = None
        self._y: _Buffer | None = None
        self._aux: dict[str, _Buffer] = {}
        self._disposed = False
        self.segments = 0  # buffers made by wrap_cache

    @staticmethod
    def start() -> "GpuLinear | None":
        """Starts the GPU, or returns None where it does not start."""
        lib = _lib.load()
        return GpuLinear(lib) if lib.lab_gpu_init() == 1 else None

    @property
    def names(self):
        return self._matrices.keys()

    # ------------------------------------------------------------ upload

    def upload(self, name: str, matrix: QuantMatrix) -> None:
        """Copies ``matrix`` (Q4 or Q8) into a GPU buffer of its own."""
        self._check_open()
        if matrix.format not in ("q4", "q8"):
            raise ArgumentError(f"cannot multiply {matrix.format} matrices")
        qs, scales = matrix.qs_bytes, matrix.scale_bytes
        scales_at = (len(qs) + 63) // 64 * 64
        nbytes = scales_at + len(scales)
        handle = self._lib.lab_gpu_buffer(nbytes)
        if handle < 0:
            raise StateError(f"GPU buffer of {nbytes} bytes failed")
        self._owned.append(handle)
        view = self._bytes_view(handle, nbytes)
        view[: len(qs)] = qs
        view[scales_at: scales_at + len(scales)] = scales
        self._replace(name, _Matrix(matrix.format == "q4", handle, 0, scales_at, matrix.rows,
                                    matrix.cols, matrix.cols))

    def wrap_cache(self, cache: Q8Cache, limit: int | None = None) -> dict[str, tuple[int, int]]:
        """Places an open weight cache in HBM and registers its matrices
        under their names (gpu.dart:938-979, ``_wrapWeights``).

        One ``lab_gpu_wrap`` per segment: matrices in file order, a segment
        starting at the 16 KiB page holding its first matrix's values and
        taking whole matrices while it stays within ``limit`` bytes
        (``lab_gpu_max_buffer_length()`` unless given). Returns each
        matrix's buffer handle and that buffer's file offset. Raises
        ``StateError`` when one matrix alone exceeds the limit or a wrap
        fails."""
        self._check_open()
        page = 16384
        if limit is None:
            limit = int(self._lib.lab_gpu_max_buffer_length())
        matrices = sorted(((name, cache.offsets(name, r, c), r, c) for name, r, c in cache.shapes),
                          key=lambda t: t[1]["qs"])
        result: dict[str, tuple[int, int]] = {}
        pending: list = []
        start = end = 0
        for i in range(len(matrices) + 1):
            item = matrices[i] if i < len(matrices) else None
            if pending and (item is None or item[1]["end"] - start > limit):
                nbytes = min(end, cache.file.length) - start
                h = int(self._lib.lab_gpu_wrap(cache.file.address + start, nbytes))
                if h < 0:
                    raise StateError("wrapping the weight cache failed")
                self._owned.append(h)
                self.segments += 1
                for name, o, r, c in pending:
                    result[name] = (h, start)
                    self._replace(name, _Matrix(o["format"] == "q4", h, o["qs"] - start,
                                                o["scales"] - start, r, c, c, owns=False))
                pending = []
            if item is None:
                break
            name, o = item[0], item[1]
            if not pending:
                start = o["qs"] // page * page
            if o["end"] - start > limit:
                raise StateError(f"{name} alone exceeds the largest GPU buffer")
            pending.append(item)
            end = o["end"]
        return result

    def upload_bf16(self, name: str, bf16: np.ndarray, rows: int, cols: int,
                    rows_pad: int | None = None, fmt: str = "q8") -> None:
        """Quantizes BF16 weights to Q8 (or Q4) on the GPU (part 4 of the path).

        The reference widens BF16 with ``p << 16`` and quantizes on the CPU
        (``vision_encoder.dart:36-66``, ``safetensors.dart:207-212``,
        ``lab_quantize_q8`` / ``lab_quantize_q4``); this does both in one
        kernel, bit-exactly. For Q8 a width that is not a multiple of 32 is
        zero-padded to the next one (the reference refuses it,
        ``native.dart:634-636``); Q4 refuses it as the reference does
        (``native.dart:793-796``). ``rows_pad`` appends zero rows, whose
        outputs are exactly 0.
        """
        bf16 = np.ascontiguousarray(bf16, dtype=np.uint16).reshape(-1)
        self._upload_quantized(name, bf16, 2, rows, cols, rows_pad, fmt)

    def upload_f32(self, name: str, w: np.ndarray, rows: int, cols: int,
                   rows_pad: int | None = None, fmt: str = "q8") -> None:
        """Quantizes fp32 weights to Q8 or Q4 on the GPU, bit-exact with
        ``NativeQ8Matrix.quantize`` / ``NativeQ4Matrix.quantize``
        (``native.dart:633-641``, ``:793-801``); padding as ``upload_bf16``."""
        w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
        self._upload_quantized(name, w, 4, rows, cols, rows_pad, fmt)

    def upload_q6k(self, name: str, blocks: np.ndarray, rows: int, cols: int) -> None:
        """Converts Q6_K super-blocks (GGUF ``token_embd.weight``) to the engine's
        Q8 on the GPU: ``importGguf``'s tied embedding / LM head
        (``gguf.dart:402-414``: ``dequantizeQ6K`` then
        ``NativeQ8Matrix.quantizeRows``), bit-exact."""
        self._check_open()
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
        if rows <= 0 or cols <= 0 or cols % 256 != 0:
            raise ArgumentError(f"Q6_K needs cols to be a multiple of 256, got {cols}")
        nsrc = rows * (cols // 256) * 210
        if blocks.size < nsrc:
            raise ArgumentError(f"{blocks.size} bytes hold fewer than {rows} x {cols} Q6_K values")
        src = self._lib.lab_gpu_buffer(nsrc)
        if src < 0:
            raise StateError("GPU buffer for the Q6_K blocks failed")
        try:
            self._bytes_view(src, nsrc)[:] = blocks[:nsrc]
            scales_at = (rows * cols + 63) // 64 * 64
            nbytes = scales_at + rows * (cols // 32) * 4
            dst = self._lib.lab_gpu_buffer(nbytes)
            if dst < 0:
                raise StateError(f"GPU buffer of {nbytes} bytes failed")
            self._owned.append(dst)
            self._lib.lab_gpu_begin()
            self._lib.lab_gpu_enc_q6k_to_q8(src, 0, dst, 0, dst, scales_at, rows, cols)
            if self._lib.lab_gpu_commit(1) != 1:
                raise StateError("GPU command buffer failed")
        finally:
            self._lib.lab_gpu_release(src)
        self._replace(name, _Matrix(False, dst, 0, scales_at, rows, cols, cols))

    def upload_gguf(self, name: str, blocks: np.ndarray, rows: int, cols: int,
                    kind: str = "q8_0") -> None:
        """Uploads GGUF Q8_0 or Q4_0 blocks as they lie in the file and splits
        them into the engine's Q8 / Q4 layout on the GPU (the reference splits
        on the CPU first: ``splitQ8_0`` ``gguf.dart:270-282``, ``splitQ4_0``
        ``:208-218``); the matrix is the same, bit for bit."""
        self._check_open()
        if kind not in ("q8_0", "q4_0"):
            raise ArgumentError(f"cannot split GGUF {kind} blocks")
        q4 = kind == "q4_0"
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
        count = rows * cols // 32
        nsrc = count * (18 if q4 else 34)
        if rows <= 0 or cols <= 0 or cols % 32 != 0 or blocks.size != nsrc:
            raise ArgumentError(f"{kind.upper()} data does not hold a [{rows}, {cols}] matrix")
        src = self._lib.lab_gpu_buffer(nsrc)
        if src < 0:
            raise StateError(f"GPU buffer for the {kind} blocks failed")
        try:
            self._bytes_view(src, nsrc)[:] = blocks
            qs_bytes = count * (16 if q4 else 32)
            scales_at = (qs_bytes + 63) // 64 * 64
            nbytes = scales_at + count * (2 if q4 else 4)
            dst = self._lib.lab_gpu_buffer(nbytes)
            if dst < 0:
                raise StateError(f"GPU buffer of {nbytes} bytes failed")
            self._owned.append(dst)
            self._lib.lab_gpu_begin()
            enc = self._lib.lab_gpu_enc_split_q4_0 if q4 else self._lib.lab_gpu_enc_split_q8_0
            enc(src, 0, dst, 0, dst, scales_at, rows, cols)
            if self._lib.lab_gpu_commit(1) != 1:
                raise StateError("GPU command buffer failed")
        finally:
            self._lib.lab_gpu_release(src)
        self._replace(name, _Matrix(q4, dst, 0, scales_at, rows, cols, cols))

    def _upload_quantized(self, name: str, src_values: np.ndarray, esize: int, rows: int,
                          cols: int, rows_pad: int | None, fmt: str) -> None:
        self._check_open()
        if fmt not in ("q4", "q8"):
            raise ArgumentError(f"cannot quantize to {fmt}")
        if rows <= 0 or cols <= 0 or src_values.size < rows * cols:
            raise ArgumentError(f"invalid weights for {rows} x {cols}")
        q4 = fmt == "q4"
        if q4 and cols % 32 != 0:
            raise ArgumentError(f"Q4 needs cols to be a multiple of 32, got {cols}")
        cols_pad = (cols + 31) // 32 * 32
        out_rows = rows if rows_pad is None else rows_pad
        if out_rows < rows:
            raise ArgumentError("rows_pad must not be below rows")
        nsrc = rows * cols * esize
        src = self._lib.lab_gpu_buffer(nsrc)
        if src < 0:
            raise StateError("GPU buffer for the source weights failed")
        try:
            self._bytes_view(src, nsrc)[:] = src_values[: rows * cols].view(np.uint8)
            qs_bytes = out_rows * (cols_pad // 2 if q4 else cols_pad)
            scales_at = (qs_bytes + 63) // 64 * 64
            nbytes = scales_at + out_rows * (cols_pad // 32) * (2 if q4 else 4)
            dst = self._lib.lab_gpu_buffer(nbytes)
            if dst < 0:
                raise StateError(f"GPU buffer of {nbytes} bytes failed")
            self._owned.append(dst)
            self._lib.lab_gpu_begin()
            if q4:
                enc = (self._lib.lab_gpu_enc_quantize_q4_bf16 if esize == 2
                       else self._lib.lab_gpu_enc_quantize_q4)
                enc(src, 0, dst, 0, dst, scales_at, rows, cols)
            else:
                enc = (self._lib.lab_gpu_enc_quantize_q8_bf16 if esize == 2
                       else self._lib.lab_gpu_enc_quantize_q8)
                enc(src, 0, dst, 0, dst, scales_at, rows, cols, cols_pad)
            if self._lib.lab_gpu_commit(1) != 1:
                raise StateError("GPU command buffer failed")
        finally:
            self._lib.lab_gpu_release(src)
        self._replace(name, _Matrix(q4, dst, 0, scales_at, out_rows, cols_pad, cols))

    def quantized(self, name: str) -> tuple[np.ndarray, np.ndarray]:
        """The Q8 values and scales a matrix holds on the GPU (for checks)."""
        w = self._matrix(name)
        if w.q4:
            qs = self._bytes_view(w.buffer, w.qs + w.rows * w.cols // 2)[w.qs:]
            sc = self._bytes_view(w.buffer, w.scales + w.rows * w.cols // 16)[w.scales:]
            return qs.reshape(w.rows, w.cols // 2).copy(), sc.view(np.uint16).reshape(w.rows, -1).copy()
        qs = self._bytes_view(w.buffer, w.qs + w.rows * w.cols)[w.qs:]
        sc = self._bytes_view(w.buffer, w.scales + w.rows * w.cols // 8)[w.scales:]
        return (qs.view(np.int8).reshape(w.rows, w.cols).copy(),
                sc.view(np.float32).reshape(w.rows, -1).copy())

    # ------------------------------------------------------------ products

    def apply(self, name: str, xs: np.ndarray, ys: np.ndarray, n: int) -> None:
        """ys[t * rows + r] = (W xs[t])[r] for t < n, xs as [n, cols]."""
        self._check_open()
        w = self._matrix(name)
        xs = np.asarray(xs, dtype=np.float32).reshape(-1)
        if n < 1 or xs.size < n * w.in_cols or ys.size < n * w.rows:
            raise ArgumentError(f"GPU product: bad shapes for n={n}")
        x = self._x = self._grow(self._x, n * w.cols)
        y = self._y = self._grow(self._y, n * w.rows)
        self._write_rows(x, xs, n, w.in_cols, w.cols)
        self._lib.lab_gpu_begin()
        w.encode(self._lib, x.handle, y.handle, 0, n)
        self._finish()
        ys.reshape(-1)[: n * w.rows] = y.view(count=n * w.rows)

    def apply_argmax(self, name: str, xs: np.ndarray, logits: np.ndarray | None = None) -> int:
        """The greedy token of one input: argmaxToken over W xs, on the GPU."""
        self._check_open()
        w = self._matrix(name)
        xs = np.asarray(xs, dtype=np.float32).reshape(-1)
        if xs.size < w.in_cols:
            raise ArgumentError("GPU argmax: short input")
        x = self._x = self._grow(self._x, w.cols)
        y = self._y = self._grow(self._y, w.rows)
        out = self._aux_buffer("argmax", 2)
        self._write_rows(x, xs, 1, w.in_cols, w.cols)
        self._lib.lab_gpu_begin()
        w.encode(self._lib, x.handle, y.handle, 0, 1)
        self._lib.lab_gpu_enc_argmax(y.handle, 0, w.rows, out.handle, 0)
        self._finish()
        if logits is not None:
            logits.reshape(-1)[: w.rows] = y.view(count=w.rows)
        return int(out.view(np.int64, count=1)[0])

    def mlp(self, gate: str, up: str, down: str, xs: np.ndarray, ys: np.ndarray, n: int) -> None:
        """LayerShard.ffn (shard.dart:448-465): w2 (SiLU(w1 x) * (w3 x)), on the GPU."""
        self._check_open()
        g_m, u_m, d_m = self._matrix(gate), self._matrix(up), self._matrix(down)
        if g_m.rows != u_m.rows or d_m.cols != g_m.rows or g_m.cols != u_m.cols:
            raise ArgumentError("MLP shapes do not chain")
        xs = np.asarray(xs, dtype=np.float32).reshape(-1)
        if n < 1 or xs.size < n * g_m.in_cols or ys.size < n * d_m.rows:
            raise ArgumentError(f"GPU MLP: bad shapes for n={n}")
        x = self._x = self._grow(self._x, n * g_m.cols)
        y = self._y = self._grow(self._y, n * d_m.rows)
        g = self._aux_buffer("g", n * g_m.rows)
        u = self._aux_buffer("u", n * g_m.rows)
        self._write_rows(x, xs, n, g_m.in_cols, g_m.cols)
        self._lib.lab_gpu_begin()
        g_m.encode(self._lib, x.handle, g.handle, 0, n)
        u_m.encode(self._lib, x.handle, u.handle, 0, n)
        self._lib.lab_gpu_enc_swiglu(g.handle, u.handle, n * g_m.rows)
        d_m.encode(self._lib, g.handle, y.handle, 0, n)
        self._finish()
        ys.reshape(-1)[: n * d_m.rows] = y.view(count=n * d_m.rows)

    def gelu_pair(self, fc1: str, fc2: str, xs: np.ndarray, ys: np.ndarray, n: int,
                  intermediate: np.ndarray | None = None) -> None:
        """fc2(GELU(fc1 xs)), the projector's linear_1 -> GELU -> linear_2
        (vision_encoder.dart:252-271) without biases. fc1's rows may carry
        zero padding up to fc2's padded width. ``intermediate`` receives
        GELU(fc1 xs) ([n][fc1 rows]) when given."""
        self._check_open()
        a, b = self._matrix(fc1), self._matrix(fc2)
        if a.rows != b.cols:
            raise ArgumentError("fc1 rows must equal fc2's (padded) width")
        xs = np.asarray(xs, dtype=np.float32).reshape(-1)
        if n < 1 or xs.size < n * a.in_cols or ys.size < n * b.rows:
            raise ArgumentError(f"GPU projector: bad shapes for n={n}")
        x = self._x = self._grow(self._x, n * a.cols)
        y = self._y = self._grow(self._y, n * b.rows)
        h = self._aux_buffer("h", n * a.rows)
        self._write_rows(x, xs, n, a.in_cols, a.cols)
        self._lib.lab_gpu_begin()
        a.encode(self._lib, x.handle, h.handle, 0, n)
        self._lib.lab_gpu_enc_gelu(h.handle, 0, n * a.rows)
        b.encode(self._lib, h.handle, y.handle, 0, n)
        self._finish()
        ys.reshape(-1)[: n * b.rows] = y.view(count=n * b.rows)
        if intermediate is not None:
            intermediate.reshape(-1)[: n * a.rows] = h.view(count=n * a.rows)

    # ------------------------------------------------------------ lifecycle

    def dispose(self) -> None:
        """Releases every GPU buffer. Using this afterwards raises."""
        if self._disposed:
            return
        self._disposed = True
        for h in self._owned:
            self._lib.lab_gpu_release(h)
        self._owned.clear()
        self._matrices.clear()
        self._aux.clear()
        self._x = self._y = None

    # ------------------------------------------------------------ helpers

    def _finish(self) -> None:
        if self._lib.lab_gpu_commit(1) != 1:
            raise StateError("GPU command buffer failed")

    def _check_open(self) -> None:
        if self._disposed:
            raise StateError("the GPU products are disposed")

    def _matrix(self, name: str) -> _Matrix:
        w = self._matrices.get(name)
        if w is None:
            raise ArgumentError(f"no GPU matrix named {name}")
        return w

    def _replace(self, name: str, m: _Matrix) -> None:
        previous = self._matrices.get(name)
        if previous is not None and previous.owns:
            self._owned.remove(previous.buffer)
            self._lib.lab_gpu_release(previous.buffer)
        self._matrices[name] = m

    def _bytes_view(self, handle: int, nbytes: int) -> np.ndarray:
        ptr = self._lib.lab_gpu_contents(handle)
        if not ptr:
            raise StateError("lab_gpu_contents returned NULL")
        return np.frombuffer((ctypes.c_char * nbytes).from_address(ptr), dtype=np.uint8)

    def _grow(self, buffer: _Buffer | None, floats: int) -> _Buffer:
        """``buffer``, or a larger one replacing it (gpu.dart:1343-1353)."""
        if buffer is not None and buffer.length >= floats:
            return buffer
        if buffer is not None:
            self._owned.remove(buffer.handle)
            self._lib.lab_gpu_release(buffer.handle)
        grown = _Buffer(self._lib, floats)
        self._owned.append(grown.handle)
        return grown

    def _aux_buffer(self, key: str, floats: int) -> _Buffer:
        b = self._grow(self._aux.get(key), floats)
        self._aux[key] = b
        return b

    @staticmethod
    def _write_rows(buf: _Buffer, xs: np.ndarray, n: int, in_cols: int, cols: int) -> None:
        view = buf.view(count=n * cols)
        if in_cols == cols:
            view[:] = xs[: n * cols]
        else:
            v = view.reshape(n, cols)
            v[:, :in_cols] = xs[: n * in_cols].reshape(n, in_cols)
            v[:, in_cols:] = 0.0
