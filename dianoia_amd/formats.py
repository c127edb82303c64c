"""Host-side weight formats on the path: GGUF block splitting, BF16 and fp16.

These run once at import or load time on the host (numpy), before weights
reach the GPU, exactly where the reference runs them in Dart:

* ``split_q8_0`` / ``split_q4_0``: GGUF Q8_0 (fp16 d + 32 int8) and Q4_0
  (fp16 d + 16 nibble bytes) blocks into the engine's separate value and
  scale arrays (lib/src/gguf.dart:206-218, 267-282; NativeQ4Matrix.
  fromGgufBlocks, native.dart:766-790). Q8_0's d is widened to fp32
  exactly; every byte is otherwise copied.
* ``widen_bf16``: bf16 bits p -> fp32 bits p << 16 (safetensors.dart:207-212).
* ``QuantMatrix``: what GpuLinear.upload takes, the reference's
  CachedMatrix (native.dart:598-608): format, rows, cols, raw value and
  scale bytes.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .errors import ArgumentError


@dataclass
class QuantMatrix:
    format: str          # "q8" or "q4"
    rows: int
    cols: int
    qs_bytes: np.ndarray     # uint8 view of the values
    scale_bytes: np.ndarray  # uint8 view of the scales

    @staticmethod
    def q8(qs: np.ndarray, scales: np.ndarray) -> "QuantMatrix":
        qs = np.ascontiguousarray(qs, dtype=np.int8)
        scales = np.ascontiguousarray(scales, dtype=np.float32)
        rows, cols = qs.shape
        if cols % 32 or scales.size != rows * cols // 32:
            raise ArgumentError(f"invalid Q8 matrix {rows} x {cols}")
        return QuantMatrix("q8", rows, cols, qs.reshape(-1).view(np.uint8),
                           scales.reshape(-1).view(np.uint8))

    @staticmethod
    def q4(qs: np.ndarray, scales: np.ndarray) -> "QuantMatrix":
        qs = np.ascontiguousarray(qs, dtype=np.uint8)
        scales = np.ascontiguousarray(scales, dtype=np.uint16)
        rows, half = qs.shape
        cols = half * 2
        if cols % 32 or scales.size != rows * cols // 32:
            raise ArgumentError(f"invalid Q4 matrix {rows} x {cols}")
        return QuantMatrix("q4", rows, cols, qs.reshape(-1), scales.reshape(-1).view(np.uint8))


def half_to_float(bits: np.ndarray) -> np.ndarray:
    """IEEE binary16 bits -> float32, exact (lab_native.c:919-921)."""
    return np.ascontiguousarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def float_to_half(values: np.ndarray) -> np.ndarray:
    """float32 -> binary16 bits, round to nearest even (lab_native.c:923-925)."""
    return np.asarray(values, dtype=np.float32).astype(np.float16).view(np.uint16)


def widen_bf16(bits: np.ndarray) -> np.ndarray:
    """bf16 bits -> float32: p << 16 (safetensors.dart:207-212)."""
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def split_q8_0(blocks: np.ndarray, rows: int, cols: int) -> QuantMatrix:
    """GGUF Q8_0 blocks -> engine Q8 (int8 values + fp32 scales), gguf.dart:270-282."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    count = rows * cols // 32
    if rows <= 0 or cols <= 0 or cols % 32 or blocks.size != count * 34:
        raise ArgumentError(f"Q8_0 data does not hold a [{rows}, {cols}] matrix")
    b = blocks.reshape(count, 34)
    scales = half_to_float(b[:, :2].copy().view(np.uint16).reshape(-1))
    # halfToDouble (native.dart:871-880) returns Dart's double.nan for every
    # NaN pattern, which a Float32List stores as 0x7FC00000.
    scales[np.isnan(scales)] = np.uint32(0x7FC00000).view(np.float32)
    qs = b[:, 2:].copy().view(np.int8).reshape(rows, cols)
    return QuantMatrix.q8(qs, scales.reshape(rows, cols // 32))


def split_q4_0(blocks: np.ndarray, rows: int, cols: int) -> QuantMatrix:
    """GGUF Q4_0 blocks -> engine Q4 (nibbles + fp16 scale bits), gguf.dart:208-218."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    count = rows * cols // 32
    if rows <= 0 or cols <= 0 or cols % 32 or blocks.size != count * 18:
        raise ArgumentError(f"invalid Q4_0 blocks for {rows} x {cols}")
    b = blocks.reshape(count, 18)
    scales = b[:, :2].copy().view(np.uint16).reshape(rows, cols // 32)
    qs = b[:, 2:].copy().reshape(rows, cols // 2)
    return QuantMatrix.q4(qs, scales)


def join_q8_0(qs: np.ndarray, d_bits: np.ndarray) -> np.ndarray:
    """Engine Q8 values + fp16 d bits -> GGUF Q8_0 blocks (the inverse layout)."""
    qs = np.ascontiguousarray(qs, dtype=np.int8).reshape(-1, 32)
    d = np.ascontiguousarray(d_bits, dtype=np.uint16).reshape(-1, 1)
    return np.concatenate([d.view(np.uint8).reshape(-1, 2), qs.view(np.uint8)], axis=1).reshape(-1)


def join_q4_0(qs: np.ndarray, d_bits: np.ndarray) -> np.ndarray:
    """Engine Q4 nibbles + fp16 d bits -> GGUF Q4_0 blocks."""
    qs = np.ascontiguousarray(qs, dtype=np.uint8).reshape(-1, 16)
    d = np.ascontiguousarray(d_bits, dtype=np.uint16).reshape(-1, 1)
    return np.concatenate([d.view(np.uint8).reshape(-1, 2), qs], axis=1).reshape(-1)
