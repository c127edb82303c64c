"""The reference's native weight cache (``LFM3Q8C1``), read and written.

Mirrors ``lib/src/q8_cache.dart`` (``Q8Cache``): a file of Q8 (int8 values,
fp32 scales per 32-block) and Q4 (nibbles, fp16 scales) matrices, written
once and memory-mapped afterwards. Layout (q8_cache.dart:9-16, 209-286):

* the 8-byte magic ``LFM3Q8C1`` and a little-endian u64 header length;
* a JSON header ``{"version": 1, "key": ..., "tensors": {name: {"format",
  "rows", "cols", "qs", "scales"}}}`` (``format`` absent means ``q8``);
* zero padding up to a fixed 1 MiB header region, then each matrix's
  values and then its scales, each at a 64-byte aligned file offset, in the
  order the writer was given them.

``Q8Cache.open`` returns None for a miss (no file, another magic, another
version or key) and raises ``FormatException`` for a file with this magic
that cannot be trusted (header or a matrix outside the file, malformed
entries), releasing its mapping first (q8_cache.dart:63-104; the failure
cases of test/failure_recovery_test.dart:27-74). ``GpuLinear.wrap_cache``
places a mapped cache in HBM in whole-matrix segments (gpu.dart:938-979).

Host code only: the bytes of a matrix are exactly what the GPU kernels and
``GpuLinear.upload`` take (``formats.QuantMatrix``).
"""

from __future__ import annotations

import json
import mmap
import os
import struct
from typing import Callable, Iterable

import numpy as np

from .errors import ArgumentError, FormatException, StateError
from .formats import QuantMatrix

MAGIC = b"LFM3Q8C1"
VERSION = 1
HEADER_REGION = 1 << 20   # data offsets start here (q8_cache.dart:217-219)
ALIGN = 64                # every values / scales offset (q8_cache.dart:222-226)
MAX_SIDE = 1 << 31        # bound on rows and cols (q8_cache.dart:133)

_FNV_OFFSET = 0xCBF29CE484222325
_FNV_PRIME = 0x100000001B3
_MASK64 = (1 << 64) - 1


def fnv1a64(data: bytes, h: int = _FNV_OFFSET) -> int:
    """64-bit FNV-1a over ``data`` starting from ``h`` (q8_cache.dart:289-299;
    Dart's int arithmetic wraps at 64 bits, as the mask does here)."""
    for b in data:
        h = ((h ^ b) * _FNV_PRIME) & _MASK64
    return h


def byte_lengths(fmt: str, rows: int, cols: int) -> tuple[int, int]:
    """Bytes of values and of scales (q8_cache.dart:278-284)."""
    if fmt == "q8":
        return rows * cols, rows * cols // 32 * 4
    if fmt == "q4":
        return rows * cols // 2, rows * cols // 32 * 2
    raise ArgumentError(f"unknown matrix format {fmt}")


class MappedFile:
    """A read-only mapping of a whole file, shared by path and counted
    (native.dart:268-320): ``open`` of a mapped path hands out the same
    mapping, and the last ``release`` unmaps it."""

    _mapped: dict[str, "MappedFile"] = {}

    def __init__(self, path: str, mm: mmap.mmap):
        self.path = path
        self._mm = mm
        self.bytes = np.frombuffer(mm, dtype=np.uint8)
        self.length = len(mm)
        self._opens = 1

    @classmethod
    def open(cls, path: str) -> "MappedFile | None":
        """Maps ``path``, or None if it cannot be opened or is empty."""
        key = os.path.abspath(path)
        f = cls._mapped.get(key)
        if f is not None:
            f._opens += 1
            return f
        try:
            with open(path, "rb") as fh:
                mm = mmap.mmap(fh.fileno(), 0, access=mmap.ACCESS_READ)
        except (OSError, ValueError):
            return None
        f = cls(key, mm)
        cls._mapped[key] = f
        return f

    @classmethod
    def is_mapped(cls, path: str) -> bool:
        return os.path.abspath(path) in cls._mapped

    @property
    def address(self) -> int:
        """The mapping's first byte, for lab_gpu_wrap."""
        return self.bytes.ctypes.data

    def release(self) -> None:
        if self._opens == 0:
            return
        self._opens -= 1
        if self._opens > 0:
            return
        self._mapped.pop(self.path, None)
        self.bytes = None
        try:
            self._mm.close()
        except BufferError:
            # Matrix views handed out earlier still export the buffer; the
            # mapping goes when the last of them is collected.
            pass


class Q8Cache:
    """An open cache: its mapping and header entries (q8_cache.dart:29-34)."""

    def __init__(self, file: MappedFile, entries: dict[str, dict]):
        self._file = file
        self._entries = entries

    # ------------------------------------------------------------ key

    @staticmethod
    def key_for(model_dir: str, weights: str = "q8") -> str:
        """Fingerprint of the checkpoint in ``model_dir`` (its safetensors
        header, the file's size, config.json) and of this cache format for
        ``weights`` (q8_cache.dart:36-54): 16 lower-case hex digits."""
        st_path = os.path.join(model_dir, "model.safetensors")
        with open(st_path, "rb") as st:
            length_bytes = st.read(8)
            (header_length,) = struct.unpack("<Q", length_bytes)
            h = fnv1a64(length_bytes)
            h = fnv1a64(st.read(header_length), h)
            h = fnv1a64(str(os.path.getsize(st_path)).encode(), h)
        with open(os.path.join(model_dir, "config.json"), "rb") as cfg:
            h = fnv1a64(cfg.read(), h)
        h = fnv1a64(f"{MAGIC.decode()} v{VERSION} {weights} block 32".encode(), h)
        return f"{h:016x}"

    # ------------------------------------------------------------ open

    @staticmethod
    def open(path: str, key: str) -> "Q8Cache | None":
        """The cache at ``path`` if it holds ``key``; None on a miss; raises
        ``FormatException`` (after releasing the mapping) for a cache of this
        magic whose header or matrices do not fit the file, and
        ``StateError`` when an existing file cannot be mapped
        (q8_cache.dart:63-104)."""
        length = os.path.getsize(path) if os.path.exists(path) else 0
        if length < 16:
            return None
        f = MappedFile.open(path)
        if f is None:
            raise StateError(f"mapping {path} ({length} bytes) failed")
        try:
            if bytes(f.bytes[:8]) != MAGIC:
                f.release()
                return None
            (header_length,) = struct.unpack("<Q", bytes(f.bytes[8:16]))
            if header_length > f.length - 16:
                raise FormatException(f"{path}: header exceeds the file")
            try:
                header = json.loads(bytes(f.bytes[16:16 + header_length]).decode("utf-8"))
            except (UnicodeDecodeError, json.JSONDecodeError) as e:
                raise FormatException(f"{path}: header is not JSON ({e})") from None
            if not isinstance(header, dict):
                raise FormatException(f"{path}: header is not an object")
            if header.get("version") != VERSION or header.get("key") != key:
                f.release()
                return None
            tensors = header.get("tensors")
            if not isinstance(tensors, dict):
                raise FormatException(f"{path}: header lacks tensors")
            entries = {}
            for name, value in tensors.items():
                if not isinstance(value, dict) or not Q8Cache._fits(value, f.length):
                    raise FormatException(f"{path}: {name} does not fit the file")
                entries[name] = value
            return Q8Cache(f, entries)
        except FormatException:
            f.release()
            raise

    @staticmethod
    def _fits(e: dict, file_length: int) -> bool:
        """Whether an entry is a matrix of a known format whose values and
        scales lie inside the file, scales aligned for their type
        (q8_cache.dart:106-131)."""
        fmt = e.get("format", "q8")
        rows, cols, qs, scales = (e.get(k) for k in ("rows", "cols", "qs", "scales"))

        def is_int(v):  # JSON integers only (a bool is no int in Dart)
            return isinstance(v, int) and not isinstance(v, bool)

        if fmt not in ("q8", "q4") or not all(is_int(v) for v in (rows, cols, qs, scales)):
            return False
        if rows <= 0 or cols <= 0 or rows > MAX_SIDE or cols > MAX_SIDE or cols % 32 != 0:
            return False
        qs_len, sc_len = byte_lengths(fmt, rows, cols)
        return (qs >= 0 and scales >= 0 and scales % (2 if fmt == "q4" else 4) == 0
                and qs <= file_length - qs_len and scales <= file_length - sc_len)

    # ------------------------------------------------------------ access

    @property
    def file(self) -> MappedFile:
        """The mapping, for handing the whole file to the GPU in one piece."""
        return self._file

    def close(self) -> None:
        """Releases the mapping (once no other open of it holds it). The
        matrices from ``matrix`` view it and must not be used afterwards."""
        self._file.release()

    @property
    def shapes(self) -> Iterable[tuple[str, int, int]]:
        """Every cached matrix: name, rows and columns."""
        return [(name, e["rows"], e["cols"]) for name, e in self._entries.items()]

    def offsets(self, name: str, rows: int, cols: int) -> dict | None:
        """Matrix ``name``'s format and the file offsets of its values and
        scales, and the end of its scales; None if absent or of another
        shape (q8_cache.dart:146-168)."""
        e = self._entries.get(name)
        if e is None or e["rows"] != rows or e["cols"] != cols:
            return None
        fmt = e.get("format", "q8")
        scale_bytes = rows * cols // 32 * (2 if fmt == "q4" else 4)
        return {"format": fmt, "qs": e["qs"], "scales": e["scales"],
                "end": e["scales"] + scale_bytes}

    def matrix(self, name: str, rows: int, cols: int) -> QuantMatrix | None:
        """The cached matrix as views of the mapping, or None
        (q8_cache.dart:170-188)."""
        o = self.offsets(name, rows, cols)
        if o is None:
            return None
        qs_len, sc_len = byte_lengths(o["format"], rows, cols)
        b = self._file.bytes
        return QuantMatrix(o["format"], rows, cols, b[o["qs"]:o["qs"] + qs_len],
                           b[o["scales"]:o["scales"] + sc_len])

    # ------------------------------------------------------------ write

    @staticmethod
    def write(path: str, key: str, matrices: dict[str, QuantMatrix]) -> None:
        """Writes ``matrices`` under ``key`` (q8_cache.dart:190-201)."""
        Q8Cache.write_each(path, key,
                           [(n, m.format, m.rows, m.cols) for n, m in matrices.items()],
                           lambda n: matrices[n])

    @staticmethod
    def write_each(path: str, key: str, shapes: list[tuple[str, str, int, int]],
                   matrix: Callable[[str], QuantMatrix],
                   done: Callable[[QuantMatrix], None] | None = None) -> None:
        """Writes the matrices ``shapes`` lists (name, format, rows, cols), in
        that order, asking ``matrix`` for each when its turn comes and passing
        it to ``done`` once written, through ``path + '.partial'`` and a
        rename so a reader never maps a half-written cache
        (q8_cache.dart:203-276)."""
        def align(v: int) -> int:
            return (v + ALIGN - 1) // ALIGN * ALIGN

        offset = HEADER_REGION
        tensors: dict[str, dict] = {}
        for name, fmt, rows, cols in shapes:
            qs_len, sc_len = byte_lengths(fmt, rows, cols)
            qs = offset = align(offset)
            offset += qs_len
            scales = offset = align(offset)
            offset += sc_len
            tensors[name] = {"format": fmt, "rows": rows, "cols": cols, "qs": qs,
                             "scales": scales}
        header = json.dumps({"version": VERSION, "key": key, "tensors": tensors},
                            separators=(",", ":")).encode()
        if 16 + len(header) > HEADER_REGION:
            raise StateError("Q8 cache header does not fit")
        temp = path + ".partial"
        with open(temp, "wb") as out:
            out.write(MAGIC + struct.pack("<Q", len(header)))
            out.write(header)
            for name, fmt, rows, cols in shapes:
                m = matrix(name)
                try:
                    qs_len, sc_len = byte_lengths(fmt, rows, cols)
                    if (m.format != fmt or m.qs_bytes.size != qs_len
                            or m.scale_bytes.size != sc_len):
                        raise StateError(f"{name} is not a {fmt} [{rows}, {cols}] matrix")
                    e = tensors[name]
                    out.seek(e["qs"])
                    out.write(np.ascontiguousarray(m.qs_bytes).tobytes())
                    out.seek(e["scales"])
                    out.write(np.ascontiguousarray(m.scale_bytes).tobytes())
                finally:
                    if done is not None:
                        done(m)
        os.replace(temp, path)
