"""The dnx_* device launchers for torch tensors already in HBM.

torch supplies device memory and the stream (plumbing); the computation is
the library's HIP kernels. Every function enqueues on the current torch
stream (or ``stream``) and raises on a non-zero return code, before which
nothing was launched.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib


def _stream(stream=None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("device launchers take CUDA (HIP) tensors")
    if not t.is_contiguous():
        raise ValueError("device launchers take contiguous tensors")
    return t.data_ptr()


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed with code {rc}")


def _need(what: str, **operands) -> None:
    """Refuses, before any launch, an operand tensor smaller than the bytes
    the kernel will touch for the given shape (the C ABI takes bare
    pointers and cannot tell)."""
    for name, (t, nbytes) in operands.items():
        if t is not None and nbytes > 0 and t.numel() * t.element_size() < nbytes:
            raise ValueError(f"{what}: {name} holds {t.numel() * t.element_size()} bytes, "
                             f"the shape needs {nbytes}")


def quantize_q8(x: torch.Tensor, qs: torch.Tensor, scales: torch.Tensor, rows: int, cols: int,
                cols_pad: int, stream=None) -> None:
    _need("quantize_q8",
          x=(x, rows * cols * 4),
          qs=(qs, rows * cols_pad),
          scales=(scales, rows * (cols_pad // 32) * 4))
    _check(_lib.load().dnx_quantize_q8(_ptr(x), _ptr(qs), _ptr(scales), rows, cols, cols_pad,
                                       _stream(stream)), "dnx_quantize_q8")


def quantize_q8_bf16(w: torch.Tensor, qs: torch.Tensor, scales: torch.Tensor, rows: int,
                     cols: int, cols_pad: int, stream=None) -> None:
    _check(_lib.load().dnx_quantize_q8_bf16(_ptr(w), _ptr(qs), _ptr(scales), rows, cols,
                                            cols_pad, _stream(stream)), "dnx_quantize_q8_bf16")


def quantize_q4(w: torch.Tensor, qs: torch.Tensor, scales: torch.Tensor, rows: int, cols: int,
                stream=None) -> None:
    """lab_quantize_q4 on the GPU: fp32 [rows][cols] -> nibbles [rows][cols/2] + fp16 bits."""
    _check(_lib.load().dnx_quantize_q4(_ptr(w), _ptr(qs), _ptr(scales), rows, cols,
                                       _stream(stream)), "dnx_quantize_q4")


def q6k_to_q8(blocks: torch.Tensor, qs: torch.Tensor, scales: torch.Tensor, rows: int, cols: int,
              stream=None) -> None:
    """Q6_K super-blocks -> the engine's Q8 (dequantizeQ6K + lab_quantize_q8, fused)."""
    _check(_lib.load().dnx_q6k_to_q8(_ptr(blocks), _ptr(qs), _ptr(scales), rows, cols,
                                     _stream(stream)), "dnx_q6k_to_q8")


def split_q8_0(blocks: torch.Tensor, qs: torch.Tensor, scales: torch.Tensor, count: int,
               stream=None) -> None:
    """GGUF Q8_0 blocks -> int8 values + fp32 scales (splitQ8_0, gguf.dart:270-282)."""
    _check(_lib.load().dnx_split_q8_0(_ptr(blocks), _ptr(qs), _ptr(scales), count,
                                      _stream(stream)), "dnx_split_q8_0")


def split_q4_0(blocks: torch.Tensor, qs: torch.Tensor, scales: torch.Tensor, count: int,
               stream=None) -> None:
    """GGUF Q4_0 blocks -> nibble bytes + fp16 scale bits (splitQ4_0, gguf.dart:208-218)."""
    _check(_lib.load().dnx_split_q4_0(_ptr(blocks), _ptr(qs), _ptr(scales), count,
                                      _stream(stream)), "dnx_split_q4_0")


def quantize_q4_bf16(w: torch.Tensor, qs: torch.Tensor, scales: torch.Tensor, rows: int,
                     cols: int, stream=None) -> None:
    """BF16 bits widened (p << 16), then lab_quantize_q4, in one kernel."""
    _check(_lib.load().dnx_quantize_q4_bf16(_ptr(w), _ptr(qs), _ptr(scales), rows, cols,
                                            _stream(stream)), "dnx_quantize_q4_bf16")


def gemv_q8(qs, scales, x, y, rows: int, cols: int, n: int = 1, stream=None) -> None:
    _need("gemv_q8",
          qs=(qs, rows * cols),
          scales=(scales, rows * (cols // 32) * 4),
          x=(x, n * cols * 4),
          y=(y, n * rows * 4))
    _check(_lib.load().dnx_gemv_q8(_ptr(qs), _ptr(scales), _ptr(x), _ptr(y), rows, cols, n,
                                   _stream(stream)), "dnx_gemv_q8")


def gemv_q4(qs, scales, x, y, rows: int, cols: int, n: int = 1, stream=None) -> None:
    _need("gemv_q4",
          qs=(qs, rows * cols // 2),
          scales=(scales, rows * (cols // 32) * 2),
          x=(x, n * cols * 4),
          y=(y, n * rows * 4))
    _check(_lib.load().dnx_gemv_q4(_ptr(qs), _ptr(scales), _ptr(x), _ptr(y), rows, cols, n,
                                   _stream(stream)), "dnx_gemv_q4")


def gemv_q8_float(qs, scales, x, y, rows: int, cols: int, n: int = 1, stream=None) -> None:
    """Float-input GEMV (lab_gemm_q8 mode 0), any n."""
    _need("gemv_q8_float",
          qs=(qs, rows * cols),
          scales=(scales, rows * (cols // 32) * 4),
          x=(x, n * cols * 4),
          y=(y, n * rows * 4))
    _check(_lib.load().dnx_gemv_q8_float(_ptr(qs), _ptr(scales), _ptr(x), _ptr(y), rows, cols, n,
                                         _stream(stream)), "dnx_gemv_q8_float")


def gemv_q4_float(qs, scales, x, y, rows: int, cols: int, n: int = 1, stream=None) -> None:
    """Float-input GEMV (lab_gemm_q4 mode 0), any n."""
    _need("gemv_q4_float",
          qs=(qs, rows * cols // 2),
          scales=(scales, rows * (cols // 32) * 2),
          x=(x, n * cols * 4),
          y=(y, n * rows * 4))
    _check(_lib.load().dnx_gemv_q4_float(_ptr(qs), _ptr(scales), _ptr(x), _ptr(y), rows, cols, n,
                                         _stream(stream)), "dnx_gemv_q4_float")


def gemv_argmax_workspace(device="cuda") -> torch.Tensor:
    """Zeroed workspace for the fused argmax GEMV; completed calls leave it zero."""
    nbytes = int(_lib.load().dnx_gemv_argmax_workspace_bytes())
    return torch.zeros(nbytes, dtype=torch.uint8, device=device)


def gemv_q8_argmax(qs, scales, x, y, out, workspace, rows: int, cols: int, stream=None) -> None:
    _check(_lib.load().dnx_gemv_q8_argmax(_ptr(qs), _ptr(scales), _ptr(x), _ptr(y), rows, cols,
                                          _ptr(out), _ptr(workspace), _stream(stream)),
           "dnx_gemv_q8_argmax")


def gemv_q4_argmax(qs, scales, x, y, out, workspace, rows: int, cols: int, stream=None) -> None:
    _check(_lib.load().dnx_gemv_q4_argmax(_ptr(qs), _ptr(scales), _ptr(x), _ptr(y), rows, cols,
                                          _ptr(out), _ptr(workspace), _stream(stream)),
           "dnx_gemv_q4_argmax")


def gate_up_q8(gq, gs, uq, us, x, h, rows: int, cols: int, n: int = 1, u=None,
               stream=None) -> None:
    _check(_lib.load().dnx_gate_up_q8(_ptr(gq), _ptr(gs), _ptr(uq), _ptr(us), _ptr(x), _ptr(h),
                                      _ptr(u), rows, cols, n, _stream(stream)), "dnx_gate_up_q8")


def gate_up_q4(gq, gs, uq, us, x, h, rows: int, cols: int, n: int = 1, u=None,
               stream=None) -> None:
    _check(_lib.load().dnx_gate_up_q4(_ptr(gq), _ptr(gs), _ptr(uq), _ptr(us), _ptr(x), _ptr(h),
                                      _ptr(u), rows, cols, n, _stream(stream)), "dnx_gate_up_q4")


def gemv_q8h(qs, scales, x, y, rows: int, cols: int, n: int = 1, stream=None) -> None:
    """Q8 GEMV with fp16 block scales (uint16 bits, the GGUF Q8_0 d)."""
    _check(_lib.load().dnx_gemv_q8h(_ptr(qs), _ptr(scales), _ptr(x), _ptr(y), rows, cols, n,
                                    _stream(stream)), "dnx_gemv_q8h")


def gemv_q8h_argmax(qs, scales, x, y, out, workspace, rows: int, cols: int, stream=None) -> None:
    _check(_lib.load().dnx_gemv_q8h_argmax(_ptr(qs), _ptr(scales), _ptr(x), _ptr(y), rows, cols,
                                           _ptr(out), _ptr(workspace), _stream(stream)),
           "dnx_gemv_q8h_argmax")


def gate_up_q8h(gq, gs, uq, us, x, h, rows: int, cols: int, n: int = 1, u=None,
                stream=None) -> None:
    _check(_lib.load().dnx_gate_up_q8h(_ptr(gq), _ptr(gs), _ptr(uq), _ptr(us), _ptr(x), _ptr(h),
                                       _ptr(u), rows, cols, n, _stream(stream)), "dnx_gate_up_q8h")


def copy_regions(regions, stream=None) -> None:
    """Byte copies in one launch: regions is a list of (src_ptr, dst_ptr,
    bytes) with device or pinned-host pointers (ints)."""
    count = len(regions)
    P = ctypes.c_void_p * max(count, 1)
    src = P(*[r[0] for r in regions])
    dst = P(*[r[1] for r in regions])
    nb = (ctypes.c_int64 * max(count, 1))(*[int(r[2]) for r in regions])
    _check(_lib.load().dnx_copy_regions(ctypes.cast(src, ctypes.c_void_p), ctypes.cast(dst, ctypes.c_void_p),
                                        ctypes.cast(nb, ctypes.c_void_p), count, _stream(stream)),
           "dnx_copy_regions")


def gemv_multi(fmt: str, mats, x, ys, cols: int, stream=None) -> None:
    """Up to 4 one-token GEMVs over the same x in one launch: mats is a list of
    (qs, scales, rows), ys the matching outputs; fmt "q8", "q4" or "q8h"."""
    segs = len(mats)
    P = ctypes.c_void_p * max(segs, 1)
    qs = P(*[_ptr(m[0]) for m in mats])
    sc = P(*[_ptr(m[1]) for m in mats])
    yp = P(*[_ptr(y) for y in ys])
    rows = (ctypes.c_int64 * max(segs, 1))(*[int(m[2]) for m in mats])
    name = {"q8": "dnx_gemv_multi_q8", "q4": "dnx_gemv_multi_q4", "q8h": "dnx_gemv_multi_q8h"}[fmt]
    _check(getattr(_lib.load(), name)(ctypes.cast(qs, ctypes.c_void_p), ctypes.cast(sc, ctypes.c_void_p),
                                      ctypes.cast(yp, ctypes.c_void_p), ctypes.cast(rows, ctypes.c_void_p),
                                      segs, _ptr(x), cols, _stream(stream)), name)


def gemv_add(fmt: str, qs, scales, x, y, resid, rows: int, cols: int, stream=None) -> None:
    """One-token GEMV whose epilogue also adds y into resid (fmt "q8" or "q4")."""
    name = {"q8": "dnx_gemv_add_q8", "q4": "dnx_gemv_add_q4"}[fmt]
    _check(getattr(_lib.load(), name)(_ptr(qs), _ptr(scales), _ptr(x), _ptr(y), _ptr(resid), rows,
                                      cols, _stream(stream)), name)


def gate_up_norm(fmt: str, gq, gs, uq, us, x, norm_w, norm_out, eps: float, h, u, rows: int,
                 cols: int, stream=None) -> None:
    """The gate/up pair and glue on RMSNorm(x) * norm_w, which also goes to norm_out."""
    name = {"q8": "dnx_gate_up_norm_q8", "q4": "dnx_gate_up_norm_q4"}[fmt]
    _check(getattr(_lib.load(), name)(_ptr(gq), _ptr(gs), _ptr(uq), _ptr(us), _ptr(x), _ptr(norm_w),
                                      _ptr(norm_out), eps, _ptr(h), _ptr(u), rows, cols,
                                      _stream(stream)), name)


def gemv_multi_norm(fmt: str, mats, x, norm_w, norm_out, eps: float, ys, cols: int,
                    stream=None) -> None:
    """gemv_multi on RMSNorm(x) * norm_w, which also goes to norm_out."""
    segs = len(mats)
    P = ctypes.c_void_p * max(segs, 1)
    qs = P(*[_ptr(m[0]) for m in mats])
    sc = P(*[_ptr(m[1]) for m in mats])
    yp = P(*[_ptr(y) for y in ys])
    rows = (ctypes.c_int64 * max(segs, 1))(*[int(m[2]) for m in mats])
    name = {"q8": "dnx_gemv_multi_norm_q8", "q4": "dnx_gemv_multi_norm_q4"}[fmt]
    _check(getattr(_lib.load(), name)(ctypes.cast(qs, ctypes.c_void_p), ctypes.cast(sc, ctypes.c_void_p),
                                      ctypes.cast(yp, ctypes.c_void_p), ctypes.cast(rows, ctypes.c_void_p),
                                      segs, _ptr(x), _ptr(norm_w), _ptr(norm_out), eps, cols,
                                      _stream(stream)), name)


def gemm_q8_float(qs, scales, x, y, rows: int, cols: int, n: int, stream=None) -> None:
    """Float-input (mode 0) GEMM on bf16 MFMA, within fp32 rounding of the CPU."""
    _need("gemm_q8_float",
          qs=(qs, rows * cols),
          scales=(scales, rows * (cols // 32) * 4),
          x=(x, n * cols * 4),
          y=(y, n * rows * 4))
    _check(_lib.load().dnx_gemm_q8_float(_ptr(qs), _ptr(scales), _ptr(x), _ptr(y), rows, cols, n,
                                         _stream(stream)), "dnx_gemm_q8_float")


def gemm_q4_float(qs, scales, x, y, rows: int, cols: int, n: int, stream=None) -> None:
    _need("gemm_q4_float",
          qs=(qs, rows * cols // 2),
          scales=(scales, rows * (cols // 32) * 2),
          x=(x, n * cols * 4),
          y=(y, n * rows * 4))
    _check(_lib.load().dnx_gemm_q4_float(_ptr(qs), _ptr(scales), _ptr(x), _ptr(y), rows, cols, n,
                                         _stream(stream)), "dnx_gemm_q4_float")


def gemm_q8(qs, scales, xq, xsc, y, rows: int, cols: int, n: int, stream=None) -> None:
    _need("gemm_q8",
          qs=(qs, rows * cols),
          scales=(scales, rows * (cols // 32) * 4),
          xq=(xq, n * cols),
          xsc=(xsc, n * (cols // 32) * 4),
          y=(y, n * rows * 4))
    _check(_lib.load().dnx_gemm_q8(_ptr(qs), _ptr(scales), _ptr(xq), _ptr(xsc), _ptr(y), rows,
                                   cols, n, _stream(stream)), "dnx_gemm_q8")


def gemm_q4(qs, scales, xq, xsc, y, rows: int, cols: int, n: int, stream=None) -> None:
    _need("gemm_q4",
          qs=(qs, rows * cols // 2),
          scales=(scales, rows * (cols // 32) * 2),
          xq=(xq, n * cols),
          xsc=(xsc, n * (cols // 32) * 4),
          y=(y, n * rows * 4))
    _check(_lib.load().dnx_gemm_q4(_ptr(qs), _ptr(scales), _ptr(xq), _ptr(xsc), _ptr(y), rows,
                                   cols, n, _stream(stream)), "dnx_gemm_q4")


def gemm_panel_bytes(n: int, cols: int) -> int:
    return int(_lib.load().dnx_gemm_panel_bytes(n, cols))


def pack_panel(xq, xsc, panel, n: int, cols: int, stream=None) -> None:
    """xq int8 [n][cols] + xsc fp32 [n][cols/32] -> the GEMM's activation panel."""
    _check(_lib.load().dnx_pack_panel(_ptr(xq), _ptr(xsc), _ptr(panel), n, cols,
                                      _stream(stream)), "dnx_pack_panel")


def quantize_q8_panel(x, panel, n: int, cols: int, stream=None) -> None:
    """fp32 x [n][cols] quantized (lab_quantize_q8) straight into the GEMM's panel."""
    _need("quantize_q8_panel", x=(x, n * cols * 4), panel=(panel, gemm_panel_bytes(n, cols)))
    _check(_lib.load().dnx_quantize_q8_panel(_ptr(x), _ptr(panel), n, cols, _stream(stream)),
           "dnx_quantize_q8_panel")


def gemm_q8_panel(qs, scales, panel, y, rows: int, cols: int, n: int, stream=None) -> None:
    _check(_lib.load().dnx_gemm_q8_panel(_ptr(qs), _ptr(scales), _ptr(panel), _ptr(y), rows,
                                         cols, n, _stream(stream)), "dnx_gemm_q8_panel")


def gemm_q4_panel(qs, scales, panel, y, rows: int, cols: int, n: int, stream=None) -> None:
    _check(_lib.load().dnx_gemm_q4_panel(_ptr(qs), _ptr(scales), _ptr(panel), _ptr(y), rows,
                                         cols, n, _stream(stream)), "dnx_gemm_q4_panel")


def f6_panel_bytes(n: int, cols: int) -> int:
    return int(_lib.load().dnx_f6_panel_bytes(n, cols))


def quantize_q8_f6panel(x, panel, n: int, cols: int, stream=None) -> None:
    """fp32 x [n][cols] quantized (lab_quantize_q8) into the fp6 GEMM's panel."""
    _need("quantize_q8_f6panel", x=(x, n * cols * 4), panel=(panel, f6_panel_bytes(n, cols)))
    _check(_lib.load().dnx_quantize_q8_f6panel(_ptr(x), _ptr(panel), n, cols, _stream(stream)),
           "dnx_quantize_q8_f6panel")


def pack_f6panel(xq, xsc, panel, n: int, cols: int, stream=None) -> None:
    """xq int8 [n][cols] + xsc fp32 [n][cols/32] -> the fp6 GEMM's panel."""
    _need("pack_f6panel",
          xq=(xq, n * cols),
          xsc=(xsc, n * (cols // 32) * 4),
          panel=(panel, f6_panel_bytes(n, cols)))
    _check(_lib.load().dnx_pack_f6panel(_ptr(xq), _ptr(xsc), _ptr(panel), n, cols,
                                        _stream(stream)), "dnx_pack_f6panel")


def gemm_q4_f6(qs, scales, panel, y, rows: int, cols: int, n: int, stream=None) -> None:
    _need("gemm_q4_f6",
          qs=(qs, rows * cols // 2),
          scales=(scales, rows * (cols // 32) * 2),
          panel=(panel, f6_panel_bytes(n, cols)),
          y=(y, n * rows * 4))
    _check(_lib.load().dnx_gemm_q4_f6(_ptr(qs), _ptr(scales), _ptr(panel), _ptr(y), rows, cols,
                                      n, _stream(stream)), "dnx_gemm_q4_f6")


def q4_f6pack_bytes(rows: int, cols: int) -> int:
    return int(_lib.load().dnx_q4_f6pack_bytes(rows, cols))


def pack_q4_f6(qs, scales, packed, rows: int, cols: int, stream=None) -> None:
    """Load-time re-encoding of Q4 weights for the fp6 GEMM (dnx_gemm_q4_f6p)."""
    _need("pack_q4_f6",
          qs=(qs, rows * cols // 2),
          scales=(scales, rows * (cols // 32) * 2),
          packed=(packed, q4_f6pack_bytes(rows, cols)))
    _check(_lib.load().dnx_pack_q4_f6(_ptr(qs), _ptr(scales), _ptr(packed), rows, cols,
                                      _stream(stream)), "dnx_pack_q4_f6")


def gemm_q4_f6p(packed, panel, y, rows: int, cols: int, n: int, stream=None) -> None:
    _need("gemm_q4_f6p",
          packed=(packed, q4_f6pack_bytes(rows, cols)),
          panel=(panel, f6_panel_bytes(n, cols)),
          y=(y, n * rows * 4))
    _check(_lib.load().dnx_gemm_q4_f6p(_ptr(packed), _ptr(panel), _ptr(y), rows, cols, n,
                                       _stream(stream)), "dnx_gemm_q4_f6p")


def gemm_q4_f6s_multi(packs, ys, rows, panel, cols: int, n: int, stream=None) -> None:
    """The chunk GEMM over 1..4 prepacked matrices reading one panel, in one
    launch (each output bit-identical to its own gemm_q4_f6s)."""
    import ctypes
    k = len(packs)
    if not (len(ys) == k == len(rows)):
        raise ValueError("gemm_q4_f6s_multi: one output and one row count per matrix")
    _need("gemm_q4_f6s_multi", panel=(panel, f6_panel_bytes(n, cols)))
    for j in range(k):
        _need("gemm_q4_f6s_multi", packed=(packs[j], q4_f6pack_bytes(rows[j], cols)),
              y=(ys[j], n * rows[j] * 4))
    pp = (ctypes.c_void_p * k)(*[_ptr(t) for t in packs])
    yp = (ctypes.c_void_p * k)(*[_ptr(t) for t in ys])
    rp = (ctypes.c_int64 * k)(*rows)
    _check(_lib.load().dnx_gemm_q4_f6s_multi(pp, yp, rp, k, _ptr(panel), cols, n,
                                             _stream(stream)), "dnx_gemm_q4_f6s_multi")


def gemm_q4_f6s(packed, panel, y, rows: int, cols: int, n: int, stream=None) -> None:
    """The prefill chunk GEMM (5..512 tokens) on prepacked Q4 weights."""
    _need("gemm_q4_f6s",
          packed=(packed, q4_f6pack_bytes(rows, cols)),
          panel=(panel, f6_panel_bytes(n, cols)),
          y=(y, n * rows * 4))
    _check(_lib.load().dnx_gemm_q4_f6s(_ptr(packed), _ptr(panel), _ptr(y), rows, cols, n,
                                       _stream(stream)), "dnx_gemm_q4_f6s")


def q8_f6pack_bytes(rows: int, cols: int) -> int:
    return int(_lib.load().dnx_q8_f6pack_bytes(rows, cols))


def pack_q8_f6(qs, scales, packed, rows: int, cols: int, stream=None) -> None:
    """Load-time re-encoding of Q8 weights for the fp6 GEMM (dnx_gemm_q8_f6p)."""
    _need("pack_q8_f6",
          qs=(qs, rows * cols),
          scales=(scales, rows * (cols // 32) * 4),
          packed=(packed, q8_f6pack_bytes(rows, cols)))
    _check(_lib.load().dnx_pack_q8_f6(_ptr(qs), _ptr(scales), _ptr(packed), rows, cols,
                                      _stream(stream)), "dnx_pack_q8_f6")


def gemm_q8_f6p(packed, panel, y, rows: int, cols: int, n: int, stream=None) -> None:
    _need("gemm_q8_f6p",
          packed=(packed, q8_f6pack_bytes(rows, cols)),
          panel=(panel, f6_panel_bytes(n, cols)),
          y=(y, n * rows * 4))
    _check(_lib.load().dnx_gemm_q8_f6p(_ptr(packed), _ptr(panel), _ptr(y), rows, cols, n,
                                       _stream(stream)), "dnx_gemm_q8_f6p")


def i8_panel_bytes(n: int, cols: int) -> int:
    return int(_lib.load().dnx_i8_panel_bytes(n, cols))


def quantize_q8_i8panel(x, panel, n: int, cols: int, stream=None) -> None:
    """fp32 x -> the int8 GEMM's activation panel (lab_quantize_q8's bits)."""
    _need("quantize_q8_i8panel", x=(x, n * cols * 4), panel=(panel, i8_panel_bytes(n, cols)))
    _check(_lib.load().dnx_quantize_q8_i8panel(_ptr(x), _ptr(panel), n, cols, _stream(stream)),
           "dnx_quantize_q8_i8panel")


def q8_i8pack_bytes(rows: int, cols: int) -> int:
    return int(_lib.load().dnx_q8_i8pack_bytes(rows, cols))


def pack_q8_i8(qs, scales, packed, rows: int, cols: int, stream=None) -> None:
    """Load-time re-encoding of Q8 weights for the int8 GEMM (dnx_gemm_q8_i8p)."""
    _need("pack_q8_i8",
          qs=(qs, rows * cols),
          scales=(scales, rows * (cols // 32) * 4),
          packed=(packed, q8_i8pack_bytes(rows, cols)))
    _check(_lib.load().dnx_pack_q8_i8(_ptr(qs), _ptr(scales), _ptr(packed), rows, cols,
                                      _stream(stream)), "dnx_pack_q8_i8")


def gemm_q8_i8p(packed, panel, y, rows: int, cols: int, n: int, stream=None) -> None:
    _need("gemm_q8_i8p",
          packed=(packed, q8_i8pack_bytes(rows, cols)),
          panel=(panel, i8_panel_bytes(n, cols)),
          y=(y, n * rows * 4))
    _check(_lib.load().dnx_gemm_q8_i8p(_ptr(packed), _ptr(panel), _ptr(y), rows, cols, n,
                                       _stream(stream)), "dnx_gemm_q8_i8p")


def gemm_q8_i8p_tile(rows: int, cols: int, n: int):
    """(weight rows, tokens) of the workgroup tile dnx_gemm_q8_i8p takes for
    a shape, or None for a shape it refuses."""
    import ctypes
    r, t = ctypes.c_int(0), ctypes.c_int(0)
    rc = _lib.load().dnx_gemm_q8_i8p_tile(rows, cols, n, ctypes.byref(r), ctypes.byref(t))
    return None if rc != 0 else (r.value, t.value)


def argmax_workspace(n: int, device="cuda") -> torch.Tensor:
    nbytes = int(_lib.load().dnx_argmax_workspace_bytes(n))
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def argmax(v: torch.Tensor, out: torch.Tensor, workspace: torch.Tensor, stream=None) -> None:
    _check(_lib.load().dnx_argmax(_ptr(v), v.numel(), _ptr(out), _ptr(workspace),
                                  _stream(stream)), "dnx_argmax")


def swiglu(g: torch.Tensor, u: torch.Tensor, stream=None) -> None:
    _check(_lib.load().dnx_swiglu(_ptr(g), _ptr(u), g.numel(), _stream(stream)), "dnx_swiglu")


def swiglu_f6panel(g, u, panel, rows: int, cols: int, stream=None) -> None:
    """swiglu in place, and the fp6 panel of the result."""
    _need("swiglu_f6panel", g=(g, rows * cols * 4), u=(u, rows * cols * 4),
          panel=(panel, f6_panel_bytes(rows, cols)))
    _check(_lib.load().dnx_swiglu_f6panel(_ptr(g), _ptr(u), _ptr(panel), rows, cols,
                                          _stream(stream)), "dnx_swiglu_f6panel")


def rms_norm_f6panel(x, w, out, panel, rows: int, cols: int, eps: float, stream=None) -> None:
    """rms_norm (no accumulate), and the fp6 panel of its output."""
    _need("rms_norm_f6panel", x=(x, rows * cols * 4), w=(w, cols * 4),
          out=(out, rows * cols * 4), panel=(panel, f6_panel_bytes(rows, cols)))
    _check(_lib.load().dnx_rms_norm_f6panel(_ptr(x), _ptr(w), _ptr(out), _ptr(panel), rows, cols,
                                            eps, _stream(stream)), "dnx_rms_norm_f6panel")


def add_rms_norm_f6panel(m, x, w, out, panel, rows: int, cols: int, eps: float,
                         stream=None) -> None:
    """add_rms_norm, and the fp6 panel of its output."""
    _need("add_rms_norm_f6panel", m=(m, rows * cols * 4), x=(x, rows * cols * 4),
          w=(w, cols * 4), out=(out, rows * cols * 4), panel=(panel, f6_panel_bytes(rows, cols)))
    _check(_lib.load().dnx_add_rms_norm_f6panel(_ptr(m), _ptr(x), _ptr(w), _ptr(out),
                                                _ptr(panel), rows, cols, eps, _stream(stream)),
           "dnx_add_rms_norm_f6panel")


def gelu(x: torch.Tensor, stream=None) -> None:
    _check(_lib.load().dnx_gelu(_ptr(x), x.numel(), _stream(stream)), "dnx_gelu")


# ---- the decoder's other layer steps (lab_gpu_enc_* semantics, fp32)

def rms_norm(x, w, out, rows: int, cols: int, eps: float, accumulate: bool = False,
             stream=None) -> None:
    _check(_lib.load().dnx_rms_norm(_ptr(x), _ptr(w), _ptr(out), rows, cols, eps,
                                    1 if accumulate else 0, _stream(stream)), "dnx_rms_norm")


def head_norm_rope(x, x_stride: int, w, rope, rope_stride: int, heads: int, hd: int, n: int,
                   eps: float, stream=None) -> None:
    _check(_lib.load().dnx_head_norm_rope(_ptr(x), x_stride, _ptr(w), _ptr(rope), rope_stride,
                                          heads, hd, n, eps, _stream(stream)),
           "dnx_head_norm_rope")


def head_norm_rope2(x0, x0_stride: int, w0, heads0: int, x1, x1_stride: int, w1, heads1: int,
                    rope, rope_stride: int, hd: int, n: int, eps: float, stream=None) -> None:
    _check(_lib.load().dnx_head_norm_rope2(_ptr(x0), x0_stride, _ptr(w0), heads0, _ptr(x1),
                                           x1_stride, _ptr(w1), heads1, _ptr(rope), rope_stride,
                                           hd, n, eps, _stream(stream)), "dnx_head_norm_rope2")


def add_rms_norm(m, x, w, out, rows: int, cols: int, eps: float, stream=None) -> None:
    _check(_lib.load().dnx_add_rms_norm(_ptr(m), _ptr(x), _ptr(w), _ptr(out), rows, cols, eps,
                                        _stream(stream)), "dnx_add_rms_norm")


def short_conv(bcx, weight, history, y, width: int, k: int, n: int, stream=None) -> None:
    _check(_lib.load().dnx_short_conv(_ptr(bcx), _ptr(weight), _ptr(history), _ptr(y), width, k,
                                      n, _stream(stream)), "dnx_short_conv")


def attention(q, keys, values, gate, out, position: int, n: int, heads: int, kv_heads: int,
              hd: int, window: int = 0, stream=None) -> None:
    _check(_lib.load().dnx_attention(_ptr(q), _ptr(keys), _ptr(values),
                                     None if gate is None else _ptr(gate), _ptr(out), position, n,
                                     heads, kv_heads, hd, window, _stream(stream)),
           "dnx_attention")


def attention_f6panel(q, keys, values, gate, out, panel, position: int, n: int, heads: int,
                      kv_heads: int, hd: int, window: int = 0, stream=None) -> int:
    """attention, and the fp6 panel of out; returns the status (DNX_EINVAL
    where the call does not take the split path whose combine writes it)."""
    _need("attention_f6panel", panel=(panel, f6_panel_bytes(n, heads * hd)))
    return int(_lib.load().dnx_attention_f6panel(
        _ptr(q), _ptr(keys), _ptr(values), None if gate is None else _ptr(gate), _ptr(out),
        _ptr(panel), position, n, heads, kv_heads, hd, window, _stream(stream)))


def attention_rope(q, keys, values, gate, out, position: int, heads: int, kv_heads: int, hd: int,
                   window: int, q_norm, k_norm, rope_row, eps: float, stream=None) -> None:
    """One decode token: head norm + RoPE of q and of keys[position], folded
    into the split-key attention (q and the key row are normed in place)."""
    _check(_lib.load().dnx_attention_rope(_ptr(q), _ptr(keys), _ptr(values),
                                          None if gate is None else _ptr(gate), _ptr(out),
                                          position, heads, kv_heads, hd, window, _ptr(q_norm),
                                          _ptr(k_norm), _ptr(rope_row), eps, _stream(stream)),
           "dnx_attention_rope")


def add(src, dst, count: int, stream=None) -> None:
    _check(_lib.load().dnx_add(_ptr(src), _ptr(dst), count, _stream(stream)), "dnx_add")


def copy(src, dst, count: int, stream=None) -> None:
    _check(_lib.load().dnx_copy(_ptr(src), _ptr(dst), count, _stream(stream)), "dnx_copy")


def steer(x, v, rows: int, cols: int, mode: int, scale: float, stream=None) -> None:
    _check(_lib.load().dnx_steer(_ptr(x), _ptr(v), rows, cols, mode, scale, _stream(stream)),
           "dnx_steer")


def matmul_workspace(cols: int, n: int, device="cuda") -> torch.Tensor:
    """Device workspace for dnx_matmul_q8 / _q4 at this shape."""
    nbytes = int(_lib.load().dnx_matmul_workspace_bytes(cols, n))
    if nbytes < 0:
        raise RuntimeError(f"dnx_matmul_workspace_bytes({cols}, {n}) refused the shape")
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)


def matmul_q8(qs, scales, x, y, rows: int, cols: int, n: int, int8_inputs: bool, workspace,
              stream=None) -> None:
    """The product route of lab_gpu_enc_matmul_q8 (dnx_matmul_q8)."""
    _check(_lib.load().dnx_matmul_q8(_ptr(qs), _ptr(scales), _ptr(x), _ptr(y), rows, cols, n,
                                     int(int8_inputs), _ptr(workspace), workspace.numel(),
                                     _stream(stream)), "dnx_matmul_q8")


def matmul_q4(qs, scales, x, y, rows: int, cols: int, n: int, int8_inputs: bool, workspace,
              stream=None) -> None:
    """The product route of lab_gpu_enc_matmul_q4 (dnx_matmul_q4)."""
    _check(_lib.load().dnx_matmul_q4(_ptr(qs), _ptr(scales), _ptr(x), _ptr(y), rows, cols, n,
                                     int(int8_inputs), _ptr(workspace), workspace.numel(),
                                     _stream(stream)), "dnx_matmul_q4")
