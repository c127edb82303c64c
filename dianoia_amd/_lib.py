"""Loads libdianoia_amd.so (built in-tree by dianoia_amd/build.py) with ctypes.

The library is the product: there is no fallback. If it is missing, every
entry point raises instead of computing anything on the CPU.
"""

from __future__ import annotations

import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "libdianoia_amd.so")
HEADERS = [os.path.join(ROOT, "include", h) for h in ("lab_gpu.h", "dnx_kernels.h")]

_i64 = ctypes.c_int64
_p = ctypes.c_void_p
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_f64 = ctypes.c_double

# argtypes / restype of every exported entry point (include/*.h).
SIGNATURES = {
    "lab_gpu_init": ([], _i64),
    "lab_gpu_buffer": ([_i64], _i64),
    "lab_gpu_readback_buffer": ([_i64], _i64),
    "lab_gpu_wrap": ([_p, _i64], _i64),
    "lab_gpu_wrap_copies": ([], _i64),
    "lab_gpu_contents": ([_i64], _p),
    "lab_gpu_release": ([_i64], None),
    "lab_gpu_live_buffers": ([], _i64),
    "lab_gpu_begin": ([], None),
    "lab_gpu_commit": ([_i64], _i64),
    "lab_gpu_wait": ([], _i64),
    "lab_gpu_last_ms": ([], ctypes.c_double),
    "lab_gpu_transfer_bytes": ([_p, _p], None),
    "lab_gpu_tracking_writes": ([], _i64),
    "lab_gpu_enc_matmul_q8": ([_i64] * 10, None),
    "lab_gpu_enc_matmul_q4": ([_i64] * 10, None),
    "lab_gpu_enc_swiglu": ([_i64] * 3, None),
    "lab_gpu_enc_rms_norm": ([_i64] * 8 + [_f64, _i64], None),
    "lab_gpu_enc_head_norm_rope": ([_i64] * 11 + [_f64], None),
    "lab_gpu_enc_conv": ([_i64] * 8, None),
    "lab_gpu_enc_attention": ([_i64] * 11, None),
    "lab_gpu_enc_copy": ([_i64] * 5, None),
    "lab_gpu_enc_add": ([_i64] * 5, None),
    "lab_gpu_enc_steer": ([_i64] * 7 + [_f64], None),
    "lab_gpu_enc_quantize_q8": ([_i64] * 9, None),
    "lab_gpu_enc_quantize_q8_bf16": ([_i64] * 9, None),
    "lab_gpu_enc_quantize_q4": ([_i64] * 8, None),
    "lab_gpu_enc_quantize_q4_bf16": ([_i64] * 8, None),
    "lab_gpu_enc_q6k_to_q8": ([_i64] * 8, None),
    "lab_gpu_enc_split_q8_0": ([_i64] * 8, None),
    "lab_gpu_enc_split_q4_0": ([_i64] * 8, None),
    "lab_gpu_enc_argmax": ([_i64] * 5, None),
    "lab_gpu_enc_gelu": ([_i64] * 3, None),
    "lab_gpu_set_profiling": ([_i64], None),
    "lab_gpu_set_int8_inputs": ([_i64], _i64),
    "lab_gpu_profile": ([_p, _p, _i64], _i64),
    "lab_gpu_set_decode_rows": ([_i64], None),
    "lab_gpu_set_q8_group": ([_i64], _i64),
    "lab_gpu_set_q8_vector": ([_i64], _i64),
    "lab_gpu_register_q8_head": ([_i64] * 5, _i64),
    "lab_gpu_device_name": ([_p, _i64], None),
    "lab_gpu_max_buffer_length": ([], _i64),
    "lab_gpu_max_shared_memory": ([], _i64),
    "lab_gpu_recommended_working_set": ([], _i64),
    "lab_gpu_thermal_state": ([], _i64),
    "lab_gpu_physical_memory": ([], _i64),
    "dnx_quantize_q8": ([_p, _p, _p, _i64, _i64, _i64, _p], _i32),
    "dnx_quantize_q8_bf16": ([_p, _p, _p, _i64, _i64, _i64, _p], _i32),
    "dnx_quantize_q4": ([_p, _p, _p, _i64, _i64, _p], _i32),
    "dnx_q6k_to_q8": ([_p, _p, _p, _i64, _i64, _p], _i32),
    "dnx_split_q8_0": ([_p, _p, _p, _i64, _p], _i32),
    "dnx_split_q4_0": ([_p, _p, _p, _i64, _p], _i32),
    "dnx_quantize_q4_bf16": ([_p, _p, _p, _i64, _i64, _p], _i32),
    "dnx_gemv_q8": ([_p, _p, _p, _p, _i64, _i64, _i64, _p], _i32),
    "dnx_gemv_q4": ([_p, _p, _p, _p, _i64, _i64, _i64, _p], _i32),
    "dnx_gemv_argmax_workspace_bytes": ([], _i64),
    "dnx_gemv_q8_argmax": ([_p, _p, _p, _p, _i64, _i64, _p, _p, _p], _i32),
    "dnx_gemv_q4_argmax": ([_p, _p, _p, _p, _i64, _i64, _p, _p, _p], _i32),
    "dnx_gate_up_q8": ([_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p], _i32),
    "dnx_gate_up_q4": ([_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p], _i32),
    "dnx_gemv_q8_float": ([_p, _p, _p, _p, _i64, _i64, _i64, _p], _i32),
    "dnx_gemv_q4_float": ([_p, _p, _p, _p, _i64, _i64, _i64, _p], _i32),
    "dnx_gemv_q8h": ([_p, _p, _p, _p, _i64, _i64, _i64, _p], _i32),
    "dnx_gemv_q8h_argmax": ([_p, _p, _p, _p, _i64, _i64, _p, _p, _p], _i32),
    "dnx_gate_up_q8h": ([_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p], _i32),
    "dnx_gemv_multi_q8": ([_p, _p, _p, _p, _i32, _p, _i64, _p], _i32),
    "dnx_copy_regions": ([_p, _p, _p, _i32, _p], _i32),
    "dnx_gemv_multi_q4": ([_p, _p, _p, _p, _i32, _p, _i64, _p], _i32),
    "dnx_gemv_multi_q8h": ([_p, _p, _p, _p, _i32, _p, _i64, _p], _i32),
    "dnx_gemv_add_q8": ([_p, _p, _p, _p, _p, _i64, _i64, _p], _i32),
    "dnx_gemv_add_q4": ([_p, _p, _p, _p, _p, _i64, _i64, _p], _i32),
    "dnx_gate_up_norm_q8": ([_p, _p, _p, _p, _p, _p, _p, _f32, _p, _p, _i64, _i64, _p], _i32),
    "dnx_gate_up_norm_q4": ([_p, _p, _p, _p, _p, _p, _p, _f32, _p, _p, _i64, _i64, _p], _i32),
    "dnx_gemv_multi_norm_q8": ([_p, _p, _p, _p, _i32, _p, _p, _p, _f32, _i64, _p], _i32),
    "dnx_gemv_multi_norm_q4": ([_p, _p, _p, _p, _i32, _p, _p, _p, _f32, _i64, _p], _i32),
    "dnx_gemm_q8": ([_p, _p, _p, _p, _p, _i64, _i64, _i64, _p], _i32),
    "dnx_gemm_q8_float": ([_p, _p, _p, _p, _i64, _i64, _i64, _p], _i32),
    "dnx_gemm_q4_float": ([_p, _p, _p, _p, _i64, _i64, _i64, _p], _i32),
    "dnx_gemm_q4": ([_p, _p, _p, _p, _p, _i64, _i64, _i64, _p], _i32),
    "dnx_gemm_panel_bytes": ([_i64, _i64], _i64),
    "dnx_pack_panel": ([_p, _p, _p, _i64, _i64, _p], _i32),
    "dnx_quantize_q8_panel": ([_p, _p, _i64, _i64, _p], _i32),
    "dnx_gemm_q8_panel": ([_p, _p, _p, _p, _i64, _i64, _i64, _p], _i32),
    "dnx_gemm_q4_panel": ([_p, _p, _p, _p, _i64, _i64, _i64, _p], _i32),
    "dnx_f6_panel_bytes": ([_i64, _i64], _i64),
    "dnx_quantize_q8_f6panel": ([_p, _p, _i64, _i64, _p], _i32),
    "dnx_pack_f6panel": ([_p, _p, _p, _i64, _i64, _p], _i32),
    "dnx_gemm_q4_f6": ([_p, _p, _p, _p, _i64, _i64, _i64, _p], _i32),
    "dnx_q4_f6pack_bytes": ([_i64, _i64], _i64),
    "dnx_pack_q4_f6": ([_p, _p, _p, _i64, _i64, _p], _i32),
    "dnx_gemm_q4_f6p": ([_p, _p, _p, _i64, _i64, _i64, _p], _i32),
    "dnx_gemm_q4_f6s": ([_p, _p, _p, _i64, _i64, _i64, _p], _i32),
    "dnx_gemm_q4_f6s_multi": ([_p, _p, _p, _i32, _p, _i64, _i64, _p], _i32),
    "dnx_swiglu_f6panel": ([_p, _p, _p, _i64, _i64, _p], _i32),
    "dnx_rms_norm_f6panel": ([_p, _p, _p, _p, _i64, _i64, _f32, _p], _i32),
    "dnx_add_rms_norm_f6panel": ([_p, _p, _p, _p, _p, _i64, _i64, _f32, _p], _i32),
    "dnx_q8_f6pack_bytes": ([_i64, _i64], _i64),
    "dnx_pack_q8_f6": ([_p, _p, _p, _i64, _i64, _p], _i32),
    "dnx_gemm_q8_f6p": ([_p, _p, _p, _i64, _i64, _i64, _p], _i32),
    "dnx_i8_panel_bytes": ([_i64, _i64], _i64),
    "dnx_quantize_q8_i8panel": ([_p, _p, _i64, _i64, _p], _i32),
    "dnx_q8_i8pack_bytes": ([_i64, _i64], _i64),
    "dnx_pack_q8_i8": ([_p, _p, _p, _i64, _i64, _p], _i32),
    "dnx_gemm_q8_i8p": ([_p, _p, _p, _i64, _i64, _i64, _p], _i32),
    "dnx_gemm_q8_i8p_tile": ([_i64, _i64, _i64, _p, _p], _i32),
    "dnx_gemm_q4_f6p_noalloc_max_floats": ([], _i64),
    "dnx_matmul_workspace_bytes": ([_i64, _i64], _i64),
    "dnx_matmul_q8": ([_p, _p, _p, _p, _i64, _i64, _i64, _i32, _p, _i64, _p], _i32),
    "dnx_matmul_q4": ([_p, _p, _p, _p, _i64, _i64, _i64, _i32, _p, _i64, _p], _i32),
    "dnx_gemm_q4_f6p_noalloc": ([_p, _p, _p, _i64, _i64, _i64, _p], _i32),
    "dnx_argmax_workspace_bytes": ([_i64], _i64),
    "dnx_argmax": ([_p, _i64, _p, _p, _p], _i32),
    "dnx_swiglu": ([_p, _p, _i64, _p], _i32),
    "dnx_gelu": ([_p, _i64, _p], _i32),
    "dnx_rms_norm": ([_p, _p, _p, _i64, _i64, _f32, _i32, _p], _i32),
    "dnx_head_norm_rope": ([_p, _i64, _p, _p, _i64, _i64, _i64, _i64, _f32, _p], _i32),
    "dnx_head_norm_rope2": ([_p, _i64, _p, _i64, _p, _i64, _p, _i64, _p, _i64, _i64, _i64, _f32, _p], _i32),
    "dnx_add_rms_norm": ([_p, _p, _p, _p, _i64, _i64, _f32, _p], _i32),
    "dnx_short_conv": ([_p, _p, _p, _p, _i64, _i64, _i64, _p], _i32),
    "dnx_attention_max_keys": ([_i64], _i64),
    "dnx_attention": ([_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p], _i32),
    "dnx_attention_f6panel": ([_p] * 6 + [_i64] * 6 + [_p], _i32),
    "dnx_attention_rope": ([_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _f32, _p], _i32),
    "dnx_add": ([_p, _p, _i64, _p], _i32),
    "dnx_copy": ([_p, _p, _i64, _p], _i32),
    "dnx_steer": ([_p, _p, _i64, _i64, _i64, _f32, _p], _i32),
}


class LibraryMissing(RuntimeError):
    pass


_lib = None


def declared_symbols() -> list[str]:
    """Every function name the C headers in include/ declare."""
    names = []
    for path in HEADERS:
        text = open(path).read()
        text = re.sub(r"//[^\n]*", "", text)
        for m in re.finditer(r"\b(lab_gpu_\w+|dnx_\w+)\s*\(", text):
            names.append(m.group(1))
    return sorted(set(names))


def load() -> ctypes.CDLL:
    """The product library, with every signature set. Raises if not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise LibraryMissing(
            f"{LIB_PATH} is not built; run `python -m dianoia_amd.build` (there is no CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
    for name, (args, res) in SIGNATURES.items():
        f = getattr(lib, name)
        f.argtypes = args
        f.restype = res
    _lib = lib
    return lib
