"""The drop-in boundary on the CPU: the library builds, loads, and exports
every symbol include/*.h declares. No compute call (no GPU here)."""

import ctypes
import os
import subprocess

from dianoia_amd import _lib

# The reference's GPU entry points that Dart binds (lib/src/gpu.dart:36-312):
# the matmul path, everything GpuLinear and the GPU layer's lifecycle,
# profiling and tuning calls reach, and the decoder's other layer steps.
REFERENCE_BOUND = [
    "lab_gpu_init", "lab_gpu_max_buffer_length", "lab_gpu_max_shared_memory",
    "lab_gpu_recommended_working_set", "lab_gpu_thermal_state", "lab_gpu_physical_memory",
    "lab_gpu_device_name", "lab_gpu_buffer", "lab_gpu_readback_buffer", "lab_gpu_wrap",
    "lab_gpu_wrap_copies", "lab_gpu_contents", "lab_gpu_release", "lab_gpu_live_buffers",
    "lab_gpu_set_decode_rows", "lab_gpu_set_q8_group", "lab_gpu_set_q8_vector",
    "lab_gpu_register_q8_head", "lab_gpu_set_profiling", "lab_gpu_profile", "lab_gpu_last_ms",
    "lab_gpu_begin", "lab_gpu_commit", "lab_gpu_wait", "lab_gpu_enc_matmul_q8",
    "lab_gpu_enc_matmul_q4", "lab_gpu_enc_swiglu", "lab_gpu_enc_rms_norm",
    "lab_gpu_enc_head_norm_rope", "lab_gpu_enc_conv", "lab_gpu_enc_attention", "lab_gpu_enc_copy",
    "lab_gpu_enc_add", "lab_gpu_enc_steer",
]


def test_library_is_built():
    assert os.path.exists(_lib.LIB_PATH), "run python -m dianoia_amd.build"


def test_exports_every_declared_symbol():
    declared = _lib.declared_symbols()
    assert len(declared) >= 40
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [s for s in declared if s not in exported]
    assert not missing, missing
    assert set(declared) == set(_lib.SIGNATURES), "ctypes signatures out of sync with headers"


def test_reference_gpu_abi_covered():
    declared = set(_lib.declared_symbols())
    assert [s for s in REFERENCE_BOUND if s not in declared] == []


def test_loads_with_ctypes():
    lib = _lib.load()
    for name in _lib.SIGNATURES:
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr)


def test_no_oracle_in_product():
    # The product library must not link the CPU oracle or the reference.
    out = subprocess.run(["ldd", _lib.LIB_PATH], capture_output=True, text=True).stdout
    assert "lab_oracle" not in out and "lab_native" not in out
    syms = subprocess.run(["nm", "-D", _lib.LIB_PATH], capture_output=True, text=True).stdout
    assert "orc_" not in syms
