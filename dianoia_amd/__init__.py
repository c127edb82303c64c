"""MI355X-native (gfx950, HIP) quantized linear layer for dianoia.

The product is ``libdianoia_amd.so``: hand-written HIP kernels behind the
reference's ``lab_gpu_*`` C ABI (include/lab_gpu.h) plus device-pointer
launchers (include/dnx_kernels.h). This package loads it with ctypes
(``_lib``), mirrors the reference's ``GpuLinear`` over it (``gpu``), holds
the host-side weight formats (``formats``) and wraps the launchers for
torch device tensors (``device``).
"""

from .errors import ArgumentError, StateError
from .formats import QuantMatrix, split_q4_0, split_q8_0, widen_bf16

__all__ = ["ArgumentError", "StateError", "QuantMatrix", "split_q4_0", "split_q8_0",
           "widen_bf16"]
