"""Builds libdianoia_amd.so (gfx950 HIP kernels + the lab_gpu_* C ABI) in-tree.

Run as ``python -m dianoia_amd.build``; ``__graft_entry__.build()`` calls
:func:`build`. The three translation units compile in parallel and link into
one shared library next to this file, so it travels with the source tree.
"""

from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(HERE, "libdianoia_amd.so")
# The issue-bound microbenchmark of the GEMM step, kept out of the product
# library (bench.py --issue-bound loads it).
UBENCH_SRC = "ubench_tile.hip"
UBENCH_LIB = os.path.join(HERE, "libdnx_ubench.so")
SOURCES = ["kernels.hip", "gemv.hip", "gemm.hip", "gemm_f16.hip", "gemm_f6.hip", "gemm_float.hip",
           "layers.hip", "matmul.hip", "lab_gpu.hip"]
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -ffp-contract=off: only explicit fmaf() fuses (the reference's float order).
# -packed-fp32-ops disabled: no v_pk_*_f32 in the device code.
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", INCLUDE, "-I", CSRC,
]


# Per-source flags. The GEMM keeps its MFMA results in ordinary VGPRs: its
# scale epilogue reads every result with VALU instructions, which cannot
# take accumulation registers (one v_accvgpr_read per value otherwise).
SOURCE_FLAGS = {src: ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]
                for src in ("gemm.hip", "gemm_f16.hip", "gemm_f6.hip", "gemm_float.hip", UBENCH_SRC)}


def _compile(src: str, build_dir: str) -> str:
    obj = os.path.join(build_dir, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, *SOURCE_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    return obj


def _link(objs: list, lib: str) -> None:
    tmp = lib + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, lib)


def build(verbose: bool = False) -> str:
    build_dir = os.path.join(HERE, "_build")
    os.makedirs(build_dir, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(len(SOURCES) + 1) as pool:
        objs = list(pool.map(lambda s: _compile(s, build_dir), SOURCES + [UBENCH_SRC]))
    ubench_obj = objs.pop()
    _link([ubench_obj], UBENCH_LIB)
    _link(objs, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
