// Issue-bound microbenchmark of the prefill GEMM's inner step.
//
// One step of the fp6 GEMM (gemm_f6.hip) on one 32x32 tile and one Q4 block
// is: one v_mfma_f32_32x32x8_f16 (the outer product of the two block scales),
// one v_mfma_scale_f32_32x32x64_f8f6f4 (the exact block dot) and 16 VALU fmas
// (acc += dot * scale for the lane's 16 outputs). This kernel runs that step
// from registers only (no memory traffic, no LDS) so its time per step is the
// floor the real kernel cannot go below, and runs each part alone and with
// other VALU counts to show where the time goes.
//
// Also here: a read-only streaming kernel, the calibration of rocprofv3's
// FETCH_SIZE for kernels that only read (the decode GEMVs).
//
// Built into its own library (libdnx_ubench.so), not the product library.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));

constexpr int kTiles = 3;  // tiles per wave per block, as in the GEMM

// MF bit 0: the f16 scale MFMA; bit 1: the fp6 dot MFMA. NV VALU fmas per
// tile, each on its own accumulator (no dependency chains between them).
template <int NV, int MF>
__global__ void __launch_bounds__(512) tile_issue_kernel(int iters, float* out) {
  const int lane = threadIdx.x & 63;
  v8i a, b[kTiles];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    a[i] = (lane * 131 + i * 7) & 0x07070707;
#pragma unroll
    for (int t = 0; t < kTiles; t++) b[t][i] = (lane * 17 + i * 3 + t) & 0x07070707;
  }
  h4 as = {(_Float16)1.5f, (_Float16)0.001f, (_Float16)0.0f, (_Float16)0.0f};
  h4 bs[kTiles];
#pragma unroll
  for (int t = 0; t < kTiles; t++) {
    bs[t] = (h4){(_Float16)(t + 1), (_Float16)(t + 1), (_Float16)(t + 1), (_Float16)0};
  }
  v16f c;
#pragma unroll
  for (int i = 0; i < 16; i++) c[i] = (float)(lane - i);
  float acc[32], x[32], y[32];
#pragma unroll
  for (int i = 0; i < 32; i++) {
    acc[i] = 0.0f;
    x[i] = (float)(lane + i);
    y[i] = 1.0f + (float)i * 1e-7f;
  }
  v16f d[kTiles] = {}, s[kTiles] = {};
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int t = 0; t < kTiles; t++) {
      if (MF & 1) s[t] = __builtin_amdgcn_mfma_f32_32x32x8f16(as, bs[t], c, 0, 0, 0);
#pragma unroll
      for (int v = 0; v < NV / 2; v++) acc[v] = fmaf(x[v], y[v], acc[v]);
      if (MF & 2) {
        d[t] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b[t], c, 2, 2, 0, 130, 0, 133);
      }
#pragma unroll
      for (int v = NV / 2; v < NV; v++) acc[v] = fmaf(x[v], y[v], acc[v]);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, NV / 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, NV - NV / 2, 0);
      __builtin_amdgcn_sched_barrier(0);
      // The results are live: the MFMAs cannot be dropped.
      asm volatile("" ::"v"(d[t]), "v"(s[t]));
    }
    // Opaque operands: nothing is hoisted out of the loop.
    asm volatile("" : "+v"(x[0]), "+v"(a), "+v"(as));
  }
  float r = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; i++) r += acc[i];
#pragma unroll
  for (int t = 0; t < kTiles; t++) r += d[t][0] + s[t][1];
  out[blockIdx.x * blockDim.x + threadIdx.x] = r;
}

template <int NV, int MF>
void launch(int ctas, int threads, int iters, float* out) {
  hipLaunchKernelGGL((tile_issue_kernel<NV, MF>), dim3((unsigned)ctas), dim3((unsigned)threads), 0,
                     0, iters, out);
}

// Reads bytes (a multiple of 16 * 256 * 4) once, with the decode GEMV's
// weight load (buffer_load16_stream: 16 bytes per lane, streaming cache
// policy, a wave's lanes on one contiguous KiB), four loads in flight per
// lane; each lane folds what it read into one word so that no load can be
// dropped, and writes it to out. Its FETCH_SIZE per byte is the read-only
// calibration (a copy kernel's reads come with its writes' request mix).
constexpr int kReadThreads = 256;

__global__ void __launch_bounds__(kReadThreads)
stream_read_kernel(const uint8_t* src, int64_t bytes, uint32_t* out) {
  const dnx::i32x4 r = dnx::buffer_rsrc(src, (uint32_t)bytes);
  const int64_t step = (int64_t)gridDim.x * kReadThreads * 16;
  uint32_t h = 0;
  for (int64_t o = ((int64_t)blockIdx.x * kReadThreads + threadIdx.x) * 16; o < bytes;
       o += 4 * step) {
    uint4 v[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int64_t ou = o + u * step;
      v[u] = dnx::buffer_load16_stream(r, ou < bytes ? (int)ou : -16);
    }
#pragma unroll
    for (int u = 0; u < 4; u++) h ^= v[u].x + v[u].y + v[u].z + v[u].w;
  }
  out[(size_t)blockIdx.x * kReadThreads + threadIdx.x] = h;
}

}  // namespace

extern "C" {

// The streaming read above over `bytes` of src (below 2 GiB, a multiple of
// 16 KiB) with `ctas` workgroups of 256 threads; out holds ctas * 256 words.
// Returns 0, -1 for bad arguments, or the HIP error of the launch.
int dnx_ubench_stream_read(const void* src, int64_t bytes, int ctas, uint32_t* out,
                           void* stream) {
  if (bytes <= 0 || bytes >= (1ll << 31) || bytes % 16384 != 0 || ctas <= 0 ||
      ((uintptr_t)src & 15)) {
    return -1;
  }
  hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)ctas), dim3(kReadThreads), 0,
                     (hipStream_t)stream, (const uint8_t*)src, bytes, out);
  return (int)hipGetLastError();
}

// Runs ctas workgroups of `threads` threads (256: one wave per SIMD, 512:
// two), each wave doing iters x 3 steps with `mfma_mask` MFMAs and `nvalu`
// fmas per step, and returns the kernel time in *ms. out holds ctas*threads
// floats. Returns 0, -1 for an unsupported (nvalu, mfma_mask), or the HIP
// error code.
int dnx_ubench_tile_issue(int nvalu, int mfma_mask, int iters, int ctas, int threads, float* out,
                          float* ms) {
  if (threads != 256 && threads != 512) return -1;
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess) return -2;
  if (hipEventCreate(&e1) != hipSuccess) return -2;
  bool ok = false;
  (void)hipEventRecord(e0, 0);
#define DNX_UB(nn, m)                       \
  if (nvalu == nn && mfma_mask == m) {      \
    launch<nn, m>(ctas, threads, iters, out); \
    ok = true;                              \
  }
#define DNX_UB_ALL(m) DNX_UB(0, m) DNX_UB(8, m) DNX_UB(16, m) DNX_UB(24, m) DNX_UB(32, m)
  DNX_UB_ALL(0) DNX_UB_ALL(1) DNX_UB_ALL(2) DNX_UB_ALL(3)
#undef DNX_UB_ALL
#undef DNX_UB
  (void)hipEventRecord(e1, 0);
  int rc = (int)hipEventSynchronize(e1);
  if (rc == 0) rc = (int)hipGetLastError();
  (void)hipEventElapsedTime(ms, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (!ok) return -1;
  return rc;
}

}  // extern "C"
