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
// Built into its own library (libdnx_ubench.so), not the product library.
#include <hip/hip_runtime.h>
#include <stdint.h>

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

}  // namespace

extern "C" {

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
