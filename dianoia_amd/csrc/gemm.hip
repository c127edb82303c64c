// Prefill / vision-encoder GEMM on gfx950 int8 MFMA with per-32-block
// scales: y[m][r] = sum_b sx[m][b] * sw[r][b] * D_b[m][r], where
// D_b = sum over block b of xq[m][k] * w[r][k] is an exact int32 from one
// v_mfma_i32_32x32x32_i8 (its K of 32 is exactly one Q block). The scale
// epilogue is fp32: cvt, s = sx * sw (rounded, as the CPU's s,
// lab_native.c:509), fma into the accumulator, block after block. The CPU
// keeps four partial lanes per block (lab_native.c:480-512); one lane per
// output here gives a different rounding, within 1e-4 relative.
//
// Workgroup tile: BM tokens x BN weight rows, 4 waves in a 2 x 2 grid, each
// wave a (BM/2) x (BN/2) tile of 32 x 32 MFMA subtiles. K is staged KB
// blocks at a time in LDS (double buffered): activations as int8, weights
// unpacked to int8 (Q4 nibbles -> q - 8 once per stage, shared by all BM
// tokens), scales as fp32.

#include "common.h"
#include "dnx_kernels.h"

using namespace dnx;

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int KB = 2;             // blocks per LDS stage
constexpr int kRowBytes = KB * 32;
constexpr int kRowStride = kRowBytes + 16;  // LDS row stride (bank spread)

struct GemmParams {
  const void* qs;
  const void* scales;
  const int8_t* xq;
  const float* xsc;
  float* y;
  int rows, cols, n;
};

// Q4 byte-dword of 4 nibble pairs -> two dwords of int8 weights q - 8:
// low nibbles (weights k) and high nibbles (weights k + 16).
DNX_DEV void unpack_q4(uint32_t v, uint32_t& lo, uint32_t& hi) {
  const uint32_t m = 0x0f0f0f0fu;
  // (q | 0x80) - 8 never borrows across bytes; ^ 0x80 gives q - 8 as int8.
  lo = (((v & m) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
  hi = ((((v >> 4) & m) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
}

template <bool kQ4, int BM, int BN>
__global__ void __launch_bounds__(kThreads) gemm_kernel(GemmParams p) {
  constexpr int WM = BM / 2, WN = BN / 2;      // wave tile
  constexpr int SM = WM / 32, SN = WN / 32;    // 32x32 subtiles per wave
  __shared__ __align__(16) int8_t sa[2][BM * kRowStride];
  __shared__ __align__(16) int8_t sb[2][BN * kRowStride];
  __shared__ __align__(16) float sxs[2][KB][BM];
  __shared__ __align__(16) float sws[2][KB][BN];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int K = p.cols, B = K / kBlock, M = p.n, N = p.rows;
  const int stages = (B + KB - 1) / KB;

  // Global -> register staging of one stage. A: BM rows x 64 B -> 16 B per
  // thread per pass. B: Q8 the same; Q4 BN rows x 32 B of nibbles.
  constexpr int APASS = BM * kRowBytes / 16 / kThreads;  // b128 loads per thread
  constexpr int BPASS = BN * (kQ4 ? kRowBytes / 2 : kRowBytes) / 16 / kThreads;
  static_assert(APASS >= 1 && BPASS >= 1, "tile too small for the staging");
  uint4 ra[APASS], rb[BPASS];
  float rsx, rsw;

  auto load_stage = [&](int s) {
    const int b0 = s * KB;
#pragma unroll
    for (int i = 0; i < APASS; i++) {
      const int idx = i * kThreads + tid;
      const int row = idx / (kRowBytes / 16), seg = idx % (kRowBytes / 16);
      const int m = m0 + row, blk = b0 + seg / 2;
      ra[i] = make_uint4(0, 0, 0, 0);
      if (m < M && blk < B) ra[i] = *(const uint4*)(p.xq + (size_t)m * K + b0 * 32 + seg * 16);
    }
#pragma unroll
    for (int i = 0; i < BPASS; i++) {
      const int idx = i * kThreads + tid;
      if (kQ4) {
        const int row = idx / KB, blk = b0 + idx % KB;
        const int r = n0 + row;
        rb[i] = make_uint4(0, 0, 0, 0);
        if (r < N && blk < B)
          rb[i] = *(const uint4*)((const uint8_t*)p.qs + (size_t)r * (K / 2) + (size_t)blk * 16);
      } else {
        const int row = idx / (kRowBytes / 16), seg = idx % (kRowBytes / 16);
        const int r = n0 + row, blk = b0 + seg / 2;
        rb[i] = make_uint4(0, 0, 0, 0);
        if (r < N && blk < B)
          rb[i] = *(const uint4*)((const int8_t*)p.qs + (size_t)r * K + b0 * 32 + seg * 16);
      }
    }
    // Scales: thread t < KB*BM loads sx, thread t < KB*BN loads sw.
    rsx = 0.0f;
    rsw = 0.0f;
    if (tid < KB * BM) {
      const int kb = tid / BM, m = m0 + tid % BM, blk = b0 + kb;
      if (m < M && blk < B) rsx = p.xsc[(size_t)m * B + blk];
    }
    if (tid < KB * BN) {
      const int kb = tid / BN, r = n0 + tid % BN, blk = b0 + kb;
      if (r < N && blk < B) {
        rsw = kQ4 ? half_bits_to_float(((const uint16_t*)p.scales)[(size_t)r * B + blk])
                  : ((const float*)p.scales)[(size_t)r * B + blk];
      }
    }
  };

  auto store_stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < APASS; i++) {
      const int idx = i * kThreads + tid;
      const int row = idx / (kRowBytes / 16), seg = idx % (kRowBytes / 16);
      *(uint4*)(&sa[buf][row * kRowStride + seg * 16]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < BPASS; i++) {
      const int idx = i * kThreads + tid;
      if (kQ4) {
        const int row = idx / KB, kb = idx % KB;
        uint4 lo, hi;
        unpack_q4(rb[i].x, lo.x, hi.x);
        unpack_q4(rb[i].y, lo.y, hi.y);
        unpack_q4(rb[i].z, lo.z, hi.z);
        unpack_q4(rb[i].w, lo.w, hi.w);
        int8_t* dst = &sb[buf][row * kRowStride + kb * 32];
        *(uint4*)dst = lo;
        *(uint4*)(dst + 16) = hi;
      } else {
        const int row = idx / (kRowBytes / 16), seg = idx % (kRowBytes / 16);
        *(uint4*)(&sb[buf][row * kRowStride + seg * 16]) = rb[i];
      }
    }
    if (tid < KB * BM) sxs[buf][tid / BM][tid % BM] = rsx;
    if (tid < KB * BN) sws[buf][tid / BN][tid % BN] = rsw;
  };

  float acc[SM][SN][16];
#pragma unroll
  for (int i = 0; i < SM; i++)
#pragma unroll
    for (int j = 0; j < SN; j++)
#pragma unroll
      for (int v = 0; v < 16; v++) acc[i][j][v] = 0.0f;

  load_stage(0);
  store_stage(0);
  __syncthreads();

  const int lrow = lane & 31, lk = (lane >> 5) * 16;
  for (int s = 0; s < stages; s++) {
    const int buf = s & 1;
    if (s + 1 < stages) load_stage(s + 1);
#pragma unroll
    for (int kb = 0; kb < KB; kb++) {
      if (s * KB + kb >= B) break;
      v4i a[SM], b[SN];
#pragma unroll
      for (int i = 0; i < SM; i++)
        a[i] = *(const v4i*)(&sa[buf][(wm * WM + i * 32 + lrow) * kRowStride + kb * 32 + lk]);
#pragma unroll
      for (int j = 0; j < SN; j++)
        b[j] = *(const v4i*)(&sb[buf][(wn * WN + j * 32 + lrow) * kRowStride + kb * 32 + lk]);
      // Scales of this lane's outputs: column n = lane % 32 of each N
      // subtile; rows (v / 4) * 8 + (lane / 32) * 4 + v % 4 of each M subtile.
      float swv[SN];
#pragma unroll
      for (int j = 0; j < SN; j++) swv[j] = sws[buf][kb][wn * WN + j * 32 + lrow];
#pragma unroll
      for (int i = 0; i < SM; i++) {
        float sxv[16];
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const float4 t = *(const float4*)(&sxs[buf][kb][wm * WM + i * 32 + g * 8 + (lane >> 5) * 4]);
          sxv[4 * g + 0] = t.x;
          sxv[4 * g + 1] = t.y;
          sxv[4 * g + 2] = t.z;
          sxv[4 * g + 3] = t.w;
        }
#pragma unroll
        for (int j = 0; j < SN; j++) {
          v16i d = {};
          d = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], d, 0, 0, 0);
#pragma unroll
          for (int v = 0; v < 16; v++) acc[i][j][v] = fmaf((float)d[v], sxv[v] * swv[j], acc[i][j][v]);
        }
      }
    }
    if (s + 1 < stages) store_stage(buf ^ 1);
    __syncthreads();
  }

  // Store: lane holds column n0 + wn*WN + j*32 + lane%32 for 16 rows.
#pragma unroll
  for (int i = 0; i < SM; i++)
#pragma unroll
    for (int j = 0; j < SN; j++) {
      const int r = n0 + wn * WN + j * 32 + lrow;
      if (r >= N) continue;
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int m = m0 + wm * WM + i * 32 + (v / 4) * 8 + (lane >> 5) * 4 + (v % 4);
        if (m < M) p.y[(size_t)m * N + r] = acc[i][j][v];
      }
    }
}

template <bool kQ4>
int launch_gemm(const void* qs, const void* scales, const int8_t* xq, const float* xsc,
                float* y, int64_t rows, int64_t cols, int64_t n, hipStream_t stream) {
  if (rows <= 0 || cols <= 0 || n <= 0 || cols % kBlock != 0) return DNX_EINVAL;
  if (rows > INT32_MAX || n > INT32_MAX || cols > INT32_MAX / 2) return DNX_EINVAL;
  if (((uintptr_t)qs & 15) || ((uintptr_t)xq & 15)) return DNX_EINVAL;
  GemmParams p{qs, scales, xq, xsc, y, (int)rows, (int)cols, (int)n};
  constexpr int BM = 128, BN = 128;
  const dim3 grid((unsigned)((rows + BN - 1) / BN), (unsigned)((n + BM - 1) / BM));
  hipLaunchKernelGGL((gemm_kernel<kQ4, BM, BN>), grid, dim3(kThreads), 0, stream, p);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

}  // namespace

extern "C" {

int dnx_gemm_q8(const int8_t* qs, const float* scales, const int8_t* xq, const float* xsc,
                float* y, int64_t rows, int64_t cols, int64_t n, hipStream_t stream) {
  return launch_gemm<false>(qs, scales, xq, xsc, y, rows, cols, n, stream);
}

int dnx_gemm_q4(const uint8_t* qs, const uint16_t* scales, const int8_t* xq, const float* xsc,
                float* y, int64_t rows, int64_t cols, int64_t n, hipStream_t stream) {
  return launch_gemm<true>(qs, scales, xq, xsc, y, rows, cols, n, stream);
}

}  // extern "C"
