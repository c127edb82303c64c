// gfx950 kernels of the quantized linear layer: Q8 activation/weight
// quantizers, the exact-order Q8/Q4 decode GEMV with the activation
// quantizer fused into its prologue, greedy argmax, and the glue between
// linears. The int8-MFMA GEMM lives in gemm.hip.
//
// Built with -ffp-contract=off: every multiply-add that the reference fuses
// is an explicit fmaf here, and every one it keeps apart stays apart.

#include "common.h"
#include "dnx_kernels.h"

#include <math.h>

using namespace dnx;

namespace {

constexpr int kThreads = 256;  // 4 waves per workgroup

// ------------------------------------------------------------ quantizer

// lab_quantize_q8 over rows x cols values into rows x cols_pad int8 and
// rows x cols_pad/32 fp32 scales (lab_native.c:407-429). cols_pad is a
// multiple of 32 and >= cols; values at cols..cols_pad are zero padding.
// One thread quantizes 4 consecutive values; 8 threads share a block.
// Input is fp32 or bf16 (widened p << 16, safetensors.dart:207-212).
template <bool kBf16>
__global__ void __launch_bounds__(kThreads)
quantize_q8_kernel(const void* __restrict__ src, int8_t* __restrict__ qs,
                   float* __restrict__ scales, int64_t rows, int64_t cols, int64_t cols_pad,
                   int vec_ok) {
  const int64_t quads_per_row = cols_pad / 4;
  const int64_t total = rows * quads_per_row;
  // Whole 8-lane groups stay together: quads_per_row is a multiple of 8.
  for (int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x; q < total;
       q += (int64_t)gridDim.x * kThreads) {
    const int64_t row = q / quads_per_row;
    const int64_t c = (q - row * quads_per_row) * 4;
    float4 v;
    if (kBf16) {
      const uint16_t* p = (const uint16_t*)src + row * cols + c;
      if (vec_ok && c + 4 <= cols) {
        const uint2 raw = *(const uint2*)p;
        v = make_float4(__uint_as_float(raw.x << 16), __uint_as_float(raw.x & 0xffff0000u),
                        __uint_as_float(raw.y << 16), __uint_as_float(raw.y & 0xffff0000u));
      } else {
        v.x = c + 0 < cols ? bf16_to_float(p[0]) : 0.0f;
        v.y = c + 1 < cols ? bf16_to_float(p[1]) : 0.0f;
        v.z = c + 2 < cols ? bf16_to_float(p[2]) : 0.0f;
        v.w = c + 3 < cols ? bf16_to_float(p[3]) : 0.0f;
      }
    } else {
      const float* p = (const float*)src + row * cols + c;
      if (vec_ok && c + 4 <= cols) {
        v = *(const float4*)p;
      } else {
        v.x = c + 0 < cols ? p[0] : 0.0f;
        v.y = c + 1 < cols ? p[1] : 0.0f;
        v.z = c + 2 < cols ? p[2] : 0.0f;
        v.w = c + 3 < cols ? p[3] : 0.0f;
      }
    }
    const float amax = group8_max(fmaxf(0.0f, max4abs(v)));
    const float scale = q8_scale(amax);
    const float inv = q8_inv(scale);
    *(int*)(qs + row * cols_pad + c) = quant4(v, inv);
    if ((c & 31) == 0) scales[row * (cols_pad / 32) + c / 32] = scale;
  }
}

// ------------------------------------------------------------ GEMV

// Decode products y[t][r] = (W x[t])[r] for n <= NT tokens, weights in the
// engine's Q8 (int8 + fp32 scale) or Q4 (nibbles + fp16 scale) layout,
// computing every (row, token) in the reference CPU kernel's exact float
// order (dot_q8_sdot lab_native.c:503-512, dot_q4_sdot :1025-1034): per
// block, four exact int32 lane sums d_l over bytes {4l..4l+3, 16+4l..19+4l};
// s = sw * sx rounded; acc_l = fma(float(d_l), s, acc_l) block after block;
// y = (acc0 + acc1) + (acc2 + acc3). The outputs are therefore bit-identical
// to lab_gemm_q8 / lab_gemm_q4 mode 1, argmax included.
//
// A workgroup owns R rows. Its prologue quantizes the n input rows into LDS
// (the fused activation quantizer, lab_native.c:556). Then, per chunk of
// blocks, all four waves stream the R rows with 16-byte coalesced loads (a
// wave instruction reads 1 KB of one row) and turn them into per-lane int32
// sums, written to LDS as floats (exact: |d| < 2^24) together with the
// per-block scales s. Finally lanes (t, r, l) run the short sequential FMA
// chains out of LDS and combine lanes with DPP.

struct GemvParams {
  const void* qs;
  const void* scales;
  const float* x;  // [n][cols] fp32, quantized in the prologue
  float* y;        // [n][rows]
  int rows, cols, n;
  int bc;          // blocks per chunk (multiple of 4)
  int bcp;         // LDS row stride of the chunk arrays, in floats
  int x_vec;       // x rows are 16-byte aligned
};

template <bool kQ4, int R, int NT>
__global__ void __launch_bounds__(kThreads) gemv_kernel(GemvParams p) {
  extern __shared__ __align__(16) unsigned char lds[];
  const int cols = p.cols, B = cols / kBlock, n = p.n;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row0 = blockIdx.x * R;

  // LDS: quantized inputs, then the chunk arrays.
  int8_t* sxq = (int8_t*)lds;                              // [NT][cols]
  float* sxs = (float*)(lds + NT * cols);                  // [NT][B]
  int* sxsum = (int*)(sxs + ((NT * B + 3) & ~3));          // Q4: [NT][B][4]
  float* sf = (float*)(sxsum + (kQ4 ? NT * B * 4 : 0));    // [NT][R][4][bcp]
  float* ss = sf + NT * R * 4 * p.bcp;                     // [NT][R][bcp]

  // Prologue: quantize x (n rows) into LDS, 4 values per thread.
  {
    const int quads = cols / 4;
    for (int q = tid; q < NT * quads; q += kThreads) {
      const int t = q / quads, c = (q - t * quads) * 4;
      float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (t < n) {
        const float* px = p.x + (size_t)t * cols + c;
        v = p.x_vec ? *(const float4*)px : make_float4(px[0], px[1], px[2], px[3]);
      }
      const float amax = group8_max(fmaxf(0.0f, max4abs(v)));
      const float scale = q8_scale(amax);
      const int packed = quant4(v, q8_inv(scale));
      *(int*)(sxq + t * cols + c) = packed;
      const int j = (c >> 2) & 7;  // quad within the block
      if (j == 0) sxs[t * B + c / 32] = scale;
      if (kQ4) {
        // -8 * (sum of x bytes meeting lane l's low and high nibbles):
        // quads l and l + 4 of the block.
        const int s = sdot4(packed, 0x01010101, 0);
        const int other = __builtin_amdgcn_ds_swizzle(s, 0x101F);  // lane ^ 4
        if (j < 4) sxsum[(t * B + c / 32) * 4 + j] = -8 * (s + other);
      }
    }
  }
  __syncthreads();

  constexpr int BPU = kQ4 ? 64 : 32;  // blocks per 1 KB wave load of a row
  constexpr int U = 8;                // unit loads in flight per lane
  const int bcp = p.bcp;
  float acc = 0.0f;
  // Chain lane assignment: chain c = (t, r, l), c = tid for c < NT * R * 4.
  const int chains = NT * R * 4;

  for (int cb = 0; cb < B; cb += p.bc) {
    const int nb = min(p.bc, B - cb);
    const int nb4 = (nb + 3) & ~3;
    const int segs = (nb + BPU - 1) / BPU;
    const int units = R * segs;
    for (int u0 = wave; u0 < units; u0 += 4 * U) {
      uint4 raw[U];
      float sw[U];
#pragma unroll
      for (int i = 0; i < U; i++) {
        const int u = u0 + 4 * i;
        const int r = u / segs, sg = u - (u / segs) * segs;
        const int bl = sg * BPU + (kQ4 ? lane : lane >> 1);
        const int row = row0 + r;
        const bool ok = u < units && bl < nb && row < p.rows;
        raw[i] = make_uint4(0, 0, 0, 0);
        sw[i] = 0.0f;
        if (ok) {
          const int blk = cb + bl;
          if (kQ4) {
            raw[i] = *(const uint4*)((const uint8_t*)p.qs + (size_t)row * (cols / 2) + blk * 16);
            sw[i] = half_bits_to_float(((const uint16_t*)p.scales)[(size_t)row * B + blk]);
          } else {
            raw[i] = *(const uint4*)((const int8_t*)p.qs + (size_t)row * cols + blk * 32 +
                                     (lane & 1) * 16);
            sw[i] = ((const float*)p.scales)[(size_t)row * B + blk];
          }
        }
      }
#pragma unroll
      for (int i = 0; i < U; i++) {
        const int u = u0 + 4 * i;
        if (u >= units) break;  // uniform across the wave
        const int r = u / segs, sg = u - (u / segs) * segs;
        const int bl = sg * BPU + (kQ4 ? lane : lane >> 1);
        const bool ok = bl < nb;  // rows past the end were loaded as zeros
        const bool pad = !ok && bl < nb4;
        const int blk = cb + (ok ? bl : 0);
#pragma unroll
        for (int t = 0; t < NT; t++) {
          if (kQ4) {
            const int4 xa = *(const int4*)(sxq + t * cols + blk * 32);
            const int4 xb = *(const int4*)(sxq + t * cols + blk * 32 + 16);
            const int4 c8 = *(const int4*)(sxsum + (t * B + blk) * 4);
            const int m = 0x0f0f0f0f;
            const int d0 = sdot4(raw[i].x & m, xa.x, sdot4((raw[i].x >> 4) & m, xb.x, c8.x));
            const int d1 = sdot4(raw[i].y & m, xa.y, sdot4((raw[i].y >> 4) & m, xb.y, c8.y));
            const int d2 = sdot4(raw[i].z & m, xa.z, sdot4((raw[i].z >> 4) & m, xb.z, c8.z));
            const int d3 = sdot4(raw[i].w & m, xa.w, sdot4((raw[i].w >> 4) & m, xb.w, c8.w));
            float* f = sf + ((t * R + r) * 4) * bcp + bl;
            if (ok) {
              f[0] = (float)d0;
              f[bcp] = (float)d1;
              f[2 * bcp] = (float)d2;
              f[3 * bcp] = (float)d3;
              ss[(t * R + r) * bcp + bl] = sw[i] * sxs[t * B + blk];
            } else if (pad) {
              f[0] = 0.0f;
              f[bcp] = 0.0f;
              f[2 * bcp] = 0.0f;
              f[3 * bcp] = 0.0f;
              ss[(t * R + r) * bcp + bl] = 0.0f;
            }
          } else {
            const int h = lane & 1;
            const int4 xv = *(const int4*)(sxq + t * cols + blk * 32 + h * 16);
            int p0 = sdot4(raw[i].x, xv.x, 0), p1 = sdot4(raw[i].y, xv.y, 0);
            int p2 = sdot4(raw[i].z, xv.z, 0), p3 = sdot4(raw[i].w, xv.w, 0);
            // Lane l's sum takes 4 bytes of each half: add the partner's.
            p0 += dpp<kQuadXor1>(p0);
            p1 += dpp<kQuadXor1>(p1);
            p2 += dpp<kQuadXor1>(p2);
            p3 += dpp<kQuadXor1>(p3);
            const float v0 = (float)(h ? p2 : p0), v1 = (float)(h ? p3 : p1);
            float* f = sf + ((t * R + r) * 4 + 2 * h) * bcp + bl;
            if (ok) {
              f[0] = v0;
              f[bcp] = v1;
              if (h == 0) ss[(t * R + r) * bcp + bl] = sw[i] * sxs[t * B + blk];
            } else if (pad) {
              f[0] = 0.0f;
              f[bcp] = 0.0f;
              if (h == 0) ss[(t * R + r) * bcp + bl] = 0.0f;
            }
          }
        }
      }
    }
    __syncthreads();
    // The FMA chains over this chunk, in block order.
    if (tid < chains) {
      const int l = tid & 3, tr = tid >> 2;  // tr = t * R + r
      const float* fp = sf + (tr * 4 + l) * bcp;
      const float* sp = ss + tr * bcp;
      for (int b = 0; b < nb4; b += 4) {
        const float4 fv = *(const float4*)(fp + b);
        const float4 sv = *(const float4*)(sp + b);
        acc = fmaf(fv.x, sv.x, acc);
        acc = fmaf(fv.y, sv.y, acc);
        acc = fmaf(fv.z, sv.z, acc);
        acc = fmaf(fv.w, sv.w, acc);
      }
    }
    __syncthreads();
  }
  // (acc0 + acc1) + (acc2 + acc3) within each group of 4 chain lanes.
  float v = acc + dppf<kQuadXor1>(acc);
  v = v + dppf<kQuadXor2>(v);
  if (tid < chains && (tid & 3) == 0) {
    const int tr = tid >> 2, t = tr / R, r = tr - t * R;
    if (t < n && row0 + r < p.rows) p.y[(size_t)t * p.rows + row0 + r] = v;
  }
}

// ------------------------------------------------------------ argmax

// argmaxToken (lib/src/sampler.dart:137-143): the first index of the
// maximum. Values become order-preserving keys (with -0 == +0 and NaN below
// everything), packed with the complemented index so that one unsigned max
// picks the largest value and, on a tie, the lowest index.
DNX_DEV uint64_t argmax_key(float v, uint32_t i) {
  uint32_t b = __float_as_uint(v);
  if (v == 0.0f) b = 0;  // -0 ties with +0
  uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  if (v != v) ord = 0;   // NaN never wins
  return ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - i);
}

DNX_DEV uint64_t wave_max_u64(uint64_t k) {
  for (int off = 32; off >= 1; off >>= 1) {
    const uint64_t o = __shfl_xor(k, off);
    k = o > k ? o : k;
  }
  return k;
}

__global__ void __launch_bounds__(kThreads)
argmax_partial_kernel(const float* __restrict__ v, int64_t n, uint64_t* __restrict__ part) {
  __shared__ uint64_t red[kThreads / 64];
  uint64_t best = 0;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads) {
    const uint64_t k = argmax_key(v[i], (uint32_t)i);
    best = k > best ? k : best;
  }
  best = wave_max_u64(best);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = red[0];
    for (int w = 1; w < kThreads / 64; w++) b = red[w] > b ? red[w] : b;
    part[blockIdx.x] = b;
  }
}

__global__ void __launch_bounds__(kThreads)
argmax_final_kernel(const float* __restrict__ v, const uint64_t* __restrict__ part, int parts,
                    int64_t* __restrict__ out) {
  __shared__ uint64_t red[kThreads / 64];
  uint64_t best = 0;
  for (int i = threadIdx.x; i < parts; i += kThreads) best = part[i] > best ? part[i] : best;
  best = wave_max_u64(best);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = red[0];
    for (int w = 1; w < kThreads / 64; w++) b = red[w] > b ? red[w] : b;
    // A NaN at index 0 is never replaced (every comparison with it is
    // false); every other NaN is skipped. All-NaN keys are 0 -> index 0.
    const int64_t idx = (int64_t)(0xffffffffu - (uint32_t)(b & 0xffffffffu));
    out[0] = (v[0] != v[0] || (b >> 32) == 0) ? 0 : idx;
  }
}

// ------------------------------------------------------------ glue

// SiLU(g) * u in place (lab_gpu_enc_swiglu; CPU glue lib/src/shard.dart:
// 457-461). The CPU does it in double and stores float32 twice: SiLU is
// computed in double here too, then rounded; the product of two floats in
// double is exact, so one float multiply rounds it identically.
DNX_DEV float silu_mul1(float g, float u) {
  const double a = (double)g;
  const float s = (float)(a / (1.0 + exp(-a)));
  return s * u;
}

__global__ void __launch_bounds__(kThreads)
swiglu_kernel(float* __restrict__ g, const float* __restrict__ u, int64_t count) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < count;
       i += (int64_t)gridDim.x * kThreads) {
    g[i] = silu_mul1(g[i], u[i]);
  }
}

// Abramowitz-Stegun 7.1.26 erf in double (lib/src/vision_encoder.dart:
// 496-509) and the projector's GELU (:260-263), stored to float.
DNX_DEV double as_erf(double value) {
  const double x = fabs(value);
  const double t = 1 / (1 + 0.3275911 * x);
  const double poly =
      (((((1.061405429 * t - 1.453152027) * t) + 1.421413741) * t - 0.284496736) * t +
       0.254829592) *
      t;
  const double result = 1 - poly * exp(-x * x);
  return value < 0 ? -result : result;
}

__global__ void __launch_bounds__(kThreads) gelu_kernel(float* __restrict__ x, int64_t count) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < count;
       i += (int64_t)gridDim.x * kThreads) {
    const double v = x[i];
    x[i] = (float)(0.5 * v * (1 + as_erf(v / 1.4142135623730951)));
  }
}

int grid_for(int64_t items, int per_block, int cap) {
  int64_t g = (items + per_block - 1) / per_block;
  if (g < 1) g = 1;
  return (int)(g > cap ? cap : g);
}

// GEMV launch shape for a problem: rows per workgroup R and the chunking.
struct GemvShape {
  int R, NT, bc, bcp;
  size_t lds;
};

size_t gemv_lds(bool q4, int R, int NT, int cols, int bcp) {
  const int B = cols / kBlock;
  // Matches the carving at the top of gemv_kernel.
  return (size_t)NT * cols + 4 * (size_t)((NT * B + 3) & ~3) + (q4 ? (size_t)NT * B * 16 : 0) +
         (size_t)NT * R * 5 * bcp * 4;
}

GemvShape gemv_shape(bool q4, int64_t rows, int64_t cols, int64_t n) {
  GemvShape s;
  s.NT = n <= 1 ? 1 : n <= 2 ? 2 : 4;
  // Enough workgroups to give every CU a few: 16 rows each on large
  // matrices, fewer on small ones.
  const int64_t tiles16 = (rows + 15) / 16;
  s.R = tiles16 >= 2048 ? 16 : (rows + 7) / 8 >= 512 ? 8 : 4;
  if (s.NT * s.R > 32) s.R = 32 / s.NT;
  const int B = (int)(cols / kBlock);
  // One chunk when the LDS allows (<= 64 KB), else chunks of a multiple of 64.
  int bc = (B + 3) & ~3;
  for (;;) {
    const int bcp = ((bc + 63) & ~63) + 4;
    const size_t lds = gemv_lds(q4, s.R, s.NT, (int)cols, bcp);
    if (lds <= 64 * 1024 || bc <= 64) {
      s.bc = bc;
      s.bcp = bcp;
      s.lds = lds;
      break;
    }
    bc = ((bc / 2) + 63) & ~63;
  }
  return s;
}

template <bool kQ4>
int launch_gemv(const void* qs, const void* scales, const float* x, float* y, int64_t rows,
                int64_t cols, int64_t n, hipStream_t stream) {
  if (rows <= 0 || cols <= 0 || n <= 0 || cols % kBlock != 0 || n > 4) return DNX_EINVAL;
  if (rows > INT32_MAX || cols > (1 << 20)) return DNX_EINVAL;
  const GemvShape s = gemv_shape(kQ4, rows, cols, n);
  if (s.lds > 64 * 1024) return DNX_EINVAL;  // K too large for one workgroup's LDS
  GemvParams p;
  p.qs = qs;
  p.scales = scales;
  p.x = x;
  p.y = y;
  p.rows = (int)rows;
  p.cols = (int)cols;
  p.n = (int)n;
  p.bc = s.bc;
  p.bcp = s.bcp;
  p.x_vec = ((uintptr_t)x & 15) == 0;
  const dim3 grid((unsigned)((rows + s.R - 1) / s.R));
#define DNX_GEMV_CASE(RR, NN)                                                               \
  if (s.R == RR && s.NT == NN) {                                                            \
    hipLaunchKernelGGL((gemv_kernel<kQ4, RR, NN>), grid, dim3(kThreads), s.lds, stream, p); \
    return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;                           \
  }
  DNX_GEMV_CASE(16, 1)
  DNX_GEMV_CASE(8, 1)
  DNX_GEMV_CASE(4, 1)
  DNX_GEMV_CASE(16, 2)
  DNX_GEMV_CASE(8, 2)
  DNX_GEMV_CASE(4, 2)
  DNX_GEMV_CASE(8, 4)
  DNX_GEMV_CASE(4, 4)
#undef DNX_GEMV_CASE
  return DNX_EINVAL;
}

}  // namespace

// ------------------------------------------------------------ C ABI

extern "C" {

int dnx_quantize_q8(const float* x, int8_t* qs, float* scales, int64_t rows, int64_t cols,
                    int64_t cols_pad, hipStream_t stream) {
  if (rows < 0 || cols <= 0 || cols_pad < cols || cols_pad % kBlock != 0) return DNX_EINVAL;
  if (rows == 0) return DNX_OK;
  const int vec = (((uintptr_t)x & 15) == 0) && (cols % 4 == 0);
  const int grid = grid_for(rows * (cols_pad / 4), kThreads, 65536);
  hipLaunchKernelGGL((quantize_q8_kernel<false>), dim3(grid), dim3(kThreads), 0, stream,
                     (const void*)x, qs, scales, rows, cols, cols_pad, vec);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int dnx_quantize_q8_bf16(const uint16_t* w, int8_t* qs, float* scales, int64_t rows,
                         int64_t cols, int64_t cols_pad, hipStream_t stream) {
  if (rows < 0 || cols <= 0 || cols_pad < cols || cols_pad % kBlock != 0) return DNX_EINVAL;
  if (rows == 0) return DNX_OK;
  const int vec = (((uintptr_t)w & 7) == 0) && (cols % 4 == 0);
  const int grid = grid_for(rows * (cols_pad / 4), kThreads, 65536);
  hipLaunchKernelGGL((quantize_q8_kernel<true>), dim3(grid), dim3(kThreads), 0, stream,
                     (const void*)w, qs, scales, rows, cols, cols_pad, vec);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int dnx_gemv_q8(const int8_t* qs, const float* scales, const float* x, float* y, int64_t rows,
                int64_t cols, int64_t n, hipStream_t stream) {
  return launch_gemv<false>(qs, scales, x, y, rows, cols, n, stream);
}

int dnx_gemv_q4(const uint8_t* qs, const uint16_t* scales, const float* x, float* y,
                int64_t rows, int64_t cols, int64_t n, hipStream_t stream) {
  return launch_gemv<true>(qs, scales, x, y, rows, cols, n, stream);
}

int64_t dnx_argmax_workspace_bytes(int64_t n) {
  (void)n;
  return 1024 * (int64_t)sizeof(uint64_t);
}

int dnx_argmax(const float* v, int64_t n, int64_t* out, void* workspace, hipStream_t stream) {
  if (n <= 0 || n > 0xffffffffLL) return DNX_EINVAL;
  const int parts = grid_for(n, kThreads * 4, 1024);
  hipLaunchKernelGGL(argmax_partial_kernel, dim3(parts), dim3(kThreads), 0, stream, v, n,
                     (uint64_t*)workspace);
  hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kThreads), 0, stream, v,
                     (const uint64_t*)workspace, parts, out);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int dnx_swiglu(float* g, const float* u, int64_t count, hipStream_t stream) {
  if (count < 0) return DNX_EINVAL;
  if (count == 0) return DNX_OK;
  hipLaunchKernelGGL(swiglu_kernel, dim3(grid_for(count, kThreads, 65536)), dim3(kThreads), 0,
                     stream, g, u, count);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int dnx_gelu(float* x, int64_t count, hipStream_t stream) {
  if (count < 0) return DNX_EINVAL;
  if (count == 0) return DNX_OK;
  hipLaunchKernelGGL(gelu_kernel, dim3(grid_for(count, kThreads, 65536)), dim3(kThreads), 0,
                     stream, x, count);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

}  // extern "C"
