// gfx950 kernels of the quantized linear layer: Q8 activation/weight
// quantizers, the standalone greedy argmax, and the glue between linears.
// The exact-order decode GEMV lives in gemv.hip, the int8-MFMA GEMM in
// gemm.hip.
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

// lab_quantize_q4 (lab_native.c:928-955, llama.cpp's quantize_row_q4_0_ref)
// over rows x cols values, cols a multiple of 32, into Q4 nibbles
// [rows][cols/2] and fp16 scale bits [rows][cols/32]. Per block: max = the
// first value (in column order) of largest magnitude (`a > amax` from 0, so
// NaN never wins and ties keep the first); d = max / -8; id = 1/d (0 when
// d == 0); q = (int8_t)(x * id + 8.5f) clamped above at 15 (two float
// roundings: the reference is built without contraction); byte k = q[k] |
// q[k + 16] << 4; the scale is d rounded to fp16 (RNE, as _mm_cvtps_ph).
// One thread takes 4 consecutive values, 8 threads a block: the group's
// largest magnitude, then the lowest (index, sign) key holding it. Lanes 0-3
// of a group write the block's 16 bytes, taking the high nibbles (values
// 16..31) from lanes 4-7. Input is fp32 or bf16 (widened p << 16).
template <bool kBf16>
__global__ void __launch_bounds__(kThreads)
quantize_q4_kernel(const void* __restrict__ src, uint8_t* __restrict__ qs,
                   uint16_t* __restrict__ scales, int64_t rows, int64_t cols, int vec_ok) {
  const int64_t quads_per_row = cols / 4;
  const int64_t total = rows * quads_per_row;
  for (int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x; q < total;
       q += (int64_t)gridDim.x * kThreads) {
    const int64_t row = q / quads_per_row;
    const int64_t c = (q - row * quads_per_row) * 4;
    float4 v;
    if (kBf16) {
      const uint16_t* p = (const uint16_t*)src + row * cols + c;
      if (vec_ok) {
        const uint2 raw = *(const uint2*)p;
        v = make_float4(__uint_as_float(raw.x << 16), __uint_as_float(raw.x & 0xffff0000u),
                        __uint_as_float(raw.y << 16), __uint_as_float(raw.y & 0xffff0000u));
      } else {
        v = make_float4(bf16_to_float(p[0]), bf16_to_float(p[1]), bf16_to_float(p[2]),
                        bf16_to_float(p[3]));
      }
    } else {
      const float* p = (const float*)src + row * cols + c;
      v = vec_ok ? *(const float4*)p : make_float4(p[0], p[1], p[2], p[3]);
    }
    const int k0 = (int)(c & 31);
    const float amax = group8_max(fmaxf(0.0f, max4abs(v)));
    // Key 2k + sign of this lane's first value of magnitude amax (64: none).
    int key = 64;
    if (amax > 0.0f) {
      const float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 3; i >= 0; i--) {
        if (fabsf(e[i]) == amax) key = 2 * (k0 + i) + (e[i] < 0.0f ? 1 : 0);
      }
    }
    key = group8_min(key);
    const float max = key == 64 ? 0.0f : (key & 1) ? -amax : amax;
    const float d = max / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    // This lane's 4 values as (int8_t) bytes; lanes 0-3 pair with lanes 4-7.
    const int own = (q4_value(v.x, id) & 0xff) | ((q4_value(v.y, id) & 0xff) << 8) |
                    ((q4_value(v.z, id) & 0xff) << 16) | ((q4_value(v.w, id) & 0xff) << 24);
    const int high = __shfl_xor(own, 4);
    if (k0 < 16) {
      uint32_t out = 0;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int lo = (int8_t)(own >> (8 * i));
        const int hi = (int8_t)(high >> (8 * i));
        out |= (uint32_t)((lo | (hi << 4)) & 0xff) << (8 * i);
      }
      *(uint32_t*)(qs + row * (cols / 2) + (c - k0) / 2 + k0) = out;
    }
    if (k0 == 0) {
      scales[row * (cols / 32) + c / 32] = __builtin_bit_cast(uint16_t, (_Float16)d);
    }
  }
}

// ------------------------------------------------------------ argmax

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

int dnx_quantize_q4(const float* w, uint8_t* qs, uint16_t* scales, int64_t rows, int64_t cols,
                    hipStream_t stream) {
  if (rows < 0 || cols <= 0 || cols % kBlock != 0 || ((uintptr_t)qs & 3)) return DNX_EINVAL;
  if (rows == 0) return DNX_OK;
  const int vec = ((uintptr_t)w & 15) == 0;
  const int grid = grid_for(rows * (cols / 4), kThreads, 65536);
  hipLaunchKernelGGL((quantize_q4_kernel<false>), dim3(grid), dim3(kThreads), 0, stream,
                     (const void*)w, qs, scales, rows, cols, vec);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int dnx_quantize_q4_bf16(const uint16_t* w, uint8_t* qs, uint16_t* scales, int64_t rows,
                         int64_t cols, hipStream_t stream) {
  if (rows < 0 || cols <= 0 || cols % kBlock != 0 || ((uintptr_t)qs & 3)) return DNX_EINVAL;
  if (rows == 0) return DNX_OK;
  const int vec = ((uintptr_t)w & 7) == 0;
  const int grid = grid_for(rows * (cols / 4), kThreads, 65536);
  hipLaunchKernelGGL((quantize_q4_kernel<true>), dim3(grid), dim3(kThreads), 0, stream,
                     (const void*)w, qs, scales, rows, cols, vec);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
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
