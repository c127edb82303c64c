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

// Items per thread per pass of the Q6_K adapter. A pass issues all of its
// loads before it uses any: one small load in flight per thread leaves a
// converter latency-bound at a quarter of HBM. The loads are raw buffer
// loads, so an item past the end or a padding column reads zeros with no
// branch and no memory access (a branch around a load makes the compiler
// wait for it right there).
constexpr int kItems = 8;
constexpr int kFar = 0x7fffff00;  // an offset past every buffer these kernels read

// Four consecutive values of row `row` from column c with plain loads (the
// generic path: unaligned inputs, odd widths, inputs of 2 GB or more);
// columns >= cols are zero.
template <bool kBf16>
DNX_DEV float4 load_quad(const void* src, int64_t row, int64_t c, int64_t cols) {
  float4 v;
  if (kBf16) {
    const uint16_t* p = (const uint16_t*)src + row * cols + c;
    v.x = c + 0 < cols ? bf16_to_float(p[0]) : 0.0f;
    v.y = c + 1 < cols ? bf16_to_float(p[1]) : 0.0f;
    v.z = c + 2 < cols ? bf16_to_float(p[2]) : 0.0f;
    v.w = c + 3 < cols ? bf16_to_float(p[3]) : 0.0f;
  } else {
    const float* p = (const float*)src + row * cols + c;
    v.x = c + 0 < cols ? p[0] : 0.0f;
    v.y = c + 1 < cols ? p[1] : 0.0f;
    v.z = c + 2 < cols ? p[2] : 0.0f;
    v.w = c + 3 < cols ? p[3] : 0.0f;
  }
  return v;
}

// lab_quantize_q8 (lab_native.c:407-429) of quad q: its 8-lane group is
// one 32-block; int8 at qs + 4q, the block's scale at scales[q / 8] (padded
// rows keep whole blocks, so the layout is linear in q).
DNX_DEV void q8_quad(float4 v, int64_t q, int8_t* qs, float* scales) {
  const float amax = group8_max(fmaxf(0.0f, max4abs(v)));
  const float scale = q8_scale(amax);
  const float inv = q8_inv(scale);
  *(int*)(qs + 4 * q) = quant4(v, inv);
  if ((q & 7) == 0) scales[q >> 3] = scale;
}

// float -> fp16 bits, round to nearest even (the reference's float_to_half,
// lab_native.c:923-925). The value goes through an empty asm first: without
// it the compiler folds d = max * -0.125 and this conversion into one
// v_fma_mix with a +0 addend, which turns d = -0 (an all-zero block) into +0.
DNX_DEV uint16_t half_rne(float f) {
  asm volatile("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// lab_quantize_q4 (lab_native.c:928-955, llama.cpp's quantize_row_q4_0_ref)
// of quad q. Per block: max = the first value (in column order) of largest
// magnitude (`a > amax` from 0, so NaN never wins and ties keep the first);
// d = max / -8; id = 1/d (0 when d == 0); q = (int8_t)(x * id + 8.5f)
// clamped above at 15 (two float roundings: the reference is built without
// contraction); byte k = q[k] | q[k + 16] << 4; the scale is d rounded to
// fp16 (RNE, as _mm_cvtps_ph). The 8-lane group finds the largest
// magnitude, then the lowest (index, sign) key holding it; lanes 0-3 write
// the block's 16 bytes at 16 (q / 8), taking the high nibbles (values
// 16..31) from lanes 4-7.
DNX_DEV void q4_quad(float4 v, int64_t q, uint8_t* qs, uint16_t* scales) {
  const int k0 = (int)((4 * q) & 31);
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
    *(uint32_t*)(qs + 16 * (q >> 3) + k0) = out;
  }
  if (k0 == 0) scales[q >> 3] = half_rne(d);
}

// Q8 (kQ4 false) or Q4 quantizer over rows x cols values (fp32 or bf16),
// with one lane per 32-block: the block's 128 (fp32) or 64 (bf16) bytes
// arrive in 16-byte buffer loads issued together, then the lane runs the
// reference's scalar loop itself (block max in column order, one division
// per block, 32 values) and stores 32 (Q8) or 16 (Q4) bytes and the scale.
// Lanes of a wave take consecutive blocks, so stores are contiguous. The
// output has rows x cols_pad values (cols_pad a multiple of 32 >= cols; Q4
// has no padding); columns >= cols load as zeros (the padding, R10's
// extension). Requires cols a multiple of 8 (no 16-byte load straddles a
// row's end) and an input below 2 GB (32-bit buffer offsets).
template <bool kQ4, bool kBf16, bool kPad>
__global__ void __launch_bounds__(kThreads)
quantize_kernel(const void* __restrict__ src, void* __restrict__ qs, void* __restrict__ scales,
                int64_t rows, int cols, int cols_pad, uint32_t src_bytes) {
  constexpr int kEsize = kBf16 ? 2 : 4;
  constexpr int kLoads = 32 * kEsize / 16;   // 16-byte loads per block
  constexpr int kPer = 16 / kEsize;          // values per load
  const int bpr = cols_pad / 32;
  const int64_t total = rows * bpr;
  const i32x4 rsrc = buffer_rsrc(src, src_bytes);
  for (int64_t b = (int64_t)blockIdx.x * kThreads + threadIdx.x; b < total;
       b += (int64_t)gridDim.x * kThreads) {
    int64_t start;   // element offset of the block's first value in src
    int c0;          // its column
    if (kPad) {      // total < 2^31: 32-bit division
      const uint32_t row = (uint32_t)b / (uint32_t)bpr;
      c0 = (int)((uint32_t)b - row * (uint32_t)bpr) * 32;
      start = (int64_t)row * cols + c0;
    } else {
      c0 = 0;
      start = b * 32;
    }
    uint4 raw[kLoads];
#pragma unroll
    for (int j = 0; j < kLoads; j++) {
      const bool in = !kPad || c0 + j * kPer < cols;
      raw[j] = buffer_load16(rsrc, in ? (int)((start + j * kPer) * kEsize) : kFar);
    }
    float v[32];
#pragma unroll
    for (int j = 0; j < kLoads; j++) {
      const uint32_t w[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
#pragma unroll
      for (int i = 0; i < 4; i++) {
        if (kBf16) {  // bf16 bits p -> float p << 16 (safetensors.dart:207-212)
          v[j * 8 + 2 * i] = __uint_as_float(w[i] << 16);
          v[j * 8 + 2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        } else {
          v[j * 4 + i] = __uint_as_float(w[i]);
        }
      }
    }
    if (kQ4) {
      // lab_quantize_q4 (lab_native.c:933-953): the first value of largest
      // magnitude, strict `>` from 0 (NaN never wins, ties keep the first).
      float amax = 0.0f, max = 0.0f;
#pragma unroll
      for (int k = 0; k < 32; k++) {
        const float a = v[k] < 0.0f ? -v[k] : v[k];
        if (a > amax) {
          amax = a;
          max = v[k];
        }
      }
      const float d = max / -8.0f;
      const float id = d != 0.0f ? 1.0f / d : 0.0f;
      const uint16_t dh = half_rne(d);
      uint32_t out[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        uint32_t word = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const int lo = q4_value(v[4 * i + k], id);
          const int hi = q4_value(v[4 * i + k + 16], id);
          word |= (uint32_t)((lo | (hi << 4)) & 0xff) << (8 * k);
        }
        out[i] = word;
      }
      *(uint4*)((uint8_t*)qs + 16 * b) = make_uint4(out[0], out[1], out[2], out[3]);
      ((uint16_t*)scales)[b] = dh;
    } else {
      // lab_quantize_q8 (lab_native.c:411-427).
      float amax = 0.0f;
#pragma unroll
      for (int k = 0; k < 32; k++) {
        const float a = fabsf(v[k]);
        amax = a > amax ? a : amax;
      }
      const float scale = q8_scale(amax);
      const float inv = q8_inv(scale);
      uint32_t out[8];
#pragma unroll
      for (int i = 0; i < 8; i++) {
        out[i] = (uint32_t)quant4(make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]),
                                  inv);
      }
      uint4* dst = (uint4*)((int8_t*)qs + 32 * b);
      dst[0] = make_uint4(out[0], out[1], out[2], out[3]);
      dst[1] = make_uint4(out[4], out[5], out[6], out[7]);
      ((float*)scales)[b] = scale;
    }
  }
}

// The quad-per-lane path of the same quantizers: one quad per thread per
// step, 8 threads per block, plain loads (any alignment, width or size; also
// the faster one for small matrices).
template <bool kQ4, bool kBf16>
__global__ void __launch_bounds__(kThreads)
quantize_generic_kernel(const void* __restrict__ src, void* __restrict__ qs,
                        void* __restrict__ scales, int64_t rows, int64_t cols, int64_t cols_pad) {
  const int64_t qpr = cols_pad / 4;
  const int64_t total = rows * qpr;
  for (int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x; q < total;
       q += (int64_t)gridDim.x * kThreads) {
    const int64_t row = q / qpr;
    const float4 v = load_quad<kBf16>(src, row, (q - row * qpr) * 4, cols);
    if (kQ4) {
      q4_quad(v, q, (uint8_t*)qs, (uint16_t*)scales);
    } else {
      q8_quad(v, q, (int8_t*)qs, (float*)scales);
    }
  }
}

// The Q6_K -> Q8 embedding / LM-head adapter (lib/src/gguf.dart:402-414):
// dequantizeQ6K (:220-254, ggml's dequantize_row_q6_K) then lab_quantize_q8
// (lab_native.c:407-429), fused. rows x cols values, cols a multiple of 256,
// arrive as 210-byte super-blocks, row after row: ql[128] (4 low bits),
// qh[64] (2 high bits each), int8 sc[16] (one per 16 values), fp16 d. Value
// v of a super-block: half h = v / 128, w = v % 128, quarter u = w / 32,
// l = w % 32; low bits from ql[64h + l + 32(u & 1)] (high nibble when
// u >= 2), high bits (qh[32h + l] >> 2u) & 3, scale sc[8h + l/16 + 2u].
// The reference computes d * sc * (q - 32) in double and stores a float:
// d * sc is exact in float (at most 19 significant bits), so one float
// multiply by (q - 32) rounds the same exact product once, identically.
// Then q8_quad, bit-exact.
//
// This kernel serves matrices below 64K output blocks (q6k_block_kernel
// below takes the larger ones). One wave takes one super-block per item
// (lane L: values 4L..4L+3, one 16-value scale group; 8 lanes per Q8
// block). Super-blocks start 2-byte
// aligned (210 = 2 x 105), so lane L loads aligned dword L of the block's
// span (one coalesced load per lane and item, bounded by the buffer) and
// each lane gathers its bytes from the wave's registers with ds_bpermute:
// 4 ql bytes and 4 qh bytes (two dwords and an alignbyte each) and its
// scale byte. d comes from a 2-byte load of the block's last bytes.
__global__ void __launch_bounds__(kThreads)
q6k_to_q8_kernel(const uint8_t* __restrict__ src, int8_t* __restrict__ qs,
                 float* __restrict__ scales, int64_t rows, int64_t cols) {
  const int64_t total = rows * (cols / 4);   // a multiple of 64: whole waves
  const int lane = threadIdx.x & 63;
  const i32x4 rsrc = buffer_rsrc(src, (uint32_t)(rows * (cols / 256) * 210));
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t q0 = (int64_t)blockIdx.x * kThreads + threadIdx.x; q0 < total;
       q0 += stride * kItems) {
    uint32_t word[kItems];
    short dbits[kItems];
#pragma unroll
    for (int u = 0; u < kItems; u++) {
      const int64_t q = q0 + u * stride;   // uniform over the wave's super-block
      const int64_t base = (q >> 6) * 210;
      const bool in = q < total;
      word[u] = (uint32_t)dnx_raw_buffer_load_i32(
          rsrc, in ? (int)((base & ~3ll) + 4 * lane) : kFar, 0, 0);
      // d on its own: the dword holding it can reach past the last block,
      // and a dword past the buffer's end reads as zero.
      dbits[u] = dnx_raw_buffer_load_i16(rsrc, in ? (int)(base + 208) : kFar, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kItems; u++) {
      const int64_t q = q0 + u * stride;
      if (q >= total) break;
      const int delta = (int)(((q >> 6) * 210) & 3);   // 0 or 2
      const int v = 4 * lane, h = v >> 7, qu = (v >> 5) & 3, l = v & 31;
      auto bytes4 = [&](int rel) {
        const int r = rel + delta;
        const uint32_t w0 = (uint32_t)__shfl((int)word[u], r >> 2);
        const uint32_t w1 = (uint32_t)__shfl((int)word[u], (r >> 2) + 1);
        return __builtin_amdgcn_alignbyte(w1, w0, (uint32_t)(r & 3));
      };
      auto byte_at = [&](int rel) {
        const int r = rel + delta;
        return ((uint32_t)__shfl((int)word[u], r >> 2) >> (8 * (r & 3))) & 0xffu;
      };
      const uint32_t ql = bytes4(64 * h + l + 32 * (qu & 1));
      const uint32_t qh = bytes4(128 + 32 * h + l);
      const int8_t sc = (int8_t)byte_at(192 + 8 * h + (l >> 4) + 2 * qu);
      const float ds = half_bits_to_float((uint16_t)dbits[u]) * (float)sc;
      const int lo_shift = (qu >> 1) * 4, hi_shift = 2 * qu;
      float e[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int qv = (int)((((ql >> (8 * j)) >> lo_shift) & 15) |
                             ((((qh >> (8 * j)) >> hi_shift) & 3) << 4)) - 32;
        e[j] = ds * (float)qv;
      }
      q8_quad(make_float4(e[0], e[1], e[2], e[3]), q, qs, scales);
    }
  }
}

// The same adapter with one lane per output 32-block (large matrices, as the
// quantizers' fast path): block j of super-block s (h = j / 4, u = j % 4)
// takes the 32-byte runs ql[64h + 32(u & 1) ..] (nibble u / 2) and
// qh[32h ..] (bits 2u, 2u + 1), the scales sc[8h + 2u] (values 0-15) and
// sc[8h + 2u + 1] (16-31) in one 2-byte load, and d. Each run arrives as 36
// bytes of 4-byte aligned loads realigned by 0 or 2 bytes (v_alignbyte);
// none reaches past its super-block. The lane then dequantizes as above and
// runs lab_quantize_q8's scalar loop on its 32 values: one pair of divisions
// per block instead of per quad.
__global__ void __launch_bounds__(kThreads)
q6k_block_kernel(const uint8_t* __restrict__ src, int8_t* __restrict__ qs,
                 float* __restrict__ scales, int64_t nblocks, uint32_t src_bytes) {
  const i32x4 rs = buffer_rsrc(src, src_bytes);
  for (int64_t b = (int64_t)blockIdx.x * kThreads + threadIdx.x; b < nblocks;
       b += (int64_t)gridDim.x * kThreads) {
    const int j = (int)(b & 7), h = j >> 2, u = j & 3;
    const int base = (int)((b >> 3) * 210);
    const int lo_at = base + 64 * h + 32 * (u & 1), hi_at = base + 128 + 32 * h;
    const uint32_t sh = (uint32_t)(base & 3);   // 0 or 2, the runs' too
    const uint4 l0 = buffer_load16(rs, lo_at & ~3), l1 = buffer_load16(rs, (lo_at & ~3) + 16);
    const uint32_t l2 = (uint32_t)dnx_raw_buffer_load_i32(rs, (lo_at & ~3) + 32, 0, 0);
    const uint4 h0 = buffer_load16(rs, hi_at & ~3), h1 = buffer_load16(rs, (hi_at & ~3) + 16);
    const uint32_t h2 = (uint32_t)dnx_raw_buffer_load_i32(rs, (hi_at & ~3) + 32, 0, 0);
    const uint32_t scw = (uint16_t)dnx_raw_buffer_load_i16(rs, base + 192 + 8 * h + 2 * u, 0, 0);
    const uint32_t dbits = (uint16_t)dnx_raw_buffer_load_i16(rs, base + 208, 0, 0);
    const uint32_t lw[9] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w, l2};
    const uint32_t hw[9] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w, h2};
    const float dd = half_bits_to_float((uint16_t)dbits);
    const float ds0 = dd * (float)(int8_t)(scw & 0xffu);
    const float ds1 = dd * (float)(int8_t)(scw >> 8);
    const int nib = 4 * (u >> 1), bit = 2 * u;
    float v[32];
#pragma unroll
    for (int w = 0; w < 8; w++) {
      const uint32_t ql = __builtin_amdgcn_alignbyte(lw[w + 1], lw[w], sh);
      const uint32_t qh = __builtin_amdgcn_alignbyte(hw[w + 1], hw[w], sh);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int q = (int)(((ql >> (8 * i + nib)) & 15u) | (((qh >> (8 * i + bit)) & 3u) << 4));
        v[4 * w + i] = (w < 4 ? ds0 : ds1) * (float)(q - 32);
      }
    }
    // lab_quantize_q8 (lab_native.c:411-427). The values are products of
    // converted floats, so any NaN among them is quiet, and v_max_f32 keeps
    // the non-NaN operand as `a > amax` does.
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < 32; k++) amax = fmaxf(amax, fabsf(v[k]));
    const float scale = q8_scale(amax);
    const float inv = q8_inv(scale);
    uint32_t out[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
      out[i] = (uint32_t)quant4(make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]),
                                inv);
    uint4* dst = (uint4*)(qs + 32 * b);
    dst[0] = make_uint4(out[0], out[1], out[2], out[3]);
    dst[1] = make_uint4(out[4], out[5], out[6], out[7]);
    scales[b] = scale;
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
// 457-461), rounded as the CPU rounds it (silu_mul_exact).
__global__ void __launch_bounds__(kThreads)
swiglu_kernel(float* __restrict__ g, const float* __restrict__ u, int64_t count) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < count;
       i += (int64_t)gridDim.x * kThreads) {
    g[i] = silu_mul_exact(g[i], u[i]);
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

DNX_DEV float gelu1(float f) {
  const double v = f;
  return (float)(0.5 * v * (1 + as_erf(v / 1.4142135623730951)));
}

// Four values per thread and pass: one 16-byte load and store, and four
// independent double chains (two IEEE divisions and an exp each) for the
// scheduler to interleave; one value per thread left each wave waiting on
// one chain (15 us for the vision pair's 4.4 M values). x16 is x from its
// first 16-byte aligned value (head values before it, tail values after the
// last whole quad: done one per thread by workgroup 0).
__global__ void __launch_bounds__(kThreads) gelu_kernel(float* __restrict__ x, int64_t count,
                                                        int head) {
  float4* x16 = (float4*)(x + head);
  const int64_t quads = (count - head) / 4;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < quads;
       i += (int64_t)gridDim.x * kThreads) {
    float4 v = x16[i];
    v.x = gelu1(v.x);
    v.y = gelu1(v.y);
    v.z = gelu1(v.z);
    v.w = gelu1(v.w);
    x16[i] = v;
  }
  if (blockIdx.x == 0) {
    const int t = threadIdx.x;
    const int64_t tail0 = head + quads * 4;
    if (t < head) x[t] = gelu1(x[t]);
    if (t < count - tail0) x[tail0 + t] = gelu1(x[tail0 + t]);
  }
}

// Grid of the Q6_K adapter: kItems quads per thread when there is enough work,
// but at least one workgroup per 256 quads up to 2048 workgroups (8 per CU),
// so small inputs still spread over the chip.
int quantizer_grid(int64_t quads) {
  int64_t g = (quads + kThreads * kItems - 1) / (kThreads * kItems);
  const int64_t spread = (quads + kThreads - 1) / kThreads;
  const int64_t lo = spread < 2048 ? spread : 2048;
  if (g < lo) g = lo;
  if (g < 1) g = 1;
  return (int)(g > 65536 ? 65536 : g);
}

int grid_for(int64_t items, int per_block, int cap) {
  int64_t g = (items + per_block - 1) / per_block;
  if (g < 1) g = 1;
  return (int)(g > cap ? cap : g);
}

// Launches a quantizer: the block-per-lane kernel when the input is 4-byte
// aligned, the output 16-byte aligned, cols a multiple of 8, the input below
// 2 GB and the matrix at least 64 K blocks, else the quad-per-lane one. Q8: cols_pad >= cols, a multiple of 32;
// Q4: cols_pad == cols.
template <bool kQ4, bool kBf16>
int launch_quantizer(const void* src, void* qs, void* scales, int64_t rows, int64_t cols,
                     int64_t cols_pad, hipStream_t stream) {
  const int64_t blocks = rows * (cols_pad / 32);
  const int64_t src_bytes = rows * cols * (kBf16 ? 2 : 4);
  // Below 64 K blocks (fewer than one wave of lanes per SIMD) the quad-per-
  // lane kernel spreads the work over 8x more lanes and finishes sooner
  // (512 x 2048 fp32: 2.8 us against 3.4).
  const bool fast = ((uintptr_t)src & 3) == 0 && ((uintptr_t)qs & 15) == 0 && cols % 8 == 0 &&
                    src_bytes < kFar && cols_pad < kFar && blocks >= 65536;
  const int grid = grid_for(blocks, kThreads, 65536);
  if (fast && cols == cols_pad) {
    hipLaunchKernelGGL((quantize_kernel<kQ4, kBf16, false>), dim3(grid), dim3(kThreads), 0,
                       stream, src, qs, scales, rows, (int)cols, (int)cols_pad,
                       (uint32_t)src_bytes);
  } else if (fast) {
    hipLaunchKernelGGL((quantize_kernel<kQ4, kBf16, true>), dim3(grid), dim3(kThreads), 0,
                       stream, src, qs, scales, rows, (int)cols, (int)cols_pad,
                       (uint32_t)src_bytes);
  } else {
    hipLaunchKernelGGL((quantize_generic_kernel<kQ4, kBf16>),
                       dim3(grid_for(rows * (cols_pad / 4), kThreads, 65536)), dim3(kThreads), 0,
                       stream, src,
                       qs, scales, rows, cols, cols_pad);
  }
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

// GGUF Q8_0 / Q4_0 blocks -> the engine's layout (splitQ8_0, gguf.dart:
// 270-282; splitQ4_0, :208-218). A GGUF block is its fp16 d, then the
// values: 34 bytes (Q8_0: 32 int8) or 18 (Q4_0: 16 nibble bytes, whose
// order both layouts share). Block b's values start at byte 34b + 2
// (18b + 2): 4-byte aligned for odd b, 2 mod 4 for even b. A lane makes one
// 16-byte piece of values (Q8_0: two per block, Q4_0: one) from a 16-byte
// load at the dword at or below the piece and a 2-byte load after it,
// realigned with v_alignbyte by 0 or 2 bytes (no branch); neither load
// reaches past its block, so the last block of a buffer that ends with it
// reads whole. The lane of a block's first piece also writes the scale:
// widened to fp32 for Q8 (exact; any NaN becomes 0x7FC00000, as the
// reference's halfToDouble makes it), the fp16 bits for Q4.
constexpr int kSplitItems = 4;

template <bool kQ4>
__global__ void __launch_bounds__(kThreads)
split_gguf_kernel(const uint8_t* __restrict__ blocks, uint8_t* __restrict__ qs,
                  void* __restrict__ scales, int count, uint32_t bytes) {
  constexpr int kBytes = kQ4 ? 18 : 34;
  constexpr int kPieces = kQ4 ? 1 : 2;
  const i32x4 rs = buffer_rsrc(blocks, bytes);
  const int pieces = count * kPieces;
  const int stride = gridDim.x * kThreads * kSplitItems;
  for (int p0 = blockIdx.x * kThreads * kSplitItems + threadIdx.x; p0 < pieces; p0 += stride) {
    uint4 lo[kSplitItems];
    uint32_t hi[kSplitItems], d[kSplitItems];
#pragma unroll
    for (int j = 0; j < kSplitItems; j++) {  // every load in flight at once
      const int p = p0 + j * kThreads, b = p / kPieces, h = p % kPieces;
      const int s = b * kBytes + 2 + 16 * h;
      const bool in = p < pieces;
      lo[j] = buffer_load16(rs, in ? (s & ~3) : kFar);
      hi[j] = (uint16_t)dnx_raw_buffer_load_i16(rs, in ? (s & ~3) + 16 : kFar, 0, 0);
      d[j] = (uint16_t)dnx_raw_buffer_load_i16(rs, in && h == 0 ? b * kBytes : kFar, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < kSplitItems; j++) {
      const int p = p0 + j * kThreads, b = p / kPieces, h = p % kPieces;
      if (p >= pieces) continue;
      const uint32_t sh = (uint32_t)((b * kBytes + 2) & 3);   // 0 or 2
      uint4 out;
      out.x = __builtin_amdgcn_alignbyte(lo[j].y, lo[j].x, sh);
      out.y = __builtin_amdgcn_alignbyte(lo[j].z, lo[j].y, sh);
      out.z = __builtin_amdgcn_alignbyte(lo[j].w, lo[j].z, sh);
      out.w = __builtin_amdgcn_alignbyte(hi[j], lo[j].w, sh);
      *(uint4*)(qs + (size_t)p * 16) = out;
      if (h == 0) {
        if (kQ4) {
          ((uint16_t*)scales)[b] = (uint16_t)d[j];
        } else {
          // halfToDouble (native.dart:871-880) gives Dart's double.nan for
          // every NaN pattern: 0x7FC00000 once stored as a float.
          const float f = half_bits_to_float((uint16_t)d[j]);
          ((float*)scales)[b] = f == f ? f : __uint_as_float(0x7FC00000u);
        }
      }
    }
  }
}

template <bool kQ4>
int split_gguf(const void* blocks, uint8_t* qs, void* scales, int64_t count, hipStream_t stream) {
  constexpr int64_t kBytes = kQ4 ? 18 : 34;
  if (count < 0 || ((uintptr_t)blocks & 3) || ((uintptr_t)qs & 15) ||
      ((uintptr_t)scales & (kQ4 ? 1 : 3))) {
    return DNX_EINVAL;
  }
  // Segments of 2^25 blocks keep buffer offsets 32-bit; an even first
  // block keeps each segment's base 4-byte aligned.
  constexpr int64_t kSeg = 1ll << 25;
  for (int64_t first = 0; first < count; first += kSeg) {
    const int64_t n = count - first < kSeg ? count - first : kSeg;
    const int64_t pieces = n * (kQ4 ? 1 : 2);
    int64_t grid = (pieces + kThreads * kSplitItems - 1) / (kThreads * kSplitItems);
    if (grid > 65536) grid = 65536;
    hipLaunchKernelGGL(split_gguf_kernel<kQ4>, dim3((unsigned)grid), dim3(kThreads), 0, stream,
                       (const uint8_t*)blocks + first * kBytes, qs + first * (kQ4 ? 16 : 32),
                       kQ4 ? (void*)((uint16_t*)scales + first) : (void*)((float*)scales + first),
                       (int)n, (uint32_t)(n * kBytes));
    if (hipGetLastError() != hipSuccess) return DNX_ELAUNCH;
  }
  return DNX_OK;
}

// Region copies in one launch (the copy-backs of a commit to the host
// views). The table travels in the kernel arguments; workgroup b copies the
// kCopyChunk-byte chunk b - chunk0[r] of region r, the region whose chunk
// range holds b (a binary search over the table). Regions whose pointers
// and size are 16-byte multiples copy 16 bytes per lane, the rest byte by
// byte. Plain vector stores, so a destination may be pinned host memory.
constexpr int kCopyChunk = 16384;
constexpr int kCopyMax = DNX_COPY_MAX;
struct CopyTable {
  const uint8_t* src[kCopyMax];
  uint8_t* dst[kCopyMax];
  int64_t bytes[kCopyMax];
  int chunk0[kCopyMax + 1];
  int count;
};

__global__ void __launch_bounds__(kThreads) copy_regions_kernel(const CopyTable t) {
  const int b = blockIdx.x;
  int lo = 0, hi = t.count - 1;  // the last r with chunk0[r] <= b
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (t.chunk0[mid] <= b) lo = mid; else hi = mid - 1;
  }
  const int r = lo;
  const int64_t off = (int64_t)(b - t.chunk0[r]) * kCopyChunk;
  const int64_t left = t.bytes[r] - off;
  const int64_t len = left < kCopyChunk ? left : kCopyChunk;
  const uint8_t* src = t.src[r] + off;
  uint8_t* dst = t.dst[r] + off;
  if ((((uintptr_t)t.src[r] | (uintptr_t)t.dst[r] | (uintptr_t)t.bytes[r]) & 15) == 0) {
    for (int64_t i = threadIdx.x; i < len / 16; i += kThreads) {
      ((uint4*)dst)[i] = ((const uint4*)src)[i];
    }
  } else {
    for (int64_t i = threadIdx.x; i < len; i += kThreads) dst[i] = src[i];
  }
}

}  // namespace

// ------------------------------------------------------------ C ABI

extern "C" {

int dnx_quantize_q8(const float* x, int8_t* qs, float* scales, int64_t rows, int64_t cols,
                    int64_t cols_pad, hipStream_t stream) {
  if (rows < 0 || cols <= 0 || cols_pad < cols || cols_pad % kBlock != 0 || ((uintptr_t)qs & 3))
    return DNX_EINVAL;
  if (rows == 0) return DNX_OK;
  return launch_quantizer<false, false>(x, qs, scales, rows, cols, cols_pad, stream);
}

int dnx_quantize_q8_bf16(const uint16_t* w, int8_t* qs, float* scales, int64_t rows,
                         int64_t cols, int64_t cols_pad, hipStream_t stream) {
  if (rows < 0 || cols <= 0 || cols_pad < cols || cols_pad % kBlock != 0 || ((uintptr_t)qs & 3))
    return DNX_EINVAL;
  if (rows == 0) return DNX_OK;
  return launch_quantizer<false, true>(w, qs, scales, rows, cols, cols_pad, stream);
}

int dnx_quantize_q4(const float* w, uint8_t* qs, uint16_t* scales, int64_t rows, int64_t cols,
                    hipStream_t stream) {
  if (rows < 0 || cols <= 0 || cols % kBlock != 0 || ((uintptr_t)qs & 3)) return DNX_EINVAL;
  if (rows == 0) return DNX_OK;
  return launch_quantizer<true, false>(w, qs, scales, rows, cols, cols, stream);
}

int dnx_quantize_q4_bf16(const uint16_t* w, uint8_t* qs, uint16_t* scales, int64_t rows,
                         int64_t cols, hipStream_t stream) {
  if (rows < 0 || cols <= 0 || cols % kBlock != 0 || ((uintptr_t)qs & 3)) return DNX_EINVAL;
  if (rows == 0) return DNX_OK;
  return launch_quantizer<true, true>(w, qs, scales, rows, cols, cols, stream);
}

int dnx_q6k_to_q8(const void* blocks, int8_t* qs, float* scales, int64_t rows, int64_t cols,
                  hipStream_t stream) {
  if (rows < 0 || cols <= 0 || cols % 256 != 0 || ((uintptr_t)qs & 3)) return DNX_EINVAL;
  // 32-bit buffer offsets into the blocks.
  if (rows * (cols / 256) * 210 >= (1ll << 31)) return DNX_EINVAL;
  if (rows == 0) return DNX_OK;
  const int64_t nblocks = rows * (cols / 32);
  if (nblocks >= 65536 && ((uintptr_t)blocks & 3) == 0 && ((uintptr_t)qs & 15) == 0) {
    // One lane per 32-block: fewer instructions per value at large sizes.
    int64_t grid = (nblocks + kThreads - 1) / kThreads;
    if (grid > 65536) grid = 65536;
    hipLaunchKernelGGL(q6k_block_kernel, dim3((unsigned)grid), dim3(kThreads), 0, stream,
                       (const uint8_t*)blocks, qs, scales, nblocks,
                       (uint32_t)(rows * (cols / 256) * 210));
    return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
  }
  const int grid = quantizer_grid(rows * (cols / 4));
  hipLaunchKernelGGL(q6k_to_q8_kernel, dim3(grid), dim3(kThreads), 0, stream,
                     (const uint8_t*)blocks, qs, scales, rows, cols);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int dnx_split_q8_0(const void* blocks, int8_t* qs, float* scales, int64_t count,
                   hipStream_t stream) {
  return split_gguf<false>(blocks, (uint8_t*)qs, scales, count, stream);
}

int dnx_split_q4_0(const void* blocks, uint8_t* qs, uint16_t* scales, int64_t count,
                   hipStream_t stream) {
  return split_gguf<true>(blocks, qs, scales, count, stream);
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

int dnx_copy_regions(const void* const* src, void* const* dst, const int64_t* bytes, int count,
                     hipStream_t stream) {
  if (count < 0 || count > kCopyMax || (count > 0 && (!src || !dst || !bytes))) return DNX_EINVAL;
  CopyTable t{};
  int chunks = 0;
  int used = 0;
  for (int i = 0; i < count; i++) {
    if (bytes[i] < 0 || (bytes[i] > 0 && (src[i] == nullptr || dst[i] == nullptr))) {
      return DNX_EINVAL;
    }
    if (bytes[i] == 0) continue;
    const int64_t c = (bytes[i] + kCopyChunk - 1) / kCopyChunk;
    if (c > (1 << 24) || chunks + c > (1 << 30)) return DNX_EINVAL;
    t.src[used] = (const uint8_t*)src[i];
    t.dst[used] = (uint8_t*)dst[i];
    t.bytes[used] = bytes[i];
    t.chunk0[used] = chunks;
    chunks += (int)c;
    used++;
  }
  t.chunk0[used] = chunks;
  t.count = used;
  if (used == 0) return DNX_OK;
  hipLaunchKernelGGL(copy_regions_kernel, dim3(chunks), dim3(kThreads), 0, stream, t);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int dnx_gelu(float* x, int64_t count, hipStream_t stream) {
  if (count < 0 || ((uintptr_t)x & 3)) return DNX_EINVAL;
  if (count == 0) return DNX_OK;
  // Values before the first 16-byte boundary (at most 3, fewer when count is).
  const int64_t to16 = (int64_t)(((16 - ((uintptr_t)x & 15)) & 15) / 4);
  const int head = (int)(to16 < count ? to16 : count);
  const int64_t quads = (count - head) / 4;
  hipLaunchKernelGGL(gelu_kernel, dim3(grid_for(quads > 0 ? quads : 1, kThreads, 65536)),
                     dim3(kThreads), 0, stream, x, count, head);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

}  // extern "C"
