// Shared device helpers for the gfx950 kernels of the quantized linear layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define DNX_DEV static __device__ __forceinline__

namespace dnx {

constexpr int kBlock = 32;  // values per Q8/Q4 block (lab_native.c:405, :902)

// DPP lane moves inside a wave (gfx9 encodings).
constexpr int kQuadXor1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int kHalfRowMirror = 0x141; // lane i <- lane 7-i within 8 lanes
constexpr int kRowMirror = 0x140;     // lane i <- lane 15-i within 16 lanes
constexpr int kRowShl4 = 0x104;       // lane i <- lane i+4 within 16 lanes (0 past the row)

template <int Ctrl>
DNX_DEV int dpp(int v) {
  return __builtin_amdgcn_mov_dpp(v, Ctrl, 0xF, 0xF, true);
}
template <int Ctrl>
DNX_DEV float dppf(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), Ctrl, 0xF, 0xF, true));
}

// The 4-byte signed dot product with accumulator: c + sum a_i * b_i.
DNX_DEV int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// Max over the 8 lanes of an aligned lane group (one Q block of 4-value
// quads); every lane of the group gets the result.
DNX_DEV float group8_max(float m) {
  m = fmaxf(m, dppf<kQuadXor1>(m));
  m = fmaxf(m, dppf<kQuadXor2>(m));
  m = fmaxf(m, dppf<kHalfRowMirror>(m));
  return m;
}

// group8_max for values >= 0 (or +inf, never NaN): their bit patterns order
// as integers, so integer max moves through DPP without the float max's
// NaN canonicalization.
DNX_DEV float group8_max_nonneg(float m) {
  int b = __float_as_int(m);
  b = max(b, dpp<kQuadXor1>(b));
  b = max(b, dpp<kQuadXor2>(b));
  b = max(b, dpp<kHalfRowMirror>(b));
  return __int_as_float(b);
}

// Lane j's value of each aligned 8-lane group, to every lane of the group
// (ds_swizzle bit mode within 32 lanes: source = (lane & 0x18) | j). Every
// lane of the group must be active.
template <int J>
DNX_DEV float bcast8(float v) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x18 | (J << 5)));
}

// Sum over a wave by an xor butterfly (offsets 32, 16, ..., 1). Each step
// adds the same two values on both partner lanes, so every lane ends with
// the same bits.
DNX_DEV float wave_sum_xor(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Element i of `splits` split-K partials (part[z][count], z in order):
// part[0][i] + part[1][i] + ... added in split order (deterministic), with
// the loads of 8 splits issued together (a loop that adds as it loads waits
// for each partial in turn). Splits past the last reload the last one
// (always in bounds) and are not added.
DNX_DEV float split_sum(const float* __restrict__ part, int64_t count, int64_t i, int splits) {
  constexpr int U = 8;
  float v = 0.0f;
  for (int z0 = 0; z0 < splits; z0 += U) {
    float t[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int z = z0 + u < splits ? z0 + u : splits - 1;
      t[u] = part[(size_t)z * count + i];
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      if (z0 + u < splits) v = z0 + u == 0 ? t[u] : v + t[u];
    }
  }
  return v;
}

// Max and sum over a wave without an LDS round trip: DPP inside each row of
// 16 lanes (quad xor 1, xor 2, half-row and row mirrors: every lane of a row
// ends with the row's result), then the four rows' results read into
// scalars and combined in a fixed order. Every lane gets the same bits. All
// lanes must be active.
DNX_DEV float lane_value(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
DNX_DEV float wave_max_dpp(float v) {
  v = fmaxf(v, dppf<kQuadXor1>(v));
  v = fmaxf(v, dppf<kQuadXor2>(v));
  v = fmaxf(v, dppf<kHalfRowMirror>(v));
  v = fmaxf(v, dppf<kRowMirror>(v));
  return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)),
               fmaxf(lane_value(v, 32), lane_value(v, 48)));
}
DNX_DEV float wave_sum_dpp(float v) {
  v += dppf<kQuadXor1>(v);
  v += dppf<kQuadXor2>(v);
  v += dppf<kHalfRowMirror>(v);
  v += dppf<kRowMirror>(v);
  return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

// The row sum of a 256-thread RMSNorm (rms_norm_vec_kernel, and the GEMV
// prologue that reproduces it): each wave's DPP sum, then the four wave
// totals in wave order through `scratch` (4 floats). Every thread gets the
// same bits.
DNX_DEV float norm_row_sum(float v, float* scratch) {
  v = wave_sum_dpp(v);
  __syncthreads();  // scratch may still be read from a previous call
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = scratch[0];
#pragma unroll
  for (int w = 1; w < 4; w++) t += scratch[w];
  return t;
}

// Min over the 8 lanes of an aligned lane group; every lane gets it.
DNX_DEV int group8_min(int m) {
  m = min(m, dpp<kQuadXor1>(m));
  m = min(m, dpp<kQuadXor2>(m));
  m = min(m, dpp<kHalfRowMirror>(m));
  return m;
}

// float -> int as x86 cvttss2si does: truncation, with NaN and values
// outside int32 giving INT_MIN. The reference's (int) cast compiles to that
// instruction on x86-64; it matters only where 1/scale overflows
// (amax < ~3.7e-37) or the input is not finite.
DNX_DEV int cvt_trunc_x86(float t) {
  return (t > -2147483904.0f && t < 2147483648.0f) ? (int)t : (int)0x80000000;
}

// One value of lab_quantize_q8 (lab_native.c:422-425): q = x * inv, then
// +-0.5 in float, truncation, clamp to [-127, 127]. Two roundings: the file
// is compiled with -ffp-contract=off.
//
// Written for few instructions: t + copysign(0.5, t) is t - 0.5 below zero
// and t + 0.5 above (at -0 it gives -0.5 instead of 0.5, which truncates to
// the same 0); clamping to [-127, 127] before the truncation equals clamping
// after it; x86's INT_MIN for NaN and t >= 2^31 becomes -127 through the
// clamp, and below -2^31 the clamp gives -127 already. The two forms agree
// for every float t (checked exhaustively over all 2^32 bit patterns).
DNX_DEV int quant1(float x, float inv) {
  float t = x * inv;
  t = t + __builtin_copysignf(0.5f, t);
  const int v = (int)__builtin_amdgcn_fmed3f(t, -127.0f, 127.0f);
  return t < 2147483648.0f ? v : -127;
}

// One value of lab_quantize_q4 (lab_native.c:949-950): (int8_t)(x * id +
// 8.5f), two float roundings, the conversion as x86 compiles it (cvttss2si,
// then the low byte), clamped above at 15.
DNX_DEV int q4_value(float x, float id) {
  const float t = x * id + 8.5f;
  const int v = (int8_t)cvt_trunc_x86(t);
  return v > 15 ? 15 : v;
}

// scale = amax / 127 and inv = 1 / scale, both correctly rounded
// (lab_native.c:418-419).
// SiLU(g) * u as the CPU glue rounds it (lib/src/shard.dart:457-461): SiLU
// in double, stored to float, then one float multiply (the product of two
// floats is exact in double, so rounding it once to float is that multiply).
DNX_DEV float silu_mul_exact(float g, float u) {
  const double a = (double)g;
  const float s = (float)(a / (1.0 + exp(-a)));
  return s * u;
}

DNX_DEV float q8_scale(float amax) { return amax / 127.0f; }
DNX_DEV float q8_inv(float scale) { return scale > 0.0f ? 1.0f / scale : 0.0f; }

// Four values quantized with one block's inv, packed little-endian.
DNX_DEV int quant4(float4 v, float inv) {
  // Low bytes of the four values: (x, y) and (z, w) pairs, then the pairs.
  const uint32_t xy = __builtin_amdgcn_perm((uint32_t)quant1(v.y, inv),
                                            (uint32_t)quant1(v.x, inv), 0x0c0c0400u);
  const uint32_t zw = __builtin_amdgcn_perm((uint32_t)quant1(v.w, inv),
                                            (uint32_t)quant1(v.z, inv), 0x0c0c0400u);
  return (int)__builtin_amdgcn_perm(zw, xy, 0x05040100u);
}

// max |v| of four values. The reference keeps amax with `a > amax` from 0
// (lab_native.c:413-417), so NaN never wins; v_max_f32 also returns the
// non-NaN operand, and |-0| = 0 changes nothing.
DNX_DEV float max4abs(float4 v) {
  return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// s_waitcnt immediate (gfx9 encoding): vmcnt <= vm, lgkmcnt <= 0, expcnt
// unconstrained.
constexpr int waitcnt_vm_lgkm0(int vm) { return (vm & 15) | ((vm >> 4) << 14) | (7 << 4); }

// 16-byte load marked non-temporal: weights are streamed once, so they
// should not displace the inputs other workgroups still reuse.
DNX_DEV uint4 load_stream16(const void* p) {
  const u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Raw buffer loads (gfx9 MUBUF): a 128-bit resource in SGPRs holds a base
// address and a byte range; a lane whose offset falls outside the range
// reads zeros without touching memory. That makes bounds checks free and
// branch-free, so the compiler can count outstanding loads exactly.
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ i32x4 dnx_raw_buffer_load_v4i32(i32x4 rsrc, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.v4i32");
__device__ int dnx_raw_buffer_load_i32(i32x4 rsrc, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.i32");
__device__ short dnx_raw_buffer_load_i16(i32x4 rsrc, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.i16");
typedef int i32x2 __attribute__((ext_vector_type(2)));
__device__ i32x2 dnx_raw_buffer_load_v2i32(i32x4 rsrc, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.v2i32");

constexpr int kBufferFlags = 0x00020000;  // gfx9 resource word 3: 32-bit raw data

// A resource for [base, base + bytes). Every field is made wave-uniform.
DNX_DEV i32x4 buffer_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  i32x4 r;
  r.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r.y = __builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));  // stride 0
  r.z = __builtin_amdgcn_readfirstlane((int)bytes);
  r.w = kBufferFlags;
  return r;
}

DNX_DEV uint4 buffer_load16(i32x4 rsrc, int offset) {
  const i32x4 v = dnx_raw_buffer_load_v4i32(rsrc, offset, 0, 0);
  return make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
}

// Cache-policy immediate of a buffer load on gfx950: the non-temporal bit.
// Weights read once per call stream through the caches without being kept:
// on the 350 MB LM head this took the GEMV from 69 to 61 us.
constexpr int kStream = 2;

DNX_DEV uint4 buffer_load16_stream(i32x4 rsrc, int offset) {
  const i32x4 v = dnx_raw_buffer_load_v4i32(rsrc, offset, 0, kStream);
  return make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
}

// 16 bytes per lane from a buffer resource straight into LDS, at lds_addr +
// 16 * lane (gfx950's LDS DMA: no VGPRs; counted by vmcnt like any load).
// lds_addr is the wave-uniform LDS byte address (lds_address below).
// Inline asm on purpose: the compiler cannot tell which part of an LDS
// array a DMA writes, so for its own LDS DMA it waits for every outstanding
// load before the next LDS read of that array. Hidden from it, the caller
// owns the wait: an s_waitcnt vmcnt that covers the DMA, then a barrier,
// before any wave reads the bytes. The compiler's own vmcnt waits do not
// count these loads, which only makes them stricter. It sets M0, which
// LLVM treats as reserved (a clobber of it is ignored): use it only in
// kernels where nothing else reads M0 (gfx950 LDS instructions do not; the
// gemm_f6 kernels' code has no other M0 access).
typedef __attribute__((address_space(3))) void* lds_ptr_t;
DNX_DEV uint32_t lds_address(const void* p) { return (uint32_t)(size_t)(lds_ptr_t)p; }
DNX_DEV void buffer_load16_to_lds(i32x4 rsrc, uint32_t lds_addr, int voffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(lds_addr), "v"(voffset), "s"(rsrc)
               : "memory");
}

// Write-through stores (gfx950 cache policy sc0 sc1): the line goes on to
// memory now instead of staying dirty in the L2 until the end-of-kernel
// write-back. For large outputs written once at a kernel's end (a GEMM's
// 12.6 MB at 512 x 6144) this took the fp6 GEMM from 22.9 to 19.0 us.
// Inline asm: the compiler does not count these in its wait counters, which
// only makes its later waits for its own loads stricter.
DNX_DEV void store_wt(float* p, float v) {
  asm volatile("global_store_dword %0, %1, off sc0 sc1" : : "v"(p), "v"(v) : "memory");
}
DNX_DEV void store_wt4(float* p, float4 v) {
  const f32x4 w = {v.x, v.y, v.z, v.w};
  asm volatile("global_store_dwordx4 %0, %1, off sc0 sc1" : : "v"(p), "v"(w) : "memory");
}

DNX_DEV float4 buffer_load_f4(i32x4 rsrc, int offset) {
  const i32x4 v = dnx_raw_buffer_load_v4i32(rsrc, offset, 0, 0);
  return make_float4(__int_as_float(v.x), __int_as_float(v.y), __int_as_float(v.z),
                     __int_as_float(v.w));
}

// x = p0 + p1 + p2 exactly, each piece a bf16 (top 16 bits of a float):
// truncation keeps 8 significant bits per piece, and the remainders are
// exact float subtractions.
DNX_DEV void split3_bf16(float x, uint32_t& p0, uint32_t& p1, uint32_t& p2) {
  const uint32_t b0 = __float_as_uint(x) & 0xffff0000u;
  const float r = x - __uint_as_float(b0);
  const uint32_t b1 = __float_as_uint(r) & 0xffff0000u;
  const float r2 = r - __uint_as_float(b1);
  p0 = b0 >> 16;
  p1 = b1 >> 16;
  p2 = __float_as_uint(r2) >> 16;
}

// Block scales applied by an MFMA. The product s = sx * sw of a 32 x 32
// tile comes from one v_mfma_f32_32x32x8_bf16 used as an outer product:
// each scale is split into three bf16 pieces and six of the products
// x_i * w_j (i + j <= 2) sit in the instruction's K slots; the dropped
// terms are below 3 * 2^-24 relative. Scale pieces in the outer-product
// MFMA's K slots. Lanes 0..31 hold slots
// 0..7 of their row (A) or column (B), lanes 32..63 slots 8..15; only the
// first four slots of each half are used:
//   A half 0: x0 x0 x1 0   B half 0: w0 w1 w0 0   -> x0w0 + x0w1 + x1w0
//   A half 1: x0 x1 x2 0   B half 1: w2 w1 w0 0   -> x0w2 + x1w1 + x2w0
DNX_DEV uint2 a_scale_half0(uint32_t p0, uint32_t p1, uint32_t) {
  return make_uint2(p0 | (p0 << 16), p1);
}
DNX_DEV uint2 a_scale_half1(uint32_t p0, uint32_t p1, uint32_t p2) {
  return make_uint2(p0 | (p1 << 16), p2);
}
DNX_DEV uint2 b_scale_half0(uint32_t p0, uint32_t p1, uint32_t) {
  return make_uint2(p0 | (p1 << 16), p0);
}
DNX_DEV uint2 b_scale_half1(uint32_t p0, uint32_t p1, uint32_t p2) {
  return make_uint2(p2 | (p1 << 16), p0);
}

DNX_DEV float bf16_to_float(uint16_t p) { return __uint_as_float((uint32_t)p << 16); }

DNX_DEV float half_bits_to_float(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

// argmaxToken (lib/src/sampler.dart:137-143): the first index of the
// maximum. A value becomes an order-preserving key (-0 == +0, NaN below
// everything) packed with the complemented index, so that one unsigned max
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

}  // namespace dnx
