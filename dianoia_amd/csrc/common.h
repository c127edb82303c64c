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
DNX_DEV int quant1(float x, float inv) {
  float t = x * inv;
  t = t < 0.0f ? t - 0.5f : t + 0.5f;
  const int v = cvt_trunc_x86(t);
  return v > 127 ? 127 : v < -127 ? -127 : v;
}

// scale = amax / 127 and inv = 1 / scale, both correctly rounded
// (lab_native.c:418-419).
DNX_DEV float q8_scale(float amax) { return amax / 127.0f; }
DNX_DEV float q8_inv(float scale) { return scale > 0.0f ? 1.0f / scale : 0.0f; }

// Four values quantized with one block's inv, packed little-endian.
DNX_DEV int quant4(float4 v, float inv) {
  return (quant1(v.x, inv) & 0xff) | ((quant1(v.y, inv) & 0xff) << 8) |
         ((quant1(v.z, inv) & 0xff) << 16) | ((quant1(v.w, inv) & 0xff) << 24);
}

// max |v| of four values. The reference keeps amax with `a > amax` from 0
// (lab_native.c:413-417), so NaN never wins; v_max_f32 also returns the
// non-NaN operand, and |-0| = 0 changes nothing.
DNX_DEV float max4abs(float4 v) {
  return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
}

DNX_DEV float bf16_to_float(uint16_t p) { return __uint_as_float((uint32_t)p << 16); }

DNX_DEV float half_bits_to_float(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

}  // namespace dnx
