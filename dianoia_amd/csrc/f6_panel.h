// The fp6 GEMMs' activation panel: its layout, and the quantization of one
// (token, block) into it by four lanes, shared by the panel quantizer
// (gemm_f6.hip) and the kernels that write the panel of what they produce
// (the prefill norms in layers.hip, SiLU * up in gemm_f6.hip), so that every
// writer makes the same bytes.
#pragma once

#include "common.h"

namespace dnx {

constexpr int kTokens = 32;      // tokens per panel group (one MFMA tile)
constexpr int kRecF = 0;         // [2 halves][64 lanes][16 B]: fp6 codes + operand dwords
constexpr int kRecHalf = 1024;   // the second 16 bytes of every lane's record
constexpr int kRecC = 2048;      // 2 halves x 16 floats: the MFMA's C input
constexpr int kRec = 2176;       // panel bytes per (32 tokens, block)

inline int64_t f6_panel_bytes(int64_t n, int64_t cols) {
  return (n + kTokens - 1) / kTokens * (cols / kBlock) * kRec;
}

template <int F>
DNX_DEV void put_field(uint32_t* d, uint32_t c) {
  constexpr int bit = 6 * F, wd = bit >> 5, sh = bit & 31;
  d[wd] |= c << sh;
  if constexpr (sh > 26) d[wd + 1] |= c >> (32 - sh);
}

// Fields (within their 96-bit half) of a lane's values 0..7: pattern 0 for
// lanes 0, 1 (values 0-7, 8-15), pattern 1 for lanes 2, 3 (16-23, 24-31).
DNX_DEV void place_pattern0(uint32_t* d, const uint32_t* c) {
  put_field<0>(d, c[0]); put_field<12>(d, c[1]); put_field<8>(d, c[2]); put_field<4>(d, c[3]);
  put_field<11>(d, c[4]); put_field<7>(d, c[5]); put_field<3>(d, c[6]); put_field<15>(d, c[7]);
}
DNX_DEV void place_pattern1(uint32_t* d, const uint32_t* c) {
  put_field<6>(d, c[0]); put_field<2>(d, c[1]); put_field<14>(d, c[2]); put_field<10>(d, c[3]);
  put_field<1>(d, c[4]); put_field<13>(d, c[5]); put_field<9>(d, c[6]); put_field<5>(d, c[7]);
}

// One (token, block) of fp32 values quantized as lab_quantize_q8 does (the
// same xq and scale bits as dnx_quantize_q8) into its panel entries, by the
// four consecutive lanes of a quad (all four must run this together: the
// block's amax and sum(xq) come by DPP over the quad). Lane j holds values
// 8j .. 8j+7 (v0, v1); r is the token's place in its group of 32, rec the
// (group, block) record. In the operand order those 8 values occupy 8
// fields of one 96-bit half (j & 1) of the 192-bit code field, at the places
// of pattern j >> 1; the two lanes of a half OR their bits together, and
// each lane then stores one 16 bytes of the token's two lane records (lane
// 0 also the C value).
DNX_DEV void panel4_lane(float4 v0, float4 v1, int j, int r, uint8_t* rec) {
  float amax = fmaxf(max4abs(v0), max4abs(v1));
  amax = fmaxf(amax, dppf<kQuadXor1>(amax));
  amax = fmaxf(amax, dppf<kQuadXor2>(amax));
  const float scale = q8_scale(amax);
  const float inv = q8_inv(scale);
  const float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
  uint32_t ch[8], cl[8];
  int sum = 0;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int xq = quant1(vv[i], inv);
    sum += xq;
    const uint32_t a = (uint32_t)(xq < 0 ? -xq : xq);
    const uint32_t sg = xq < 0 ? 0x20u : 0u;
    ch[i] = sg | (a >> 3);
    cl[i] = sg | (a & 7u);
  }
  sum += dpp<kQuadXor1>(sum);
  sum += dpp<kQuadXor2>(sum);
  uint32_t h0[3] = {0, 0, 0}, h1[3] = {0, 0, 0}, l0[3] = {0, 0, 0}, l1[3] = {0, 0, 0};
  place_pattern0(h0, ch);
  place_pattern1(h1, ch);
  place_pattern0(l0, cl);
  place_pattern1(l1, cl);
  const bool p1 = (j >> 1) != 0;
  uint32_t hw[3], lw[3];
#pragma unroll
  for (int d = 0; d < 3; d++) {
    hw[d] = p1 ? h1[d] : h0[d];
    lw[d] = p1 ? l1[d] : l0[d];
    hw[d] |= (uint32_t)dpp<kQuadXor2>((int)hw[d]);   // the other lane of this half
    lw[d] |= (uint32_t)dpp<kQuadXor2>((int)lw[d]);
  }
  // Lanes 0, 2 hold dwords 0-2 of the field, lanes 1, 3 dwords 3-5; the
  // first 16 bytes of a record also need dword 3 (the other half's first).
  const uint32_t h3 = (uint32_t)dpp<kQuadXor1>((int)hw[0]);
  const uint32_t l3 = (uint32_t)dpp<kQuadXor1>((int)lw[0]);
  // scale = 2^e * mant, mant in [1, 2) (a subnormal keeps e = -126, mant <
  // 1); mant = p0 + p1 + p2 exactly in fp16 pieces; E8M0 bytes 2^(6 + e)
  // for the h codes (value h / 8 -> 8 h), 2^(3 + e) for the l codes.
  const uint32_t bits = __float_as_uint(scale);
  const int ef = (int)((bits >> 23) & 0xff);
  int e = ef == 0 ? -126 : ef - 127;
  float mant = ef == 0 ? scale * 0x1p126f : __uint_as_float((bits & 0x807fffffu) | 0x3f800000u);
  if (scale == 0.0f) {
    e = 0;
    mant = 0.0f;
  }
  const _Float16 p0 = (_Float16)mant;
  const float r1 = mant - (float)p0;
  const _Float16 pp1 = (_Float16)r1;
  const _Float16 p2 = (_Float16)(r1 - (float)pp1);
  const uint32_t sh_h = (uint32_t)(127 + 6 + e), sh_l = (uint32_t)(127 + 3 + e);
  const uint32_t s0 = (uint32_t)__builtin_bit_cast(uint16_t, p0) |
                      ((uint32_t)__builtin_bit_cast(uint16_t, pp1) << 16);
  const uint32_t s1 = sh_h | ((uint32_t)__builtin_bit_cast(uint16_t, p2) << 16);
  // Lane 0: h codes, first half; 1: h codes, second half + operand; 2, 3
  // the same for the l codes.
  uint4 o;
  if (j == 0) o = make_uint4(hw[0], hw[1], hw[2], h3);
  else if (j == 1) o = make_uint4(hw[1], hw[2], s0, s1);
  else if (j == 2) o = make_uint4(lw[0], lw[1], lw[2], l3);
  else o = make_uint4(lw[1], lw[2], 0u, sh_l);
  const int lane_rec = (j & 2) ? 32 + r : r;
  *(uint4*)(rec + kRecF + (j & 1) * kRecHalf + lane_rec * 16) = o;
  if (j == 0) {
    const float c = sum == 0 ? 0.0f : ldexpf((float)(-8 * sum), e);
    *(float*)(rec + kRecC + ((((r >> 2) & 1) * 16 + (r >> 3) * 4 + (r & 3)) * 4)) = c;
  }
}

}  // namespace dnx
