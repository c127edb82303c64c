// Prefill / encoder GEMM for Q4 weights on the gfx950 fp6 matrix cores:
//   y[m][r] = sum_b sx[m][b] * sw[r][b] * D_b[m][r],
//   D_b[m][r] = sum over block b of xq[m][k] * (q[r][k] - 8)   (exact integer)
// with xq, sx exactly lab_quantize_q8's (lab_native.c:407-429) and the
// product of lab_gemm_q4 mode 1 (lab_native.c:1059-1080) up to the fp32
// rounding of the scaled sum.
//
// The block dot on one scaled fp6 MFMA. v_mfma_scale_f32_32x32x64_f8f6f4
// multiplies 32 x 64 by 64 x 32 operands of 6-bit floats, each lane's 32
// values carrying its own power-of-two (E8M0) scale, in 33 clocks: twice the
// int8 MFMA's multiply-adds per clock. Both factors of a block dot are
// exact in it:
//   * a Q4 nibble q in 0..15 is the fp6 E2M3 code of q / 8 (codes 0..15 are
//     the subnormals and the first binade, value = code / 8), so a weight
//     needs no arithmetic beyond moving its 4 bits into a 6-bit field;
//   * |xq| <= 127 splits as 8 h + l (h in 0..15, l in 0..7), both E2M3
//     codes with the sign of xq. The 64 K slots hold the block twice:
//     slots 0..31 pair the h codes (scale 2^6) with the weights (scale
//     2^3), slots 32..63 the l codes (scale 2^3) with the weights again;
//   * the -8 of q - 8 enters as the MFMA's C input, -8 * sum(xq) per token.
// Every product and partial sum is an integer below 2^24, so D_b is exact.
// The activation scale's exponent rides in the same E8M0 scale (2^e_x),
// leaving mant(sx) in [1, 2): the scale product s = mant(sx) * sw comes from
// one v_mfma_f32_32x32x8_f16 used as an outer product (mant(sx) as three
// fp16 pieces that sum to it exactly, sw as its own fp16 bits), and the
// epilogue is one fma per output per block, blocks in order.
// Per 32 x 32 tile and block: 33 + 32 MFMA clocks and 16 fma, against 64 + 32
// MFMA clocks for the fp16 form (gemm_f16.hip).
//
// Operands.
//   Activations: a "f6 panel" written by the quantizer below from fp32 x
//   (or from xq + xsc), per 32 tokens and block (kRec bytes): each MFMA
//   lane's 32-byte record (6 dwords of fp6 codes, then the scale MFMA's
//   four fp16 operand slots, the E8M0 scale byte riding in the third: see
//   write_f6_entries) split into two 1 KB halves, [half][64 lanes][16 B],
//   so that each of a wave's two 16-byte loads reads 1 KB contiguous; then
//   the 32 tokens' C values. A wave loads its tokens' records straight into
//   registers, four blocks ahead; the C values are staged through LDS with
//   the weights.
//   Weights: staged through LDS once per workgroup, shared by its 8 waves:
//   each 16-byte Q4 block becomes 6 dwords of fp6 codes with 16 VALU
//   operations (kFieldK below is the resulting order of the weights in the
//   fields; the panel writes the activations in the same order), next to
//   the scale MFMA's operand (sw, sw, sw, 0).
//
// Workgroup: 512 threads, 128 tokens x SN * 32 weight rows. Wave w takes
// the 32 tokens (w % 4) and every other block (parity w / 4), so the two
// waves of a SIMD work on the same outputs and one hides the other's
// latencies; their sums are added at the end through LDS in a fixed order.

#include <mutex>

#include "common.h"
#include "dnx_kernels.h"
#include "f6_panel.h"

using namespace dnx;

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));

constexpr int kPanelThreads = 256;
constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;

// The weight index held by each of a block's 32 fp6 fields after
// q4_to_f6 (below) and so the order in which the panel lays out the
// activations: field f of the 192-bit operand holds weight kFieldK[f].
__constant__ const int8_t kFieldK[32] = {0,  20, 17, 6,  3,  23, 16, 5,  2,  22, 19,
                                         4,  1,  21, 18, 7,  8,  28, 25, 14, 11, 31,
                                         24, 13, 10, 30, 27, 12, 9,  29, 26, 15};
constexpr int8_t kFieldKHost[32] = {0,  20, 17, 6,  3,  23, 16, 5,  2,  22, 19,
                                    4,  1,  21, 18, 7,  8,  28, 25, 14, 11, 31,
                                    24, 13, 10, 30, 27, 12, 9,  29, 26, 15};

// Two dwords of Q4 nibbles (a: weights 4j.., b: the next dword) -> three
// dwords of 6-bit fields, each nibble under two zero bits (the E2M3 code of
// q / 8). Nibbles of a at bits 0, 12, 24 / 4, 16, 28 / 8, 20 stay where
// they are in the first / second / third output dword; nibbles of b move up
// by two bits (4 -> 6, ..., 28 -> 30 with its top half carried to the next
// dword's bits 0-1).
DNX_DEV void q4_group_to_f6(uint32_t a, uint32_t b, uint32_t* o) {
  const uint32_t t = b << 2;
  o[0] = (a & 0x0F00F00Fu) | (t & 0xC03C03C0u);
  o[1] = (a & 0xF00F00F0u) | (t & 0x03C03C00u) | (b >> 30);
  o[2] = (a & 0x00F00F00u) | (t & 0x3C03C03Cu);
}

// ---------------------------------------------------------------- the panel

// One (token, block): its 32 quantized values -> the panel record entries
// of lane (token, 0) (h codes), lane (token, 1) (l codes), the scale
// MFMA operand and the C value.
DNX_DEV void write_f6_entries(uint8_t* rec, int r, const int* xq, float scale) {
  int sum = 0;
#pragma unroll
  for (int k = 0; k < 32; k++) sum += xq[k];
  // scale = 2^e * mant, mant in [1, 2); a subnormal scale keeps e = -126
  // and mant < 1 (its products lie far below any fp32 result's ulp).
  const uint32_t bits = __float_as_uint(scale);
  const int ef = (int)((bits >> 23) & 0xff);
  int e = ef == 0 ? -126 : ef - 127;
  float mant = ef == 0 ? scale * 0x1p126f : __uint_as_float((bits & 0x807fffffu) | 0x3f800000u);
  if (scale == 0.0f) {
    e = 0;
    mant = 0.0f;
  }
  // mant = p0 + p1 + p2 exactly (for mant in [1, 2): 11 + 11 + 2 bits).
  const _Float16 p0 = (_Float16)mant;
  const float r1 = mant - (float)p0;
  const _Float16 p1 = (_Float16)r1;
  const _Float16 p2 = (_Float16)(r1 - (float)p1);
  uint32_t hw[6] = {0, 0, 0, 0, 0, 0}, lw[6] = {0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int f = 0; f < 32; f++) {
    const int v = xq[kFieldKHost[f]];
    const uint32_t a = (uint32_t)(v < 0 ? -v : v);
    const uint32_t sg = v < 0 ? 0x20u : 0u;
    const uint32_t hc = sg | (a >> 3), lc = sg | (a & 7u);
    const int bit = 6 * f, wd = bit >> 5, sh = bit & 31;
    hw[wd] |= hc << sh;
    lw[wd] |= lc << sh;
    if (sh > 26) {  // the field runs into the next dword
      hw[wd + 1] |= hc >> (32 - sh);
      lw[wd + 1] |= lc >> (32 - sh);
    }
  }
  // E8M0 scales: 2^(6 + e) for the h codes (value h / 8 -> 8 h), 2^(3 + e)
  // for the l codes.
  const uint32_t sh_h = (uint32_t)(127 + 6 + e), sh_l = (uint32_t)(127 + 3 + e);
  // Dwords 6-7: the scale MFMA's fp16 slots (p0, p1, E8M0 byte, p2) on the
  // h lanes and (0, 0, E8M0 byte, 0) on the l lanes. The weights' slots are
  // (sw, sw, 0, sw), so the byte's slot (a finite subnormal) meets a zero,
  // and the fp6 MFMA reads the byte as its scale operand (byte 0 of dword 7).
  const uint32_t s0 = (uint32_t)__builtin_bit_cast(uint16_t, p0) |
                      ((uint32_t)__builtin_bit_cast(uint16_t, p1) << 16);
  const uint32_t s1 = sh_h | ((uint32_t)__builtin_bit_cast(uint16_t, p2) << 16);
  // Lane r holds the h codes of token r, lane 32 + r its l codes.
  uint8_t* fh = rec + kRecF + r * 16;
  uint8_t* fl = rec + kRecF + (32 + r) * 16;
  *(uint4*)fh = make_uint4(hw[0], hw[1], hw[2], hw[3]);
  *(uint4*)(fh + kRecHalf) = make_uint4(hw[4], hw[5], s0, s1);
  *(uint4*)fl = make_uint4(lw[0], lw[1], lw[2], lw[3]);
  *(uint4*)(fl + kRecHalf) = make_uint4(lw[4], lw[5], 0u, sh_l);
  // C of output row r: lanes of half (r / 4) % 2 hold it at 4 (r / 8) + r % 4.
  const float c = sum == 0 ? 0.0f : ldexpf((float)(-8 * sum), e);
  *(float*)(rec + kRecC + ((((r >> 2) & 1) * 16 + (r >> 3) * 4 + (r & 3)) * 4)) = c;
}

// fp32 x [n][cols] -> f6 panel [groups][B][kRec]: lab_quantize_q8 of each
// (token, block) (the same xq and scale bits as dnx_quantize_q8), then its
// panel entries, with four lanes per (token, block) (panel4_lane; a lane
// per block spent its time packing 32 values in series). Tokens past n get
// zero records.
__global__ void __launch_bounds__(kPanelThreads) quantize_f6_panel4_kernel(
    const float* __restrict__ x, uint8_t* __restrict__ panel, int n, int cols, int groups) {
  const int B = cols / kBlock;
  const int64_t total = (int64_t)groups * B * kTokens * 4;  // whole quads
  for (int64_t idx = (int64_t)blockIdx.x * kPanelThreads + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * kPanelThreads) {
    const int j = (int)(idx & 3);
    const int64_t q = idx >> 2;
    const int r = (int)(q & (kTokens - 1));
    const int64_t gb = q >> 5;
    const int b = (int)(gb % B);
    const int g = (int)(gb / B);
    const int m = g * kTokens + r;
    const bool live = m < n;
    const float4* src = (const float4*)(x + (int64_t)(live ? m : 0) * cols + b * kBlock + 8 * j);
    const float4 v0 = live ? src[0] : make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 v1 = live ? src[1] : make_float4(0.f, 0.f, 0.f, 0.f);
    panel4_lane(v0, v1, j, r, panel + gb * kRec);
  }
}

// SiLU(g) * u in place (swiglu_kernel's values) over g, u [n][cols], and
// the panel of the result for the matmul that reads it (a prefill chunk's
// down projection): one pass, four lanes per (token, block), each lane 8
// consecutive values. Tokens past n get zero records.
__global__ void __launch_bounds__(kPanelThreads) swiglu_f6panel_kernel(
    float* __restrict__ g, const float* __restrict__ u, uint8_t* __restrict__ panel, int n,
    int cols, int groups) {
  const int B = cols / kBlock;
  const int64_t total = (int64_t)groups * B * kTokens * 4;  // whole quads
  for (int64_t idx = (int64_t)blockIdx.x * kPanelThreads + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * kPanelThreads) {
    const int j = (int)(idx & 3);
    const int64_t q = idx >> 2;
    const int r = (int)(q & (kTokens - 1));
    const int64_t gb = q >> 5;
    const int b = (int)(gb % B);
    const int m = (int)(gb / B) * kTokens + r;
    float4 h0 = make_float4(0.f, 0.f, 0.f, 0.f), h1 = h0;
    if (m < n) {
      float4* gp = (float4*)(g + (int64_t)m * cols + b * kBlock + 8 * j);
      const float4* up = (const float4*)(u + (int64_t)m * cols + b * kBlock + 8 * j);
      const float4 g0 = gp[0], g1 = gp[1], u0 = up[0], u1 = up[1];
      h0 = make_float4(silu_mul_exact(g0.x, u0.x), silu_mul_exact(g0.y, u0.y),
                       silu_mul_exact(g0.z, u0.z), silu_mul_exact(g0.w, u0.w));
      h1 = make_float4(silu_mul_exact(g1.x, u1.x), silu_mul_exact(g1.y, u1.y),
                       silu_mul_exact(g1.z, u1.z), silu_mul_exact(g1.w, u1.w));
      gp[0] = h0;
      gp[1] = h1;
    }
    panel4_lane(h0, h1, j, r, panel + gb * kRec);
  }
}

// The same panel from already quantized xq int8 [n][cols] + xsc [n][cols/32],
// one thread per (token, block).
__global__ void __launch_bounds__(kPanelThreads) pack_f6_panel_kernel(
    const int8_t* __restrict__ xq, const float* __restrict__ xsc, uint8_t* __restrict__ panel,
    int n, int cols, int groups) {
  const int B = cols / kBlock;
  const int64_t total = (int64_t)groups * B * kTokens;
  for (int64_t idx = (int64_t)blockIdx.x * kPanelThreads + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * kPanelThreads) {
    const int r = (int)(idx & (kTokens - 1));
    const int64_t gb = idx >> 5;
    const int b = (int)(gb % B);
    const int g = (int)(gb / B);
    const int m = g * kTokens + r;
    int q[32];
    float scale = 0.0f;
    if (m < n) {
      const uint4* src = (const uint4*)(xq + (int64_t)m * cols + b * kBlock);
      const uint4 lo = src[0], hi = src[1];
      const uint32_t w[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
      for (int k = 0; k < 32; k++) q[k] = (int)(int8_t)(w[k >> 2] >> (8 * (k & 3)));
      scale = xsc[(int64_t)m * B + b];
    } else {
#pragma unroll
      for (int k = 0; k < 32; k++) q[k] = 0;
    }
    write_f6_entries(panel + gb * kRec, r, q, scale);
  }
}

// ----------------------------------------------------------------- the GEMM

constexpr int kTileM = 4;   // 32-token groups per workgroup

// Bytes of LDS the epilogue below uses: both parities' partial tiles of the
// workgroup, [token group][parity][32 tokens][BN + 4 floats].
template <int SN>
constexpr int epilogue_lds_bytes() {
  return kTileM * 2 * kTokens * (SN * 32 + 4) * 4;
}

// The workgroup's 128 x BN outputs: every wave puts its partial sums (one
// parity of K) into LDS in [token][row] order, then every wave adds the two
// parities (even + odd, a fixed order) for 1/8 of the outputs and stores
// them 16 bytes per lane, consecutive lanes along a token's row (a row of
// BN floats is BN / 4 lanes), write-through (store_wt4). `vec` (uniform): out and N allow 16-byte
// stores; otherwise each value is stored alone. Called by all waves after
// the K loop's last barrier (the partials overwrite the stage buffers).
template <int SN>
DNX_DEV void store_tile_sums(uint8_t* lds, const v16f* acc, int wave, int lane, int m0, int n0,
                             int M, int N, float* out, bool vec) {
  constexpr int BN = SN * 32;
  constexpr int RS = BN + 4;  // row stride in floats (spreads the two rows a write covers)
  constexpr int C4 = BN / 4;  // float4 per token row
  constexpr int PER = kTileM * kTokens * C4 / kWaves / 64;
  static_assert(kTileM * kTokens * C4 % (kWaves * 64) == 0, "whole float4 per lane");
  const int mg = wave & 3, kp = wave >> 2;
  float* part = (float*)lds + (size_t)(mg * 2 + kp) * kTokens * RS;
#pragma unroll
  for (int j = 0; j < SN; j++)
#pragma unroll
    for (int v = 0; v < 16; v++) {
      const int m = (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
      part[m * RS + j * 32 + (lane & 31)] = acc[j][v];
    }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < PER; it++) {
    const int idx = (wave * PER + it) * 64 + lane;
    const int tok = idx / C4, c4 = idx - tok * C4;
    const float* e = (const float*)lds + ((size_t)((tok >> 5) * 2) * kTokens + (tok & 31)) * RS + c4 * 4;
    const float4 a = *(const float4*)e;
    const float4 b = *(const float4*)(e + kTokens * RS);
    const int m = m0 + tok, r = n0 + c4 * 4;
    if (m >= M || r >= N) continue;
    const float4 o = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
    float* dst = out + (size_t)m * N + r;
    if (vec) {
      store_wt4(dst, o);
    } else {
      store_wt(dst, o.x);
      if (r + 1 < N) store_wt(dst + 1, o.y);
      if (r + 2 < N) store_wt(dst + 2, o.z);
      if (r + 3 < N) store_wt(dst + 3, o.w);
    }
  }
}

// The same sums with half the LDS (wide tiles whose two parities' partials
// would not fit a CU's 160 KB): the parity-1 waves put their partials into
// LDS, the parity-0 waves add theirs to them in place (the same sum,
// parity 0 + parity 1), then every wave stores as above.
template <int SN>
constexpr int epilogue_lds_bytes_inplace() {
  return kTileM * kTokens * (SN * 32 + 4) * 4;
}

template <int SN>
DNX_DEV void store_tile_sums_inplace(uint8_t* lds, const v16f* acc, int wave, int lane, int m0,
                                     int n0, int M, int N, float* out, bool vec) {
  constexpr int BN = SN * 32;
  constexpr int RS = BN + 4;
  constexpr int C4 = BN / 4;
  constexpr int PER = kTileM * kTokens * C4 / kWaves / 64;
  static_assert(kTileM * kTokens * C4 % (kWaves * 64) == 0, "whole float4 per lane");
  const int mg = wave & 3, kp = wave >> 2;
  float* part = (float*)lds + (size_t)mg * kTokens * RS;
  if (kp == 1) {
#pragma unroll
    for (int j = 0; j < SN; j++)
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int m = (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
        part[m * RS + j * 32 + (lane & 31)] = acc[j][v];
      }
  }
  __syncthreads();
  if (kp == 0) {
#pragma unroll
    for (int j = 0; j < SN; j++)
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int m = (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
        float* e = &part[m * RS + j * 32 + (lane & 31)];
        *e = acc[j][v] + *e;
      }
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < PER; it++) {
    const int idx = (wave * PER + it) * 64 + lane;
    const int tok = idx / C4, c4 = idx - tok * C4;
    const float4 o = *(const float4*)((const float*)lds + (size_t)tok * RS + c4 * 4);
    const int m = m0 + tok, r = n0 + c4 * 4;
    if (m >= M || r >= N) continue;
    float* dst = out + (size_t)m * N + r;
    if (vec) {
      store_wt4(dst, o);
    } else {
      store_wt(dst, o.x);
      if (r + 1 < N) store_wt(dst + 1, o.y);
      if (r + 2 < N) store_wt(dst + 2, o.z);
      if (r + 3 < N) store_wt(dst + 3, o.w);
    }
  }
}

// The sums of a 64-token tile whose 8 waves are 2 token groups x 4 block
// parities: every wave puts its partials into LDS, then every wave adds the
// four parities (in parity order) for 1/8 of the outputs and stores them as
// store_tile_sums does.
template <int SN>
constexpr int epilogue_lds_bytes_par4() {
  return 2 * 4 * kTokens * (SN * 32 + 4) * 4;
}

template <int SN>
DNX_DEV void store_tile_sums_par4(uint8_t* lds, const v16f* acc, int wave, int lane, int m0,
                                  int n0, int M, int N, float* out, bool vec) {
  constexpr int BN = SN * 32;
  constexpr int RS = BN + 4;
  constexpr int C4 = BN / 4;
  constexpr int PER = 2 * kTokens * C4 / kWaves / 64;
  static_assert(2 * kTokens * C4 % (kWaves * 64) == 0, "whole float4 per lane");
  const int mg = wave & 1, kp = wave >> 1;
  float* part = (float*)lds + (size_t)(mg * 4 + kp) * kTokens * RS;
#pragma unroll
  for (int j = 0; j < SN; j++)
#pragma unroll
    for (int v = 0; v < 16; v++) {
      const int m = (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
      part[m * RS + j * 32 + (lane & 31)] = acc[j][v];
    }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < PER; it++) {
    const int idx = (wave * PER + it) * 64 + lane;
    const int tok = idx / C4, c4 = idx - tok * C4;
    const float* e = (const float*)lds + ((size_t)((tok >> 5) * 4) * kTokens + (tok & 31)) * RS + c4 * 4;
    float4 o = *(const float4*)e;
#pragma unroll
    for (int q = 1; q < 4; q++) {
      const float4 b = *(const float4*)(e + q * kTokens * RS);
      o = make_float4(o.x + b.x, o.y + b.y, o.z + b.z, o.w + b.w);
    }
    const int m = m0 + tok, r = n0 + c4 * 4;
    if (m >= M || r >= N) continue;
    float* dst = out + (size_t)m * N + r;
    if (vec) {
      store_wt4(dst, o);
    } else {
      store_wt(dst, o.x);
      if (r + 1 < N) store_wt(dst + 1, o.y);
      if (r + 2 < N) store_wt(dst + 2, o.z);
      if (r + 3 < N) store_wt(dst + 3, o.w);
    }
  }
}

struct F6Params {
  const uint8_t* qs;       // Q4 nibbles [rows][cols/2]
  const uint16_t* scales;  // fp16 bits [rows][cols/32]
  const uint8_t* panel;    // f6 panel of the n tokens
  float* y;                // [n][rows]
  float* part;             // split partials [splits][n][rows], or null
  int rows, cols, n;
  int tiles_m, tiles;      // workgroup tiles (128 tokens x BN rows) of one K split
  int split_blocks;        // blocks per K split (blockIdx.y), a multiple of kKB
  int vec;                 // the output allows 16-byte stores (16-byte aligned, rows % 4 == 0)
};

constexpr int kKB = 16;     // blocks per stage
constexpr int kRecW = 32;   // LDS bytes per staged (row, block): 6 fp6 dwords + 2 operand dwords
constexpr int kRing = 4;    // activation records in flight per wave (its next blocks)

template <int SN>
__global__ void __launch_bounds__(kThreads) gemm_f6_q4_kernel(F6Params p) {
  constexpr int BN = SN * 32;
  constexpr int RS = kKB * kRecW + 16;          // LDS bytes per staged weight row (bank spread)
  constexpr int kW = BN * RS;                   // staged weights of a stage
  constexpr int kC = kTileM * kKB * 128;        // staged C inputs of a stage
  constexpr int kStage = kW + kC;
  constexpr int kPairs = BN * kKB;              // (row, block) per stage
  constexpr int PP = (kPairs + kThreads - 1) / kThreads;
  constexpr int kCPieces = kC / 16;
  constexpr int CP = (kCPieces + kThreads - 1) / kThreads;
  constexpr int kLds = 2 * kStage > epilogue_lds_bytes<SN>() ? 2 * kStage : epilogue_lds_bytes<SN>();
  static_assert((kKB / 2) % kRing == 0, "ring slots must repeat each stage");
  __shared__ __align__(16) uint8_t lds[kLds];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int mg = wave & 3, kp = wave >> 2;
  const int K = p.cols, B = K / kBlock, M = p.n, N = p.rows;

  // XCD-aware order: workgroups are dealt round-robin to the 8 XCDs, so
  // workgroup i runs tile (i % 8) * (tiles / 8) + i / 8 and each XCD walks a
  // contiguous run of tiles (all token groups of consecutive weight rows).
  const int i = blockIdx.x;
  const int t = (p.tiles % 8 == 0) ? (i % 8) * (p.tiles / 8) + i / 8 : i;
  const int tm = t % p.tiles_m, tn = t / p.tiles_m;
  const int n0 = tn * BN;
  const int groups = (M + kTokens - 1) / kTokens;
  const int g = tm * kTileM + mg;                // this wave's token group
  const int b_begin = blockIdx.y * p.split_blocks;
  const int b_end = min(B, b_begin + p.split_blocks);
  const int stages = (b_end - b_begin + kKB - 1) / kKB;

  const i32x4 rpanel = buffer_rsrc(p.panel, (uint32_t)((size_t)groups * B * kRec));
  const i32x4 rqs = buffer_rsrc(p.qs, (uint32_t)((size_t)N * (K / 2)));
  const i32x4 rsc = buffer_rsrc(p.scales, (uint32_t)((size_t)N * B * 2));

  // ---- staging of a stage: weights as (row j, block kb) pairs, kb fastest
  // (coalesced rows), and the C inputs of the workgroup's 4 token groups.
  // Offsets are recomputed per stage from the thread index (few registers).
  uint4 rq[PP];
  short rs[PP];
  float4 rc[CP];
  // Loads of stage s; blocks past this split's end read zeros.
  auto load_stage = [&](int s) {
    const int b0 = b_begin + s * kKB;
#pragma unroll
    for (int e = 0; e < PP; e++) {
      const int q = e * kThreads + tid;
      const int j = q / kKB, b = b0 + (q - j * kKB);
      const bool ok = q < kPairs && n0 + j < N && b < b_end;
      rq[e] = buffer_load16(rqs, ok ? (n0 + j) * (K / 2) + b * 16 : -64);
      rs[e] = dnx_raw_buffer_load_i16(rsc, ok ? ((n0 + j) * B + b) * 2 : -4, 0, 0);
    }
#pragma unroll
    for (int e = 0; e < CP; e++) {
      const int q = e * kThreads + tid;        // 16-byte piece: (group, block, piece of 8)
      const int gg = q / (kKB * 8), b = b0 + (q / 8) % kKB;
      const bool ok = q < kCPieces && tm * kTileM + gg < groups && b < b_end;
      rc[e] = buffer_load_f4(rpanel,
                             ok ? ((tm * kTileM + gg) * B + b) * kRec + kRecC + (q % 8) * 16 : -64);
    }
  };
  auto store_stage = [&](int buf) {
    uint8_t* base = lds + buf * kStage;
#pragma unroll
    for (int e = 0; e < PP; e++) {
      const int q = e * kThreads + tid;
      if (q >= kPairs) continue;
      const int j = q / kKB, kb = q - j * kKB;
      uint32_t f[6];
      q4_group_to_f6(rq[e].x, rq[e].y, f);
      q4_group_to_f6(rq[e].z, rq[e].w, f + 3);
      const uint32_t sw = (uint32_t)(uint16_t)rs[e];
      uint4* d = (uint4*)(base + j * RS + kb * kRecW);
      d[0] = make_uint4(f[0], f[1], f[2], f[3]);
      // The scale MFMA's weight slots (sw, sw, 0, sw).
      d[1] = make_uint4(f[4], f[5], sw | (sw << 16), sw << 16);
    }
#pragma unroll
    for (int e = 0; e < CP; e++) {
      const int q = e * kThreads + tid;
      if (q >= kCPieces) continue;
      const int gg = q / (kKB * 8), kb = (q / 8) % kKB;
      *(float4*)(base + kW + (gg * kKB + kb) * 128 + (q % 8) * 16) = rc[e];
    }
  };

  // ---- this wave's activation lane records, kRing blocks ahead
  const bool live = g < groups;
  // Out-of-range blocks (past this split, or a token group past n) read
  // zeros through an offset past the resource. The select is arithmetic:
  // a branch here splits the loop into blocks the scheduler cannot cross.
  auto load_a = [&](int b, i32x4& lo, i32x4& hi) {
    const int ok = -(int)(live & (b < b_end));
    const int base = (((g * B + b) * kRec + kRecF) & ok) | (~ok & -(1 << 20));
    lo = dnx_raw_buffer_load_v4i32(rpanel, base + lane * 16, 0, 0);
    hi = dnx_raw_buffer_load_v4i32(rpanel, base + kRecHalf + lane * 16, 0, 0);
  };

  v16f acc[SN];
#pragma unroll
  for (int j = 0; j < SN; j++)
#pragma unroll
    for (int v = 0; v < 16; v++) acc[j][v] = 0.0f;

  // One block of this wave: SN tiles, each an fp6 MFMA (the exact dot with
  // the -8 sum(xq) C input, scaled by 2^e_x), an f16 outer-product MFMA
  // (mant(sx) * sw) and 16 fma. Software-pipelined over (block, tile): the
  // fmas of a tile run after the next tile's MFMAs are issued (the last
  // tile's fmas open the next block), and a tile's weight fragment is read
  // from LDS while the previous tile's fmas run.
  v16f pd, ps;  // MFMA results of the tile before, not yet folded
  auto fold = [&](int j) {
#pragma unroll
    for (int v = 0; v < 16; v++) acc[j][v] = fmaf(pd[v], ps[v], acc[j][v]);
  };
  auto compute = [&](const uint8_t* sbase, int kb, i32x4 lo, i32x4 hi, bool first) {
    // The MFMA wants the 6 code dwords in consecutive registers; the two
    // loads land apart, so the compiler copies one half next to the other.
    // Defining both halves here keeps that copy (which waits for its load)
    // at the point of use, blocks after the load, not right behind it.
    asm volatile("" : "+v"(lo), "+v"(hi));
    const v8i a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    const int sa = hi[3];  // byte 0: the E8M0 scale
    const h4 as = __builtin_bit_cast(h4, make_uint2((uint32_t)hi[2], (uint32_t)hi[3]));
    const float* cp = (const float*)(sbase + kW + (mg * kKB + kb) * 128 + (lane >> 5) * 64);
    const uint8_t* wrow = sbase + (lane & 31) * RS + kb * kRecW;
    v16f c;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float4 cv = *(const float4*)(cp + 4 * j);
      c[4 * j] = cv.x;
      c[4 * j + 1] = cv.y;
      c[4 * j + 2] = cv.z;
      c[4 * j + 3] = cv.w;
    }
    uint4 w0 = *(const uint4*)wrow, w1 = *(const uint4*)(wrow + 16);
#pragma unroll
    for (int j = 0; j < SN; j++) {
      const v8i bq = {(int)w0.x, (int)w0.y, (int)w0.z, (int)w0.w, (int)w1.x, (int)w1.y, 0, 0};
      const h4 bs = __builtin_bit_cast(h4, make_uint2(w1.z, w1.w));
      const v16f z = {};
      const v16f sc = __builtin_amdgcn_mfma_f32_32x32x8f16(as, bs, z, 0, 0, 0);
      const v16f d = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, bq, c, 2, 2, 0, sa, 0, 130);
      if (j + 1 < SN) {
        w0 = *(const uint4*)(wrow + (j + 1) * 32 * RS);
        w1 = *(const uint4*)(wrow + (j + 1) * 32 * RS + 16);
      }
      if (j > 0) {
        fold(j - 1);
      } else if (!first) {
        fold(SN - 1);
      }
      pd = d;
      ps = sc;
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // ---- main loop: stages of kKB blocks; this wave takes blocks of its parity
  i32x4 rlo[kRing], rhi[kRing];
#pragma unroll
  for (int r = 0; r < kRing; r++) load_a(b_begin + kp + 2 * r, rlo[r], rhi[r]);
  load_stage(0);
  store_stage(0);
  __syncthreads();
  bool first = true;
  for (int s = 0; s < stages; s++) {
    const int buf = s & 1;
    if (s + 1 < stages) load_stage(s + 1);
    const uint8_t* sbase = lds + buf * kStage;
    const int b0 = b_begin + s * kKB;
#pragma unroll 1
    for (int u0 = 0; u0 < kKB / 2; u0 += kRing) {
#pragma unroll
      for (int r = 0; r < kRing; r++) {
        const int kb = kp + 2 * (u0 + r);
        compute(sbase, kb, rlo[r], rhi[r], first);
        first = false;
        load_a(b0 + kb + 2 * kRing, rlo[r], rhi[r]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (s + 1 < stages) store_stage(buf ^ 1);
    __syncthreads();
  }

  if (!first) fold(SN - 1);

  float* out = p.part ? p.part + (size_t)blockIdx.y * M * N : p.y;
  store_tile_sums<SN>(lds, acc, wave, lane, tm * kTileM * kTokens, n0, M, N, out, p.vec != 0);
}

// ----------------------------------------------- prepacked weights (load time)
//
// The engine's Q4 layout needs 16 VALU operations per 32 weights to become
// fp6 fields, and its -8 offset costs the MFMA a C input (16 more register
// reads per tile). Weights are immutable after upload, so they can be
// re-encoded once: per (row, block) a 32-byte record, the E2M3 codes of the
// signed weights w = q - 8 (sign bit, |w| in 0..8 as the code of |w| / 8) in
// the fields' order, then the scale MFMA's slots (sw, sw, 0, sw).
//
// The records are laid out tile-major, exactly as one B fragment sits in
// LDS: per 32-row group and block one 1 KB chunk, [half][32 rows][16 B]
// (half 0 = each record's first 16 bytes). Rows past the matrix, up to the
// group's 32, hold zero records. One 16-byte LDS DMA per lane moves a whole
// chunk from HBM into LDS, with no registers and no staging pass.

constexpr int kChunk = 1024;  // one (32-row group, block) of the prepack

DNX_DEV uint32_t f6_signed_code(uint32_t q) {
  return q >= 8 ? q - 8 : 0x20u | (8 - q);
}

// One thread per (row, block) of the matrix padded to whole 32-row groups:
// 16 nibble bytes + the fp16 scale -> the record's two halves.
__global__ void __launch_bounds__(kPanelThreads) pack_q4_f6_kernel(
    const uint8_t* __restrict__ qs, const uint16_t* __restrict__ scales,
    uint8_t* __restrict__ out, int rows, int B, int64_t count) {
  for (int64_t i = (int64_t)blockIdx.x * kPanelThreads + threadIdx.x; i < count;
       i += (int64_t)gridDim.x * kPanelThreads) {
    const int r = (int)(i / B), b = (int)(i - (int64_t)r * B);
    uint32_t o[6] = {0, 0, 0, 0, 0, 0};
    uint32_t sw = 0;
    if (r < rows) {
      const uint4 v = *(const uint4*)(qs + i * 16);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int f = 0; f < 32; f++) {
        const int k = kFieldKHost[f];
        const int byte = k & 15;
        const uint32_t q = (w[byte >> 2] >> (8 * (byte & 3) + (k >= 16 ? 4 : 0))) & 15u;
        const uint32_t c = f6_signed_code(q);
        const int bit = 6 * f, wd = bit >> 5, sh = bit & 31;
        o[wd] |= c << sh;
        if (sh > 26) o[wd + 1] |= c >> (32 - sh);
      }
      sw = scales[i];
    }
    uint8_t* d = out + ((int64_t)(r >> 5) * B + b) * kChunk + (r & 31) * 16;
    *(uint4*)d = make_uint4(o[0], o[1], o[2], o[3]);
    *(uint4*)(d + kChunk / 2) = make_uint4(o[4], o[5], sw | (sw << 16), sw << 16);
  }
}

// Q8 weights (int8 w in [-128, 127] + an fp32 scale per block, the engine's
// layout, lab_native.c:398-405) need two fp6 digits, |w| = 8 wh + wl (wh <=
// 15, wl <= 8; both E2M3 codes with w's sign): the dot takes two MFMAs per
// block, the h codes against wh (B scale 2^6) and against wl (2^3), chained
// through the C input (every partial sum an integer below 2^24: exact). The
// scale sw = mant * 2^ew puts ew into the B operand's E8M0 scales and mant
// into two fp16 pieces m0 + m1 (22 of its 24 bits) for the scale MFMA:
// lanes 0..31 pair (p0, p1, byte, p2) of the activation with (m0, m0, 0, m0),
// lanes 32..63 pair (p0, p1, byte, 0) with (m1, m1, 0, 0), giving
// (p0 + p1 + p2) m0 + (p0 + p1) m1 (dropped terms below 2^-22 relative).
// Per 32-row group and block, 2.5 KB: five [32 rows][16 B] parts: wh codes
// 0..3; wh codes 4..5 + the low lanes' scale slots; the same + the high
// lanes' slots; wl codes 0..3; wl codes 4..5 + the two E8M0 bytes.
constexpr int kChunk8 = 2560;

__global__ void __launch_bounds__(kPanelThreads) pack_q8_f6_kernel(
    const int8_t* __restrict__ qs, const float* __restrict__ scales, uint8_t* __restrict__ out,
    int rows, int B, int64_t count) {
  for (int64_t i = (int64_t)blockIdx.x * kPanelThreads + threadIdx.x; i < count;
       i += (int64_t)gridDim.x * kPanelThreads) {
    const int r = (int)(i / B), b = (int)(i - (int64_t)r * B);
    uint32_t h[6] = {0, 0, 0, 0, 0, 0}, l[6] = {0, 0, 0, 0, 0, 0};
    float sw = 0.0f;
    if (r < rows) {
      const uint4 v0 = *(const uint4*)(qs + i * 32), v1 = *(const uint4*)(qs + i * 32 + 16);
      const uint32_t w[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
      for (int f = 0; f < 32; f++) {
        const int k = kFieldKHost[f];
        const int v = (int)(int8_t)(w[k >> 2] >> (8 * (k & 3)));
        const uint32_t a = (uint32_t)(v < 0 ? -v : v);
        const uint32_t wh = a >> 3 > 15 ? 15 : a >> 3, wl = a - 8 * wh;
        const uint32_t sg = v < 0 ? 0x20u : 0u;
        const uint32_t ch = sg | wh, cl = sg | wl;
        const int bit = 6 * f, wd = bit >> 5, sh = bit & 31;
        h[wd] |= ch << sh;
        l[wd] |= cl << sh;
        if (sh > 26) {
          h[wd + 1] |= ch >> (32 - sh);
          l[wd + 1] |= cl >> (32 - sh);
        }
      }
      sw = scales[i];
    }
    // sw = mant * 2^ew, mant in [1, 2) (a subnormal keeps ew = -126, mant < 1;
    // beyond 2^120 the rest of the exponent moves into mant).
    const uint32_t bits = __float_as_uint(sw);
    const int ef = (int)((bits >> 23) & 0xff);
    int ew = ef == 0 ? -126 : ef - 127;
    float mant = ef == 0 ? sw * 0x1p126f : __uint_as_float((bits & 0x807fffffu) | 0x3f800000u);
    if (ew > 120) {
      mant = ldexpf(mant, ew - 120);
      ew = 120;
    }
    if (sw == 0.0f) {
      ew = 0;
      mant = 0.0f;
    }
    const _Float16 m0 = (_Float16)mant;
    const _Float16 m1 = (_Float16)(mant - (float)m0);
    const uint32_t b0 = __builtin_bit_cast(uint16_t, m0), b1 = __builtin_bit_cast(uint16_t, m1);
    uint8_t* d = out + ((int64_t)(r >> 5) * B + b) * kChunk8 + (r & 31) * 16;
    *(uint4*)d = make_uint4(h[0], h[1], h[2], h[3]);
    *(uint4*)(d + 512) = make_uint4(h[4], h[5], b0 | (b0 << 16), b0 << 16);
    *(uint4*)(d + 1024) = make_uint4(h[4], h[5], b1 | (b1 << 16), 0u);
    *(uint4*)(d + 1536) = make_uint4(l[0], l[1], l[2], l[3]);
    *(uint4*)(d + 2048) = make_uint4(l[4], l[5], (uint32_t)(127 + 6 + ew), (uint32_t)(127 + 3 + ew));
  }
}

constexpr int kPKB = 8;     // blocks per stage of the prepacked GEMM
static_assert(kKB % kPKB == 0, "a K split holds whole prepacked stages");

struct F6PParams {
  const uint8_t* packed;   // tile-major prepack [groups of 32 rows][cols/32][1 KB]
  const uint8_t* panel;    // f6 panel of the n tokens
  float* y;
  float* part;
  int rows, cols, n;
  int tiles_m, tiles;
  int split_blocks;        // a multiple of kKB (whole stages)
  int vec;                 // the output allows 16-byte stores
};

// Stages of kPKB blocks (Q8: kPKB / 2); a stage's weights (SN row groups x
// its blocks: 24 KB of Q4, 30 KB of Q8, so that two or three workgroups fit
// a CU's LDS; contiguous per row group in the prepack) move
// into one of two LDS buffers by DMA in 1 KB pieces, spread over the waves,
// issued at the start of the stage before: they arrive while that stage
// computes. The activation records stay in a register ring one stage
// (half the stage's blocks, this wave's parity) ahead. The DMA is inline asm (buffer_load16_to_lds),
// so the compiler's waits ignore it; each stage ends with an explicit vmcnt
// that covers this wave's DMA (only the stage's ring refills are younger)
// and a barrier that publishes every wave's DMA and retires the buffer just
// read. Blocks past this split's end and row groups past the matrix read
// whatever lies there (the next blocks or row group, or zeros past the
// prepack): finite codes and scales that meet zero activations or are
// never stored.
template <int SN, bool kQ8>
__global__ void __launch_bounds__(kThreads) gemm_f6p_kernel(F6PParams p) {
  constexpr int BN = SN * 32;
  constexpr int kCh = kQ8 ? kChunk8 : kChunk;         // bytes per (row group, block)
  constexpr int kPK = kQ8 ? kPKB / 2 : kPKB;          // blocks per stage
  constexpr int kGroupBytes = kPK * kCh;             // a row group's stage, contiguous
  constexpr int kStage = SN * kGroupBytes;
  constexpr int kPieces = kStage / 1024;              // DMA instructions per stage
  constexpr int kPiecesPerGroup = kGroupBytes / 1024;
  static_assert(kGroupBytes % 1024 == 0, "whole 1 KB pieces per row group");
  constexpr int kRingP = kPK / 2;                    // own-parity blocks per stage
  constexpr int kLds = 2 * kStage > epilogue_lds_bytes<SN>() ? 2 * kStage : epilogue_lds_bytes<SN>();
  __shared__ __align__(16) uint8_t lds[kLds];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int mg = wave & 3, kp = wave >> 2;
  const int K = p.cols, B = K / kBlock, M = p.n, N = p.rows;
  const int groups_n = (N + 31) >> 5;

  const int i = blockIdx.x;
  const int t = (p.tiles % 8 == 0) ? (i % 8) * (p.tiles / 8) + i / 8 : i;
  const int tm = t % p.tiles_m, tn = t / p.tiles_m;
  const int n0 = tn * BN, g0 = tn * SN;
  const int groups = (M + kTokens - 1) / kTokens;
  const int g = tm * kTileM + mg;
  const int b_begin = blockIdx.y * p.split_blocks;
  const int b_end = min(B, b_begin + p.split_blocks);
  const int stages = (b_end - b_begin + kPK - 1) / kPK;
  const i32x4 rpanel = buffer_rsrc(p.panel, (uint32_t)((size_t)groups * B * kRec));
  const i32x4 rpk = buffer_rsrc(p.packed, (uint32_t)((size_t)groups_n * B * kCh));
  const uint32_t lds0 = lds_address(lds);

  // Stage s's weights into buffer `buf`, [row group j][block kb][kCh].
  auto dma_w = [&](int s, int buf) {
    const int b0 = b_begin + s * kPK;
#pragma unroll
    for (int e = 0; e < (kPieces + kWaves - 1) / kWaves; e++) {
      const int c = wave + kWaves * e;
      if (c < kPieces) {
        const int j = c / kPiecesPerGroup, q = c - j * kPiecesPerGroup;
        buffer_load16_to_lds(rpk, lds0 + buf * kStage + j * kGroupBytes + q * 1024,
                             ((g0 + j) * B + b0) * kCh + q * 1024 + lane * 16);
      }
    }
  };

  const bool live = g < groups;
  auto load_a = [&](int b, i32x4& lo, i32x4& hi) {
    const int ok = -(int)(live & (b < b_end));
    const int base = (((g * B + b) * kRec + kRecF) & ok) | (~ok & -(1 << 20));
    lo = dnx_raw_buffer_load_v4i32(rpanel, base + lane * 16, 0, 0);
    hi = dnx_raw_buffer_load_v4i32(rpanel, base + kRecHalf + lane * 16, 0, 0);
  };

  v16f acc[SN];
#pragma unroll
  for (int j = 0; j < SN; j++)
#pragma unroll
    for (int v = 0; v < 16; v++) acc[j][v] = 0.0f;
  // Software pipeline over tiles: the products of tile j are folded into
  // the accumulators while the matrix cores run tile j + 1, and the LDS
  // fragments of the next tile are read while they run tile j. The order
  // inside a tile is pinned (MFMAs, then LDS reads, then the previous fold):
  // left to itself the scheduler folds a tile right behind its own MFMA and
  // every fold then waits out the MFMA latency.
  v16f pd, ps;
#pragma unroll
  for (int v = 0; v < 16; v++) pd[v] = ps[v] = 0.0f;
  auto fold = [&](int j) {
#pragma unroll
    for (int v = 0; v < 16; v++) acc[j][v] = fmaf(pd[v], ps[v], acc[j][v]);
  };
  // B fragment of one tile: lane l takes row l % 32's parts (both lane
  // halves the same codes: the K slots of the h and the l activation codes).
  // Q4: codes 0..3, then codes 4..5 + scale slots. Q8: wh 0..3, wh 4..5 +
  // this lane half's scale slots, wl 0..3, wl 4..5 + the E8M0 bytes.
  struct BFrag {
    uint4 c[kQ8 ? 4 : 2];
  };
  auto read_b = [&](const uint8_t* sbase, int kb, int j) {
    const uint8_t* q = sbase + (j * kPK + kb) * kCh + (lane & 31) * 16;
    BFrag f;
    f.c[0] = *(const uint4*)q;
    if constexpr (kQ8) {
      f.c[1] = *(const uint4*)(q + 512 + (lane >> 5) * 512);
      f.c[2] = *(const uint4*)(q + 1536);
      f.c[3] = *(const uint4*)(q + 2048);
    } else {
      f.c[1] = *(const uint4*)(q + 512);
    }
    return f;
  };
  // One block of K for the SN tiles; `nb` holds tile 0 of this block on
  // entry and tile 0 of block kb_next on exit.
  auto compute = [&](const uint8_t* sbase, int kb, int kb_next, i32x4 lo, i32x4 hi, BFrag& nb) {
    asm volatile("" : "+v"(lo), "+v"(hi));
    const v8i a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    const int sa = hi[3];
    // The scale MFMA's activation slots: (p0, p1, byte, p2) on the h lanes;
    // for Q8 the l lanes take (p0, p1) of their token's h lane (a
    // permlane32 swap broadcasts the low half), beside their (byte, 0).
    uint32_t s01 = (uint32_t)hi[2];
    if constexpr (kQ8) s01 = (uint32_t)__builtin_amdgcn_permlane32_swap(hi[2], hi[2], false, false)[0];
    const h4 as = __builtin_bit_cast(h4, make_uint2(s01, (uint32_t)hi[3]));
    BFrag cur = nb;
#pragma unroll
    for (int j = 0; j < SN; j++) {
      const v8i bq = {(int)cur.c[0].x, (int)cur.c[0].y, (int)cur.c[0].z, (int)cur.c[0].w,
                      (int)cur.c[1].x, (int)cur.c[1].y, 0, 0};
      const h4 bs = __builtin_bit_cast(h4, make_uint2(cur.c[1].z, cur.c[1].w));
      const v16f z = {};
      const v16f sc = __builtin_amdgcn_mfma_f32_32x32x8f16(as, bs, z, 0, 0, 0);
      v16f d;
      if constexpr (kQ8) {
        const v8i bl = {(int)cur.c[2].x, (int)cur.c[2].y, (int)cur.c[2].z, (int)cur.c[2].w,
                        (int)cur.c[3].x, (int)cur.c[3].y, 0, 0};
        d = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, bq, z, 2, 2, 0, sa, 0,
                                                           (int)cur.c[3].z);
        d = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, bl, d, 2, 2, 0, sa, 0,
                                                           (int)cur.c[3].w);
      } else {
        d = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, bq, z, 2, 2, 0, sa, 0, 130);
      }
      if (j + 1 < SN) {
        cur = read_b(sbase, kb, j + 1);
      } else {
        nb = read_b(sbase, kb_next, 0);
      }
      fold(j > 0 ? j - 1 : SN - 1);
      pd = d;
      ps = sc;
      __builtin_amdgcn_sched_group_barrier(0x008, kQ8 ? 3 : 2, 0);   // the MFMAs
      __builtin_amdgcn_sched_group_barrier(0x100, kQ8 ? 4 : 2, 0);   // next fragment
      __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);            // previous fold
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  i32x4 rlo[kRingP], rhi[kRingP];
  dma_w(0, 0);
#pragma unroll
  for (int r = 0; r < kRingP; r++) load_a(b_begin + kp + 2 * r, rlo[r], rhi[r]);
  if (stages > 1) dma_w(1, 1);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int s = 0; s < stages; s++) {
    const int buf = s & 1;
    // W(s + 1) into the buffer stage s - 1 read (every wave is past it).
    if (s >= 1 && s + 1 < stages) dma_w(s + 1, buf ^ 1);
    const uint8_t* sbase = lds + buf * kStage;
    const int b0 = b_begin + s * kPK;
    BFrag nb = read_b(sbase, kp, 0);
#pragma unroll
    for (int r = 0; r < kRingP; r++) {
      const int kb = kp + 2 * r;
      compute(sbase, kb, min(kb + 2, kPK - 1), rlo[r], rhi[r], nb);
      load_a(b0 + kb + 2 * kRingP, rlo[r], rhi[r]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // This wave's W(s + 1) has landed: only the 2 * kRingP ring refills of
    // this stage were issued after it.
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(2 * kRingP));
    __syncthreads();
  }
  fold(SN - 1);
  float* out = p.part ? p.part + (size_t)blockIdx.y * M * N : p.y;
  store_tile_sums<SN>(lds, acc, wave, lane, tm * kTileM * kTokens, n0, M, N, out, p.vec != 0);
}

// ------------------------------------------- skinny prefill (5..512 tokens)
//
// A prefill chunk (the reference prefills in chunks of up to 64 tokens,
// lib/src/model.dart:91) or another batch of a few hundred tokens against a
// whole weight matrix: the weights dominate the bytes, the MFMA work is
// small. One workgroup owns 32
// weight rows and 64 tokens (G groups of 32; more tokens take more
// workgroups along y, which read the same weights) over the whole K, so no
// K split, no partials and no reduce launch: its 8 waves take blocks b = w,
// w + 8, ..., each wave loads its B chunks (the prepack) and A records (the
// panel) straight into a 4-block register ring, runs the fp6 dot and the
// scale MFMA per (token group, block) and folds; then the 8 waves' sums are
// added through LDS in wave order (deterministic) and stored write-through.

// Up to kMaxSegs matrices over the same x in one launch (a prefill chunk's
// q, k and v, or gate and up): their 32-row groups laid end to end along
// grid x, seg_end holding the cumulative group ends.
constexpr int kMaxSegs = 4;

struct F6SParams {
  const uint8_t* panel;    // f6 panel of the n tokens
  int cols, n;
  int segs;
  int seg_end[kMaxSegs];
  const uint8_t* packed[kMaxSegs];   // tile-major prepacks
  float* y[kMaxSegs];                // [n][rows]
  int rows[kMaxSegs];
};

// R: blocks in flight per wave (the register ring); kOnce: every wave has
// at most R blocks, all loaded at the start (no refills); RG: 32-row groups
// per workgroup (seg_end counts workgroups).
template <int G, int R, bool kOnce, int RG = 1>
__global__ void __launch_bounds__(kThreads) gemm_f6s_kernel(F6SParams p) {
  constexpr int kTile = G * kTokens * 32;              // outputs of one row group
  constexpr int kOut = RG * kTile;                     // outputs of the workgroup
  __shared__ __align__(16) float red[kWaves * kOut];   // each wave's sums, [wave][group][token][row]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // This workgroup's matrix (uniform: scalar selects over the segments).
  int seg = 0;
#pragma unroll
  for (int k = 1; k < kMaxSegs; k++) seg += (k < p.segs && (int)blockIdx.x >= p.seg_end[k - 1]);
  const int K = p.cols, B = K / kBlock, M = p.n;
  const int N = p.rows[seg];
  float* const yout = p.y[seg];
  const int rg = (blockIdx.x - (seg > 0 ? p.seg_end[seg - 1] : 0)) * RG;   // first 32-row group
  const int t0 = blockIdx.y * G;                       // first token group
  const int groups = (M + kTokens - 1) / kTokens;
  const int groups_n = (N + 31) >> 5;
  const i32x4 rpanel = buffer_rsrc(p.panel, (uint32_t)((size_t)groups * B * kRec));
  const i32x4 rpk = buffer_rsrc(p.packed[seg], (uint32_t)((size_t)groups_n * B * kChunk));

  // Block i of this wave is b = wave + 8 i; blocks past K read zeros (offset
  // past the resources), so their products vanish.
  struct Slot {
    i32x4 w0[RG], w1[RG]; // B: the record halves of row lane % 32 of each row group
    i32x4 lo[G], hi[G];   // A: the token groups' lane records
  };
  auto load = [&](int i, Slot& sl) {
    const int b = wave + kWaves * i;
    const int ok = -(int)(b < B);
    // Row groups past the matrix read zeros (offsets past the resource).
#pragma unroll
    for (int j = 0; j < RG; j++) {
      const int wb = (((rg + j) * B + b) * kChunk & ok) | (~ok & -(1 << 30));
      sl.w0[j] = dnx_raw_buffer_load_v4i32(rpk, wb + (lane & 31) * 16, 0, 0);
      sl.w1[j] = dnx_raw_buffer_load_v4i32(rpk, wb + kChunk / 2 + (lane & 31) * 16, 0, 0);
    }
    // A lane whose token lies past n (a chunk of 8 tokens fills a quarter of
    // its 32-token group) reads zeros without a memory access.
#pragma unroll
    for (int t = 0; t < G; t++) {
      const int tok = -(int)((t0 + t) * kTokens + (lane & 31) < M);
      const int ab = ((((t0 + t) * B + b) * kRec + kRecF + lane * 16) & ok & tok) |
                     (~(ok & tok) & -(1 << 30));
      sl.lo[t] = dnx_raw_buffer_load_v4i32(rpanel, ab, 0, 0);
      sl.hi[t] = dnx_raw_buffer_load_v4i32(rpanel, ab + kRecHalf, 0, 0);
    }
  };

  v16f acc[RG][G];
#pragma unroll
  for (int j = 0; j < RG; j++)
#pragma unroll
    for (int t = 0; t < G; t++)
#pragma unroll
      for (int v = 0; v < 16; v++) acc[j][t][v] = 0.0f;
  const int nb = (B - wave + kWaves - 1) / kWaves;     // this wave's blocks
  Slot ring[R];
#pragma unroll
  for (int r = 0; r < R; r++) load(r, ring[r]);
  for (int i0 = 0; i0 < nb; i0 += R) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      Slot& sl = ring[r];
#pragma unroll
      for (int j = 0; j < RG; j++) {
        i32x4 w0 = sl.w0[j], w1 = sl.w1[j];
        asm volatile("" : "+v"(w0), "+v"(w1));
        const v8i bq = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], 0, 0};
        const h4 bs = __builtin_bit_cast(h4, make_uint2((uint32_t)w1[2], (uint32_t)w1[3]));
#pragma unroll
        for (int t = 0; t < G; t++) {
          i32x4 lo = sl.lo[t], hi = sl.hi[t];
          asm volatile("" : "+v"(lo), "+v"(hi));
          const v8i a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
          const h4 as = __builtin_bit_cast(h4, make_uint2((uint32_t)hi[2], (uint32_t)hi[3]));
          const v16f z = {};
          const v16f sc = __builtin_amdgcn_mfma_f32_32x32x8f16(as, bs, z, 0, 0, 0);
          const v16f d = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, bq, z, 2, 2, 0,
                                                                         hi[3], 0, 130);
#pragma unroll
          for (int v = 0; v < 16; v++) acc[j][t][v] = fmaf(d[v], sc[v], acc[j][t][v]);
        }
        // Two row groups: one group's MFMA results live at a time.
        if constexpr (RG > 1) __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (!kOnce) load(i0 + r + R, sl);
    }
  }

  // Each wave's sums into LDS as [token][row], then every thread adds one
  // float4 of rows over the 8 waves in wave order and stores it.
  float* mine = red + wave * kOut;
#pragma unroll
  for (int j = 0; j < RG; j++)
#pragma unroll
    for (int t = 0; t < G; t++)
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int m = t * kTokens + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
        mine[j * kTile + m * 32 + (lane & 31)] = acc[j][t][v];
      }
  __syncthreads();
  for (int q = tid; q < kOut / 4; q += kThreads) {
    const int j = q / (kTile / 4), qq = q - j * (kTile / 4);
    const int m = qq >> 3, c = (qq & 7) * 4;
    float4 o = *(const float4*)(red + j * kTile + m * 32 + c);
#pragma unroll
    for (int w = 1; w < kWaves; w++) {
      const float4 e = *(const float4*)(red + w * kOut + j * kTile + m * 32 + c);
      o = make_float4(o.x + e.x, o.y + e.y, o.z + e.z, o.w + e.w);
    }
    const int r = (rg + j) * 32 + c, mt = t0 * kTokens + m;
    if (mt >= M || r >= N) continue;
    float* dst = yout + (size_t)mt * N + r;
    if (r + 3 < N && ((uintptr_t)dst & 15) == 0) {
      store_wt4(dst, o);
    } else {
      store_wt(dst, o.x);
      if (r + 1 < N) store_wt(dst + 1, o.y);
      if (r + 2 < N) store_wt(dst + 2, o.z);
      if (r + 3 < N) store_wt(dst + 3, o.w);
    }
  }
}

// y = the split partials summed in split order (deterministic).
__global__ void __launch_bounds__(256) f6_splitk_reduce_kernel(const float* __restrict__ part,
                                                               float* __restrict__ y,
                                                               int64_t count, int splits) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < count;
       i += (int64_t)gridDim.x * 256) {
    store_wt(y + i, split_sum(part, count, i, splits));
  }
}

// Library-owned split partials, grown on demand: a call at a larger shape
// than any before allocates, so such a call must not be the first inside a
// graph capture.
float* gF6Part = nullptr;
size_t gF6PartBytes = 0;

float* part_workspace(size_t bytes) {
  if (bytes <= gF6PartBytes) return gF6Part;
  if (gF6Part != nullptr) {
    if (hipDeviceSynchronize() != hipSuccess) return nullptr;
    (void)hipFree(gF6Part);
    gF6Part = nullptr;
    gF6PartBytes = 0;
  }
  if (hipMalloc(&gF6Part, bytes) != hipSuccess) {
    gF6Part = nullptr;
    return nullptr;
  }
  gF6PartBytes = bytes;
  return gF6Part;
}

// Blocks per K part of the fp6 GEMMs (both layouts, so that they add the
// same partials in the same order). A workgroup's registers fill its CU, so
// a launch runs in rounds of 256 workgroups: K is split only when the tiles
// leave at least half the CUs idle (from 129 to 255 tiles a split would add
// a round and gain nothing), into the most parts that still fit one round
// (tiles x parts <= 256), each of whole kKB-block stages.
int f6_split_blocks(int tiles, int B) {
  int splits = 1;
  if (tiles <= 128) {
    splits = 256 / tiles;
    const int max_splits = (B + kKB - 1) / kKB;
    if (splits > max_splits) splits = max_splits;
  }
  const int per = (B + splits - 1) / splits;
  return (per + kKB - 1) / kKB * kKB;
}

// Split partials of dnx_gemm_q4_f6p_noalloc: a fixed array in the code
// object, so that entry point never allocates. Every GPU the library runs on
// holds its own copy from the module's load until the process ends. In host
// code `scratch` names only a host-side stand-in: kernels get the address
// hipGetSymbolAddress returns for the current device (scratch_on_device).
// Size: K is split into at most 256 / tiles parts (f6_split_blocks), and
// n x rows <= (128 x tiles_m) x (96 x tiles_n) = 12288 x tiles, so the
// partials never exceed 12288 x 256 floats (12 MiB) for any shape the GEMM
// accepts; the bound is still checked on every call.
constexpr size_t kScratchFloats = (size_t)12288 * 256;
static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
std::mutex gScratchMu;
float* gScratchPtr[kMaxDevices] = {};

// The device address of `scratch` on the current device, looked up once per
// device (nullptr when the lookup fails).
float* scratch_on_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(gScratchMu);
  if (gScratchPtr[dev] == nullptr) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) {
      return nullptr;
    }
    gScratchPtr[dev] = (float*)ptr;
  }
  return gScratchPtr[dev];
}


bool f6_shape_ok(int64_t rows, int64_t cols, int64_t n) {
  if (rows <= 0 || cols <= 0 || n <= 0 || cols % kBlock != 0) return false;
  // 32-bit buffer offsets: each operand below 2 GB.
  return rows * (cols / 2) < (1ll << 31) && f6_panel_bytes(n, cols) < (1ll << 31) &&
         rows * (cols / kBlock) * 2 < (1ll << 31) && n * rows < (1ll << 31);
}

// The prepacked operand (whole 32-row groups, 1 KB per group and block for
// Q4, 2.5 KB for Q8) below 2 GB as well.
bool f6p_shape_ok(int64_t rows, int64_t cols, int64_t n, bool q8 = false) {
  return f6_shape_ok(rows, cols, n) &&
         (rows + 31) / 32 * (cols / kBlock) * (q8 ? kChunk8 : kChunk) < (1ll << 31);
}

template <int SN>
int launch_f6(const uint8_t* qs, const uint16_t* scales, const uint8_t* panel, float* y,
              int64_t rows, int64_t cols, int64_t n, hipStream_t stream) {
  constexpr int BN = SN * 32;
  F6Params p{};
  p.qs = qs;
  p.scales = scales;
  p.panel = panel;
  p.y = y;
  p.rows = (int)rows;
  p.cols = (int)cols;
  p.n = (int)n;
  p.tiles_m = (int)((n + kTileM * kTokens - 1) / (kTileM * kTokens));
  p.tiles = p.tiles_m * (int)((rows + BN - 1) / BN);
  const int B = (int)(cols / kBlock);
  p.split_blocks = f6_split_blocks(p.tiles, B);
  int splits = (B + p.split_blocks - 1) / p.split_blocks;
  const int64_t count = n * rows;
  p.part = nullptr;
  if (splits > 1) {
    p.part = part_workspace((size_t)splits * count * 4);
    if (p.part == nullptr) return DNX_ENOMEM;
  }
  p.vec = (rows % 4 == 0 && ((uintptr_t)(p.part ? (void*)p.part : (void*)y) & 15) == 0) ? 1 : 0;
  hipLaunchKernelGGL((gemm_f6_q4_kernel<SN>), dim3((unsigned)p.tiles, (unsigned)splits),
                     dim3(kThreads), 0, stream, p);
  if (hipGetLastError() != hipSuccess) return DNX_ELAUNCH;
  if (splits > 1) {
    const int64_t blocks = (count + 255) / 256;
    hipLaunchKernelGGL(f6_splitk_reduce_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)),
                       dim3(256), 0, stream, p.part, y, count, splits);
    if (hipGetLastError() != hipSuccess) return DNX_ELAUNCH;
  }
  return DNX_OK;
}

template <int SN, bool kQ8 = false>
int launch_f6p(const uint8_t* packed, const uint8_t* panel, float* y, int64_t rows,
               int64_t cols, int64_t n, hipStream_t stream, float* fixed_part = nullptr,
               size_t fixed_floats = 0) {
  constexpr int BN = SN * 32;
  F6PParams p{};
  p.packed = packed;
  p.panel = panel;
  p.y = y;
  p.rows = (int)rows;
  p.cols = (int)cols;
  p.n = (int)n;
  p.tiles_m = (int)((n + kTileM * kTokens - 1) / (kTileM * kTokens));
  p.tiles = p.tiles_m * (int)((rows + BN - 1) / BN);
  const int B = (int)(cols / kBlock);
  // The same split of K as launch_f6 (whole kKB-block parts, kKB a multiple
  // of kPKB), so that both kernels add the same partials in the same order.
  p.split_blocks = f6_split_blocks(p.tiles, B);
  int splits = (B + p.split_blocks - 1) / p.split_blocks;
  const int64_t count = n * rows;
  p.part = nullptr;
  if (splits > 1) {
    if (fixed_part != nullptr) {
      // The allocation-free entry point: its partials must fit the array.
      if ((size_t)splits * (size_t)count > fixed_floats) return DNX_ESCRATCH;
      p.part = fixed_part;
    } else {
      p.part = part_workspace((size_t)splits * count * 4);
      if (p.part == nullptr) return DNX_ENOMEM;
    }
  }
  p.vec = (rows % 4 == 0 && ((uintptr_t)(p.part ? (void*)p.part : (void*)y) & 15) == 0) ? 1 : 0;
  hipLaunchKernelGGL((gemm_f6p_kernel<SN, kQ8>), dim3((unsigned)p.tiles, (unsigned)splits),
                     dim3(kThreads), 0, stream, p);
  if (hipGetLastError() != hipSuccess) return DNX_ELAUNCH;
  if (splits > 1) {
    const int64_t blocks = (count + 255) / 256;
    hipLaunchKernelGGL(f6_splitk_reduce_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)),
                       dim3(256), 0, stream, p.part, y, count, splits);
    if (hipGetLastError() != hipSuccess) return DNX_ELAUNCH;
  }
  return DNX_OK;
}

// ----------------------------------- Q8 weights, prepacked, on int8 MFMA
//
// The Q8 GEMM at batch sizes (the vision encoder's fc1 / fc2 at 1024
// tokens, lib/src/vision_encoder.dart:275-316; the product of lab_gemm_q8
// mode 1, lab_native.c:1059-1080). One v_mfma_i32_32x32x32_i8 takes a whole
// Q8 block (K = 32) and gives its exact int32 dot D_b, where the fp6 form
// above needs two digits of each weight and two MFMAs per block. The scale
// product s = sx * sw of a 32 x 32 tile comes from the bf16 outer-product
// MFMA (three exact bf16 pieces of each scale, a_scale_half* /
// b_scale_half* in common.h), and the fold per output and block is cvt +
// fma: acc += float(D_b) * s, blocks in order.
//
// Both operands sit in HBM in fragment order, so a wave's loads (weights by
// LDS DMA, activations straight into registers) need no rearranging: per 32
// rows (or tokens) and block a 1536-byte record, [2 lane halves][32 rows][16
// B] of int8 values (half 0: k = 0..15, half 1: k = 16..31), then [2 lane
// halves][32 rows][8 B] of the scale's bf16 pieces. The workgroup, its
// stages and the split of K follow gemm_f6p_kernel: 128 tokens x SN * 32
// rows, wave w on the 32 tokens (w % 4) and the blocks of parity w / 4,
// 8-block stages in two LDS buffers, the fold of one tile under the MFMAs of
// the next.
constexpr int kI8Rec = 1536;   // bytes per (32 rows or tokens, block)
constexpr int kI8Sc = 1024;    // the scale pieces' offset in a record
constexpr int kI8KB = 8;       // blocks per stage

int64_t i8_panel_bytes(int64_t n, int64_t cols) {
  return (n + kTokens - 1) / kTokens * (cols / kBlock) * kI8Rec;
}

// fp32 x [n][cols] -> the int8 panel, lab_quantize_q8 of each (token,
// block) (the same xq and scale bits as dnx_quantize_q8), four lanes per
// (token, block): lane j quantizes values 8j .. 8j+7 and stores them as 8
// bytes of its token's half j / 2; lanes 0 and 1 store the scale's two
// halves of bf16 pieces. All four lanes of a quad run every iteration
// together (the block maximum comes by DPP over the quad). Tokens past n
// get zero records.
__global__ void __launch_bounds__(kPanelThreads) quantize_i8_panel_kernel(
    const float* __restrict__ x, uint8_t* __restrict__ panel, int n, int cols, int groups) {
  const int B = cols / kBlock;
  const int64_t total = (int64_t)groups * B * kTokens * 4;  // whole quads
  for (int64_t idx = (int64_t)blockIdx.x * kPanelThreads + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * kPanelThreads) {
    const int j = (int)(idx & 3);
    const int64_t q = idx >> 2;
    const int r = (int)(q & (kTokens - 1));
    const int64_t gb = q >> 5;
    const int b = (int)(gb % B);
    const int m = (int)(gb / B) * kTokens + r;
    const bool live = m < n;
    const float4* src = (const float4*)(x + (int64_t)(live ? m : 0) * cols + b * kBlock + 8 * j);
    const float4 v0 = live ? src[0] : make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 v1 = live ? src[1] : make_float4(0.f, 0.f, 0.f, 0.f);
    float amax = fmaxf(max4abs(v0), max4abs(v1));
    amax = fmaxf(amax, dppf<kQuadXor1>(amax));
    amax = fmaxf(amax, dppf<kQuadXor2>(amax));
    const float scale = q8_scale(amax);
    const float inv = q8_inv(scale);
    const float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    uint32_t w[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; i++) w[i >> 2] |= ((uint32_t)quant1(vv[i], inv) & 0xffu) << (8 * (i & 3));
    uint8_t* rec = panel + gb * kI8Rec;
    *(uint2*)(rec + (j >> 1) * 512 + r * 16 + (j & 1) * 8) = make_uint2(w[0], w[1]);
    if (j < 2) {
      uint32_t p0, p1, p2;
      split3_bf16(scale, p0, p1, p2);
      *(uint2*)(rec + kI8Sc + j * 256 + r * 8) =
          j == 0 ? a_scale_half0(p0, p1, p2) : a_scale_half1(p0, p1, p2);
    }
  }
}

// Q8 weights (int8 codes [rows][cols] + fp32 scales [rows][cols/32], the
// engine's layout, lab_native.c:398-405) -> the int8 prepack, one thread per
// (row, block) of the matrix padded to whole 32-row groups (rows past the
// matrix: zero records).
__global__ void __launch_bounds__(kPanelThreads) pack_q8_i8_kernel(
    const int8_t* __restrict__ qs, const float* __restrict__ scales, uint8_t* __restrict__ out,
    int rows, int B, int64_t count) {
  for (int64_t i = (int64_t)blockIdx.x * kPanelThreads + threadIdx.x; i < count;
       i += (int64_t)gridDim.x * kPanelThreads) {
    const int r = (int)(i / B), b = (int)(i - (int64_t)r * B);
    uint4 c0 = make_uint4(0u, 0u, 0u, 0u), c1 = c0;
    float sw = 0.0f;
    if (r < rows) {
      c0 = *(const uint4*)(qs + i * 32);
      c1 = *(const uint4*)(qs + i * 32 + 16);
      sw = scales[i];
    }
    uint8_t* rec = out + ((int64_t)(r >> 5) * B + b) * kI8Rec;
    *(uint4*)(rec + (r & 31) * 16) = c0;
    *(uint4*)(rec + 512 + (r & 31) * 16) = c1;
    uint32_t p0, p1, p2;
    split3_bf16(sw, p0, p1, p2);
    *(uint2*)(rec + kI8Sc + (r & 31) * 8) = b_scale_half0(p0, p1, p2);
    *(uint2*)(rec + kI8Sc + 256 + (r & 31) * 8) = b_scale_half1(p0, p1, p2);
  }
}

typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef int v16i_t __attribute__((ext_vector_type(16)));
typedef short s4_t __attribute__((ext_vector_type(4)));

// The GEMM on the int8 prepack and panel. Stage s (kI8KB blocks of the
// workgroup's SN row groups, 12 KB per group, contiguous in the prepack)
// moves into one of two LDS buffers by DMA, issued one stage ahead; each
// wave's activation records (16 + 8 bytes per lane and block) ride a
// register ring of its parity's blocks one stage ahead. Waits and barriers
// as in gemm_f6p_kernel. Blocks past this split's end and row groups past
// the matrix read what lies there (finite codes and scales that meet zero
// activations or are never stored); tokens past n read zeros.
template <int SN, int kTM>
__global__ void __launch_bounds__(kThreads) gemm_i8p_kernel(F6PParams p) {
  static_assert(kTM == 4 || kTM == 2, "128- or 64-token tiles");
  constexpr int kPar = kWaves / kTM;                 // block parities
  constexpr int BN = SN * 32;
  constexpr int kGroupBytes = kI8KB * kI8Rec;
  constexpr int kStage = SN * kGroupBytes;
  constexpr int kPieces = kStage / 1024;
  constexpr int kPiecesPerGroup = kGroupBytes / 1024;
  static_assert(kGroupBytes % 1024 == 0, "whole 1 KB pieces per row group");
  constexpr int kRingP = kI8KB / kPar;
  // 128-token tiles: up to 4 row groups both parities' partials fit beside
  // nothing else, wider tiles add them in place; 64-token tiles keep their
  // four parities' partials.
  constexpr bool kInplace = kTM == 4 && epilogue_lds_bytes<SN>() > 160 * 1024;
  constexpr int kEpi = kTM == 2 ? epilogue_lds_bytes_par4<SN>()
                       : kInplace ? epilogue_lds_bytes_inplace<SN>() : epilogue_lds_bytes<SN>();
  constexpr int kLds = 2 * kStage > kEpi ? 2 * kStage : kEpi;
  static_assert(kLds <= 160 * 1024, "a CU's LDS");
  __shared__ __align__(16) uint8_t lds[kLds];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int mg = wave % kTM, kp = wave / kTM;
  const int K = p.cols, B = K / kBlock, M = p.n, N = p.rows;
  const int groups_n = (N + 31) >> 5;

  const int i = blockIdx.x;
  const int t = (p.tiles % 8 == 0) ? (i % 8) * (p.tiles / 8) + i / 8 : i;
  const int tm = t % p.tiles_m, tn = t / p.tiles_m;
  const int n0 = tn * BN, g0 = tn * SN;
  const int groups = (M + kTokens - 1) / kTokens;
  const int g = tm * kTM + mg;
  const int b_begin = blockIdx.y * p.split_blocks;
  const int b_end = min(B, b_begin + p.split_blocks);
  const int stages = (b_end - b_begin + kI8KB - 1) / kI8KB;
  const i32x4 rpanel = buffer_rsrc(p.panel, (uint32_t)((size_t)groups * B * kI8Rec));
  const i32x4 rpk = buffer_rsrc(p.packed, (uint32_t)((size_t)groups_n * B * kI8Rec));
  const uint32_t lds0 = lds_address(lds);

  auto dma_w = [&](int s, int buf) {
    const int b0 = b_begin + s * kI8KB;
#pragma unroll
    for (int e = 0; e < (kPieces + kWaves - 1) / kWaves; e++) {
      const int c = wave + kWaves * e;
      if (c < kPieces) {
        const int j = c / kPiecesPerGroup, q = c - j * kPiecesPerGroup;
        buffer_load16_to_lds(rpk, lds0 + buf * kStage + j * kGroupBytes + q * 1024,
                             ((g0 + j) * B + b0) * kI8Rec + q * 1024 + lane * 16);
      }
    }
  };

  // This lane's bytes of a record: row lane % 32's values of its lane half,
  // and that half's scale pieces.
  const int off_c = (lane >> 5) * 512 + (lane & 31) * 16;
  const int off_s = kI8Sc + (lane >> 5) * 256 + (lane & 31) * 8;
  const bool live = g < groups;
  auto load_a = [&](int b, i32x4& c, i32x2& s) {
    const int ok = -(int)(live & (b < b_end));
    const int base = (((g * B + b) * kI8Rec) & ok) | (~ok & -(1 << 20));
    c = dnx_raw_buffer_load_v4i32(rpanel, base + off_c, 0, 0);
    s = dnx_raw_buffer_load_v2i32(rpanel, base + off_s, 0, 0);
  };

  v16f acc[SN];
#pragma unroll
  for (int j = 0; j < SN; j++)
#pragma unroll
    for (int v = 0; v < 16; v++) acc[j][v] = 0.0f;
  v16i_t pd;
  v16f ps;
#pragma unroll
  for (int v = 0; v < 16; v++) {
    pd[v] = 0;
    ps[v] = 0.0f;
  }
  auto fold = [&](int j) {
#pragma unroll
    for (int v = 0; v < 16; v++) acc[j][v] = fmaf((float)pd[v], ps[v], acc[j][v]);
  };
  struct BFrag {
    uint4 c;
    uint2 s;
  };
  auto read_b = [&](const uint8_t* sbase, int kb, int j) {
    const uint8_t* q = sbase + (j * kI8KB + kb) * kI8Rec;
    BFrag f;
    f.c = *(const uint4*)(q + off_c);
    f.s = *(const uint2*)(q + off_s);
    return f;
  };
  // One block of K for the SN tiles; `nb` holds tile 0 of this block on
  // entry and tile 0 of block kb_next on exit. The order inside a tile is
  // pinned (MFMAs, the next fragment's LDS reads, the previous tile's fold).
  auto compute = [&](const uint8_t* sbase, int kb, int kb_next, i32x4 c, i32x2 s, BFrag& nb) {
    asm volatile("" : "+v"(c), "+v"(s));
    const v4i_t a = __builtin_bit_cast(v4i_t, c);
    const s4_t as = __builtin_bit_cast(s4_t, s);
    BFrag cur = nb;
#pragma unroll
    for (int j = 0; j < SN; j++) {
      const v4i_t bq = __builtin_bit_cast(v4i_t, cur.c);
      const s4_t bs = __builtin_bit_cast(s4_t, cur.s);
      const v16f z = {};
      const v16i_t zi = {};
      const v16f sc = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(as, bs, z, 0, 0, 0);
      const v16i_t d = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bq, zi, 0, 0, 0);
      if (j + 1 < SN) {
        cur = read_b(sbase, kb, j + 1);
      } else {
        nb = read_b(sbase, kb_next, 0);
      }
      fold(j > 0 ? j - 1 : SN - 1);
      pd = d;
      ps = sc;
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);    // the MFMAs
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);    // next fragment
      __builtin_amdgcn_sched_group_barrier(0x002, 32, 0);   // previous fold
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  i32x4 rc[kRingP];
  i32x2 rs[kRingP];
  dma_w(0, 0);
#pragma unroll
  for (int r = 0; r < kRingP; r++) load_a(b_begin + kp + kPar * r, rc[r], rs[r]);
  if (stages > 1) dma_w(1, 1);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int s = 0; s < stages; s++) {
    const int buf = s & 1;
    if (s >= 1 && s + 1 < stages) dma_w(s + 1, buf ^ 1);
    const uint8_t* sbase = lds + buf * kStage;
    const int b0 = b_begin + s * kI8KB;
    BFrag nb = read_b(sbase, kp, 0);
#pragma unroll
    for (int r = 0; r < kRingP; r++) {
      const int kb = kp + kPar * r;
      compute(sbase, kb, min(kb + kPar, kI8KB - 1), rc[r], rs[r], nb);
      load_a(b0 + kb + kI8KB, rc[r], rs[r]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // This wave's W(s + 1) has landed: only the 2 * kRingP ring refills of
    // this stage were issued after it.
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(2 * kRingP));
    __syncthreads();
  }
  fold(SN - 1);
  float* out = p.part ? p.part + (size_t)blockIdx.y * M * N : p.y;
  if constexpr (kTM == 2) {
    store_tile_sums_par4<SN>(lds, acc, wave, lane, tm * kTM * kTokens, n0, M, N, out,
                             p.vec != 0);
  } else if constexpr (kInplace) {
    store_tile_sums_inplace<SN>(lds, acc, wave, lane, tm * kTM * kTokens, n0, M, N, out,
                                p.vec != 0);
  } else {
    store_tile_sums<SN>(lds, acc, wave, lane, tm * kTM * kTokens, n0, M, N, out, p.vec != 0);
  }
}

// Blocks per K part of the int8 prepacked GEMM: as f6_split_blocks (a split
// only at 128 tiles or fewer, the most parts that fit one round of 256
// workgroups), in whole kI8KB-block stages.
int i8_split_blocks(int tiles, int B) {
  int splits = 1;
  if (tiles <= 128) {
    splits = 256 / tiles;
    const int max_splits = (B + kI8KB - 1) / kI8KB;
    if (splits > max_splits) splits = max_splits;
  }
  const int per = (B + splits - 1) / splits;
  return (per + kI8KB - 1) / kI8KB * kI8KB;
}

bool i8p_shape_ok(int64_t rows, int64_t cols, int64_t n) {
  if (rows <= 0 || cols <= 0 || n <= 0 || cols % kBlock != 0) return false;
  return (rows + 31) / 32 * (cols / kBlock) * kI8Rec < (1ll << 31) &&
         i8_panel_bytes(n, cols) < (1ll << 31) && n * rows < (1ll << 31);
}

// The tile of the int8 prepacked GEMM: row groups per workgroup SN (3, 4 or
// 5: 96 to 160 rows) and token groups TM (4: 128 tokens, the waves in two
// block parities; 2: 64 tokens in four parities), the one whose launch
// takes the least time by a model of its measured costs. A workgroup fills
// its CU, so a launch runs in rounds of 256 workgroups; per round the
// slowest SIMD runs its two waves' tiles of their parities' blocks (about
// 100 ns per tile and block each, 120 on 64-token tiles), plus about 2 us of prologue and
// epilogue; a K split adds the reduce launch (about 1 us plus its partials
// read at 4 TB/s). The vision encoder's fc1 (4320 x 1152 at 1024 tokens)
// takes 128 x 160 tiles (216 workgroups, one round, against 360 in two);
// 1024 x 1024 at 1024 tokens 64 x 96 tiles (176 workgroups with no K split:
// 9.8 against 16.2 us for 128 x 96 tiles in two K parts).
struct I8PTile {
  int sn, tm;
};

I8PTile i8p_tile(int64_t rows, int64_t cols, int64_t n) {
  const int64_t gn = (rows + 31) / 32;
  const int B = (int)(cols / kBlock);
  I8PTile best{3, 4};
  double best_ns = -1.0;
  for (int tmg = 4; tmg >= 2; tmg -= 2) {
    const int par = kWaves / tmg;
    const int64_t tm = (n + tmg * kTokens - 1) / (tmg * kTokens);
    for (int sn = 3; sn <= (tmg == 4 ? 5 : 4); sn++) {
      const int64_t tiles = tm * ((gn + sn - 1) / sn);
      if (tiles > 0x7fffffff) continue;
      const int per = i8_split_blocks((int)tiles, B);
      const int64_t splits = (B + per - 1) / per;
      const int64_t rounds = (tiles * splits + 255) / 256;
      // 64-token tiles: each staged weight serves half the tokens, about
      // 1.2x the time per tile and block (measured).
      const double step_ns = tmg == 4 ? 100.0 : 120.0;
      double ns = (double)rounds * (2.0 * sn * ((per + par - 1) / par) * step_ns + 2000.0);
      if (splits > 1) ns += 1000.0 + (double)splits * (double)n * (double)rows / 1000.0;
      if (best_ns < 0.0 || ns < best_ns) {
        best = {sn, tmg};
        best_ns = ns;
      }
    }
  }
  return best;
}

template <int SN, int kTM>
int launch_i8p(const uint8_t* packed, const uint8_t* panel, float* y, int64_t rows, int64_t cols,
               int64_t n, hipStream_t stream) {
  constexpr int BN = SN * 32;
  F6PParams p{};
  p.packed = packed;
  p.panel = panel;
  p.y = y;
  p.rows = (int)rows;
  p.cols = (int)cols;
  p.n = (int)n;
  p.tiles_m = (int)((n + kTM * kTokens - 1) / (kTM * kTokens));
  p.tiles = p.tiles_m * (int)((rows + BN - 1) / BN);
  const int B = (int)(cols / kBlock);
  p.split_blocks = i8_split_blocks(p.tiles, B);
  const int splits = (B + p.split_blocks - 1) / p.split_blocks;
  const int64_t count = n * rows;
  p.part = nullptr;
  if (splits > 1) {
    p.part = part_workspace((size_t)splits * count * 4);
    if (p.part == nullptr) return DNX_ENOMEM;
  }
  p.vec = (rows % 4 == 0 && ((uintptr_t)(p.part ? (void*)p.part : (void*)y) & 15) == 0) ? 1 : 0;
  hipLaunchKernelGGL((gemm_i8p_kernel<SN, kTM>), dim3((unsigned)p.tiles, (unsigned)splits),
                     dim3(kThreads), 0, stream, p);
  if (hipGetLastError() != hipSuccess) return DNX_ELAUNCH;
  if (splits > 1) {
    const int64_t blocks = (count + 255) / 256;
    hipLaunchKernelGGL(f6_splitk_reduce_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)),
                       dim3(256), 0, stream, p.part, y, count, splits);
    if (hipGetLastError() != hipSuccess) return DNX_ELAUNCH;
  }
  return DNX_OK;
}

int panel_grid(int64_t total) {
  const int64_t blocks = (total + kPanelThreads - 1) / kPanelThreads;
  return (int)(blocks < 16384 ? blocks : 16384);
}

}  // namespace

extern "C" {

int64_t dnx_f6_panel_bytes(int64_t n, int64_t cols) {
  if (n <= 0 || cols <= 0 || cols % kBlock != 0) return -1;
  return f6_panel_bytes(n, cols);
}

int dnx_swiglu_f6panel(float* g, const float* u, void* panel, int64_t n, int64_t cols,
                       dnx_stream_t stream) {
  if (n <= 0 || cols <= 0 || cols % kBlock != 0 || ((uintptr_t)g & 15) || ((uintptr_t)u & 15) ||
      ((uintptr_t)panel & 15) || f6_panel_bytes(n, cols) >= (1ll << 31)) {
    return DNX_EINVAL;
  }
  const int groups = (int)((n + kTokens - 1) / kTokens);
  const int64_t total = (int64_t)groups * (cols / kBlock) * kTokens * 4;
  hipLaunchKernelGGL(swiglu_f6panel_kernel, dim3(panel_grid(total)), dim3(kPanelThreads), 0,
                     (hipStream_t)stream, g, u, (uint8_t*)panel, (int)n, (int)cols, groups);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int dnx_quantize_q8_f6panel(const float* x, void* panel, int64_t n, int64_t cols,
                            dnx_stream_t stream) {
  if (n <= 0 || cols <= 0 || cols % kBlock != 0 || ((uintptr_t)x & 15) ||
      ((uintptr_t)panel & 15) || f6_panel_bytes(n, cols) >= (1ll << 31)) {
    return DNX_EINVAL;
  }
  const int groups = (int)((n + kTokens - 1) / kTokens);
  const int64_t total = (int64_t)groups * (cols / kBlock) * kTokens * 4;
  hipLaunchKernelGGL(quantize_f6_panel4_kernel, dim3(panel_grid(total)), dim3(kPanelThreads), 0,
                     (hipStream_t)stream, x, (uint8_t*)panel, (int)n, (int)cols, groups);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int dnx_pack_f6panel(const int8_t* xq, const float* xsc, void* panel, int64_t n, int64_t cols,
                     dnx_stream_t stream) {
  if (n <= 0 || cols <= 0 || cols % kBlock != 0 || ((uintptr_t)xq & 15) || (cols % 16) ||
      ((uintptr_t)panel & 15) || f6_panel_bytes(n, cols) >= (1ll << 31)) {
    return DNX_EINVAL;
  }
  const int groups = (int)((n + kTokens - 1) / kTokens);
  const int64_t total = (int64_t)groups * (cols / kBlock) * kTokens;
  hipLaunchKernelGGL(pack_f6_panel_kernel, dim3(panel_grid(total)), dim3(kPanelThreads), 0,
                     (hipStream_t)stream, xq, xsc, (uint8_t*)panel, (int)n, (int)cols, groups);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int dnx_gemm_q4_f6(const uint8_t* qs, const uint16_t* scales, const void* panel, float* y,
                   int64_t rows, int64_t cols, int64_t n, dnx_stream_t stream) {
  if (!f6_shape_ok(rows, cols, n) || ((uintptr_t)panel & 15) || ((uintptr_t)qs & 15) ||
      ((uintptr_t)scales & 1) || ((uintptr_t)y & 3)) {
    return DNX_EINVAL;
  }
  return launch_f6<3>(qs, scales, (const uint8_t*)panel, y, rows, cols, n, (hipStream_t)stream);
}

int64_t dnx_q4_f6pack_bytes(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0 || cols % kBlock != 0) return -1;
  return (rows + 31) / 32 * (cols / kBlock) * kChunk;
}

int dnx_pack_q4_f6(const uint8_t* qs, const uint16_t* scales, void* packed, int64_t rows,
                   int64_t cols, dnx_stream_t stream) {
  if (rows <= 0 || cols <= 0 || cols % kBlock != 0 || rows >= (1ll << 31) || ((uintptr_t)qs & 15) ||
      ((uintptr_t)scales & 1) || ((uintptr_t)packed & 15)) {
    return DNX_EINVAL;
  }
  const int64_t count = (rows + 31) / 32 * 32 * (cols / kBlock);
  hipLaunchKernelGGL(pack_q4_f6_kernel, dim3(panel_grid(count)), dim3(kPanelThreads), 0,
                     (hipStream_t)stream, qs, scales, (uint8_t*)packed, (int)rows,
                     (int)(cols / kBlock), count);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int dnx_gemm_q4_f6p(const void* packed, const void* panel, float* y, int64_t rows, int64_t cols,
                    int64_t n, dnx_stream_t stream) {
  if (!f6p_shape_ok(rows, cols, n) || ((uintptr_t)panel & 15) || ((uintptr_t)packed & 15) ||
      ((uintptr_t)y & 3)) {
    return DNX_EINVAL;
  }
  return launch_f6p<3>((const uint8_t*)packed, (const uint8_t*)panel, y, rows, cols, n,
                       (hipStream_t)stream);
}

int dnx_gemm_q4_f6s(const void* packed, const void* panel, float* y, int64_t rows, int64_t cols,
                    int64_t n, dnx_stream_t stream) {
  return dnx_gemm_q4_f6s_multi(&packed, &y, &rows, 1, panel, cols, n, stream);
}

int dnx_gemm_q4_f6s_multi(const void* const* packed, float* const* y, const int64_t* rows,
                          int count, const void* panel, int64_t cols, int64_t n,
                          dnx_stream_t stream) {
  if (count < 1 || count > kMaxSegs || n > 65535 * 2 * kTokens || ((uintptr_t)panel & 15)) {
    return DNX_EINVAL;
  }
  F6SParams p{};
  p.panel = (const uint8_t*)panel;
  p.cols = (int)cols;
  p.n = (int)n;
  p.segs = count;
  int64_t groups = 0;
  for (int k = 0; k < count; k++) {
    if (!f6p_shape_ok(rows[k], cols, n) || ((uintptr_t)packed[k] & 15) ||
        ((uintptr_t)y[k] & 3)) {
      return DNX_EINVAL;
    }
    groups += (rows[k] + 31) / 32;
    if (groups > 0x7fffffff) return DNX_EINVAL;
    p.seg_end[k] = (int)groups;
    p.packed[k] = (const uint8_t*)packed[k];
    p.y[k] = y[k];
    p.rows[k] = (int)rows[k];
  }
  // Token groups of 32 per workgroup (one weight read for all of them):
  // the fewest that keep the launch to one round of 256 workgroups (a
  // workgroup fills its CU's registers, so more run in two rounds: 64
  // tokens of 6144 x 2048 take 192 workgroups of two groups in 6.5 us
  // against 7.9 with 384 of one; 375 tokens of 768 x 768, 144 of two in 4.3
  // us against 6.2 with 288 of one). Three groups fit the registers only
  // with a wave's blocks all loaded at once (K up to 1024), and are taken
  // only where they make one round (375 tokens of 1792 x 768: 5.8 us against
  // 7.4 with two groups; two rounds of three groups were slower than two
  // of two).
  const int nb = (int)(cols / kBlock + kWaves - 1) / kWaves;
  auto workgroups = [&](int64_t g) { return groups * ((n + g * kTokens - 1) / (g * kTokens)); };
  int G = 1;
  if (n > kTokens && workgroups(1) > 256) {
    G = (n > 2 * kTokens && workgroups(2) > 256 && workgroups(3) <= 256 && nb <= 4) ? 3 : 2;
  }
  const int per = G * kTokens;
  // Two 32-row groups per workgroup where the launch would otherwise need
  // more than one round (a chunk's gate and up: 384 workgroups of two token
  // groups -> 192).
  const int RG = (G == 2 && nb > 4 && workgroups(2) > 256) ? 2 : 1;
  int64_t wgs = 0;
  for (int k = 0; k < count; k++) {
    wgs += ((rows[k] + 31) / 32 + RG - 1) / RG;
    p.seg_end[k] = (int)wgs;
  }
  const dim3 grid((unsigned)wgs, (unsigned)((n + per - 1) / per));
  // A wave's blocks all loaded at once where they fit the ring (one round
  // trip: 8 blocks of one token group, 4 of two or three), else a ring of 4.
  if (RG == 2) {
    // A ring of 3 (4 spills with two row groups' fragments).
    hipLaunchKernelGGL((gemm_f6s_kernel<2, 3, false, 2>), grid, dim3(kThreads), 0,
                       (hipStream_t)stream, p);
  } else if (G == 3) {
    hipLaunchKernelGGL((gemm_f6s_kernel<3, 4, true>), grid, dim3(kThreads), 0,
                       (hipStream_t)stream, p);
  } else if (G == 2) {
    if (nb <= 4) {
      hipLaunchKernelGGL((gemm_f6s_kernel<2, 4, true>), grid, dim3(kThreads), 0,
                         (hipStream_t)stream, p);
    } else {
      hipLaunchKernelGGL((gemm_f6s_kernel<2, 4, false>), grid, dim3(kThreads), 0,
                         (hipStream_t)stream, p);
    }
  } else if (nb <= 4) {
    hipLaunchKernelGGL((gemm_f6s_kernel<1, 4, true>), grid, dim3(kThreads), 0,
                       (hipStream_t)stream, p);
  } else if (nb <= 8) {
    hipLaunchKernelGGL((gemm_f6s_kernel<1, 8, true>), grid, dim3(kThreads), 0,
                       (hipStream_t)stream, p);
  } else {
    hipLaunchKernelGGL((gemm_f6s_kernel<1, 4, false>), grid, dim3(kThreads), 0,
                       (hipStream_t)stream, p);
  }
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int64_t dnx_q8_f6pack_bytes(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0 || cols % kBlock != 0) return -1;
  return (rows + 31) / 32 * (cols / kBlock) * kChunk8;
}

int dnx_pack_q8_f6(const int8_t* qs, const float* scales, void* packed, int64_t rows,
                   int64_t cols, dnx_stream_t stream) {
  if (rows <= 0 || cols <= 0 || cols % kBlock != 0 || rows >= (1ll << 31) || ((uintptr_t)qs & 15) ||
      ((uintptr_t)scales & 3) || ((uintptr_t)packed & 15)) {
    return DNX_EINVAL;
  }
  const int64_t count = (rows + 31) / 32 * 32 * (cols / kBlock);
  hipLaunchKernelGGL(pack_q8_f6_kernel, dim3(panel_grid(count)), dim3(kPanelThreads), 0,
                     (hipStream_t)stream, qs, scales, (uint8_t*)packed, (int)rows,
                     (int)(cols / kBlock), count);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int dnx_gemm_q8_f6p(const void* packed, const void* panel, float* y, int64_t rows, int64_t cols,
                    int64_t n, dnx_stream_t stream) {
  if (!f6p_shape_ok(rows, cols, n, true) || ((uintptr_t)panel & 15) ||
      ((uintptr_t)packed & 15) || ((uintptr_t)y & 3)) {
    return DNX_EINVAL;
  }
  return launch_f6p<3, true>((const uint8_t*)packed, (const uint8_t*)panel, y, rows, cols, n,
                             (hipStream_t)stream);
}

int64_t dnx_i8_panel_bytes(int64_t n, int64_t cols) {
  if (n <= 0 || cols <= 0 || cols % kBlock != 0) return -1;
  return i8_panel_bytes(n, cols);
}

int dnx_quantize_q8_i8panel(const float* x, void* panel, int64_t n, int64_t cols,
                            dnx_stream_t stream) {
  if (n <= 0 || cols <= 0 || cols % kBlock != 0 || ((uintptr_t)x & 15) ||
      ((uintptr_t)panel & 15) || i8_panel_bytes(n, cols) >= (1ll << 31)) {
    return DNX_EINVAL;
  }
  const int groups = (int)((n + kTokens - 1) / kTokens);
  const int64_t total = (int64_t)groups * (cols / kBlock) * kTokens * 4;
  hipLaunchKernelGGL(quantize_i8_panel_kernel, dim3(panel_grid(total)), dim3(kPanelThreads), 0,
                     (hipStream_t)stream, x, (uint8_t*)panel, (int)n, (int)cols, groups);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int64_t dnx_q8_i8pack_bytes(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0 || cols % kBlock != 0) return -1;
  return (rows + 31) / 32 * (cols / kBlock) * kI8Rec;
}

int dnx_pack_q8_i8(const int8_t* qs, const float* scales, void* packed, int64_t rows,
                   int64_t cols, dnx_stream_t stream) {
  if (rows <= 0 || cols <= 0 || cols % kBlock != 0 || rows >= (1ll << 31) ||
      ((uintptr_t)qs & 15) || ((uintptr_t)scales & 3) || ((uintptr_t)packed & 15)) {
    return DNX_EINVAL;
  }
  const int64_t count = (rows + 31) / 32 * 32 * (cols / kBlock);
  hipLaunchKernelGGL(pack_q8_i8_kernel, dim3(panel_grid(count)), dim3(kPanelThreads), 0,
                     (hipStream_t)stream, qs, scales, (uint8_t*)packed, (int)rows,
                     (int)(cols / kBlock), count);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int dnx_gemm_q8_i8p(const void* packed, const void* panel, float* y, int64_t rows, int64_t cols,
                    int64_t n, dnx_stream_t stream) {
  if (!i8p_shape_ok(rows, cols, n) || ((uintptr_t)panel & 15) || ((uintptr_t)packed & 15) ||
      ((uintptr_t)y & 3)) {
    return DNX_EINVAL;
  }
  const uint8_t* pk = (const uint8_t*)packed;
  const uint8_t* pn = (const uint8_t*)panel;
  const I8PTile tile = i8p_tile(rows, cols, n);
  const hipStream_t st = (hipStream_t)stream;
  if (tile.tm == 2) {
    return tile.sn == 4 ? launch_i8p<4, 2>(pk, pn, y, rows, cols, n, st)
                        : launch_i8p<3, 2>(pk, pn, y, rows, cols, n, st);
  }
  switch (tile.sn) {
    case 5: return launch_i8p<5, 4>(pk, pn, y, rows, cols, n, st);
    case 4: return launch_i8p<4, 4>(pk, pn, y, rows, cols, n, st);
    default: return launch_i8p<3, 4>(pk, pn, y, rows, cols, n, st);
  }
}

int dnx_gemm_q8_i8p_tile(int64_t rows, int64_t cols, int64_t n, int* tile_rows,
                         int* tile_tokens) {
  if (!i8p_shape_ok(rows, cols, n) || tile_rows == nullptr || tile_tokens == nullptr) {
    return DNX_EINVAL;
  }
  const I8PTile tile = i8p_tile(rows, cols, n);
  *tile_rows = 32 * tile.sn;
  *tile_tokens = kTokens * tile.tm;
  return DNX_OK;
}

int64_t dnx_gemm_q4_f6p_noalloc_max_floats(void) { return (int64_t)kScratchFloats; }

int dnx_gemm_q4_f6p_noalloc(const void* packed, const void* panel, float* y, int64_t rows,
                            int64_t cols, int64_t n, dnx_stream_t stream) {
  if (!f6p_shape_ok(rows, cols, n) || ((uintptr_t)panel & 15) || ((uintptr_t)packed & 15) ||
      ((uintptr_t)y & 3)) {
    return DNX_EINVAL;
  }
  float* part = scratch_on_device();
  if (part == nullptr) return DNX_ESCRATCH;
  return launch_f6p<3>((const uint8_t*)packed, (const uint8_t*)panel, y, rows, cols, n,
                       (hipStream_t)stream, part, kScratchFloats);
}

}  // extern "C"
