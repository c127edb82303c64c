// Prefill / vision-encoder GEMM for large n on gfx950 fp16 and bf16 MFMA:
//   y[m][r] = sum_b sx[m][b] * sw[r][b] * D_b[m][r],
//   D_b[m][r] = sum over block b of xq[m][k] * w[r][k]   (w = q - 8 for Q4).
//
// Why not int8 MFMA. One v_mfma_i32_32x32x32_i8 gives a block's 32 x 32
// int32 dots in 32 clocks per SIMD, but applying the block's scales then
// costs three VALU operations per output (cvt, s = sx * sw, fma): 48
// wave64 instructions, 192 clocks, so the int8 kernel cannot pass about
// 1/6 of the int8 peak. Here:
//   * D_b comes from two v_mfma_f32_32x32x16_f16 on integer-valued fp16
//     operands (|xq| <= 127, |w| <= 127 are exact in fp16; every partial sum
//     is an integer below 2^24, so D_b is exact and already a float: no cvt).
//   * s = sx * sw for the whole 32 x 32 tile comes from one
//     v_mfma_f32_32x32x16_bf16 used as an outer product: each scale is split
//     into three bf16 pieces (x0 + x1 + x2 == sx exactly, likewise w), and
//     the six products x_i * w_j with i + j <= 2 sit in six of its 16 K slots.
//     The dropped terms are below 3 * 2^-24 relative, and the MFMA rounds
//     their sum once: s matches the rounded product sx * sw to ~2^-23.
//   * The epilogue is one fma per output per block: acc = fma(D, s, acc),
//     blocks in order, as lab_native.c:509-510 accumulates per lane.
// Per 32 x 32 tile and block: 96 MFMA clocks (64 + 32) against 16 VALU
// instructions (64 clocks), so the bound is the MFMA pipe at one third of
// the int8 peak instead of the VALU at one sixth.
//
// Operands. Activations arrive as a "panel" (dnx_gemm_panel_* below): per
// group of 32 token rows and per block, the two fp16 A fragments of the
// block in MFMA lane order (2 KB) and the bf16 scale pieces (512 B), so a
// wave loads its A operands with fully coalesced 16-byte loads straight
// into registers, a stage ahead. Weights are staged through LDS once per
// workgroup and shared by its 4 waves (4 x 32 token rows): a Q4 byte pair
// becomes fp16 (q - 8) with one v_perm_b32 (the nibble under the fp16
// exponent of 1024) and one packed fp16 subtract of 1032; Q8 bytes the
// same way with 1152. The weight scales are split into bf16 pieces once
// per workgroup as well.
//
// Workgroup: 256 threads, 4 waves along M (32 rows each), SN x 32 weight
// rows; tile t of a launch whose tile count is a multiple of 8 is remapped
// so that each XCD (workgroups are dealt round-robin to the 8 XCDs) owns a
// contiguous run of weight-row tiles with all their token tiles: every
// weight tile is fetched into one L2 only.

#include "common.h"
#include "dnx_kernels.h"

using namespace dnx;

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short s4 __attribute__((ext_vector_type(4)));   // 4 bf16 (bits)

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kRowsPerWave = 32;
constexpr int kBM = kWaves * kRowsPerWave;   // token rows per workgroup
constexpr int kPanelA = 2048;                // fp16 fragments of one (group, block)
constexpr int kPanelS = 512;                 // bf16 scale pieces of one (group, block)
constexpr int kPanelBlock = kPanelA + kPanelS;

// Two bytes of `v` (selected by `sel`) as the fp16 pair (1024 + byte),
// minus `bias` from both halves: exact for bytes 0..255.
DNX_DEV uint32_t bytes_to_h2(uint32_t v, uint32_t sel, _Float16 bias) {
  const uint32_t t = __builtin_amdgcn_perm(0x64646464u, v, sel);
  const h2 r = __builtin_bit_cast(h2, t) - h2{bias, bias};
  return __builtin_bit_cast(uint32_t, r);
}
constexpr uint32_t kSel01 = 0x04010400u;  // bytes [v0, 0x64, v1, 0x64]
constexpr uint32_t kSel23 = 0x04030402u;  // bytes [v2, 0x64, v3, 0x64]

// 8 weights of 4 bytes each in two dwords -> one 16-byte fp16 fragment.
DNX_DEV uint4 frag_from_bytes(uint32_t a, uint32_t b, _Float16 bias) {
  return make_uint4(bytes_to_h2(a, kSel01, bias), bytes_to_h2(a, kSel23, bias),
                    bytes_to_h2(b, kSel01, bias), bytes_to_h2(b, kSel23, bias));
}

// ---------------------------------------------------------------- the panel

// xq int8 [n][cols] + xsc fp32 [n][cols/32] -> panel [groups][B][2560 B].
// Fragment h (K half) of lane l: row 32g + l % 32, k = 16h + 8(l / 32) + 0..7.
// Rows past n are zeros. One thread per (row, block); consecutive threads
// take consecutive rows of a group, so the 16-byte stores are contiguous.
__global__ void __launch_bounds__(kThreads) pack_panel_kernel(const int8_t* __restrict__ xq,
                                                              const float* __restrict__ xsc,
                                                              uint8_t* __restrict__ panel,
                                                              int n, int cols, int groups) {
  const int B = cols / kBlock;
  const int64_t total = (int64_t)groups * kRowsPerWave * B;
  for (int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * kThreads) {
    const int r = (int)(idx % kRowsPerWave);
    const int64_t gb = idx / kRowsPerWave;
    const int b = (int)(gb % B);
    const int g = (int)(gb / B);
    const int m = g * kRowsPerWave + r;
    uint8_t* dst = panel + gb * kPanelBlock;
    uint4 w[8];
    float sx = 0.0f;
    if (m < n) {
      const uint4* src = (const uint4*)(xq + (int64_t)m * cols + b * kBlock);
      const uint4 lo = src[0], hi = src[1];
      const uint32_t v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
      for (int i = 0; i < 4; i++) w[i] = frag_from_bytes(v[2 * i] ^ 0x80808080u,
                                                        v[2 * i + 1] ^ 0x80808080u,
                                                        (_Float16)1152.0f);
      sx = xsc[(int64_t)m * B + b];
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) w[i] = make_uint4(0, 0, 0, 0);
    }
    // w[i] holds k = 8i..8i+7: (h, kg) = (i / 2, i % 2).
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int h = i >> 1, kg = i & 1;
      *(uint4*)(dst + h * 1024 + (kg * 32 + r) * 16) = w[i];
    }
    uint32_t p0, p1, p2;
    split3_bf16(sx, p0, p1, p2);
    *(uint2*)(dst + kPanelA + r * 8) = a_scale_half0(p0, p1, p2);
    *(uint2*)(dst + kPanelA + (32 + r) * 8) = a_scale_half1(p0, p1, p2);
  }
}

// lab_quantize_q8 (lab_native.c:407-429) of fp32 x [n][cols] straight into
// the panel: the same values as dnx_quantize_q8 (bit-exact: the same block
// max, scale, 1/scale and rounding), stored as the fp16 fragments and bf16
// scale pieces the GEMM reads. One thread quantizes 4 consecutive values
// (8 threads share a block, as in the plain quantizer) over the padded rows
// of the last group, whose values are zeros.
__global__ void __launch_bounds__(kThreads) quantize_panel_kernel(const float* __restrict__ x,
                                                                  uint8_t* __restrict__ panel,
                                                                  int n, int cols, int groups) {
  const int B = cols / kBlock;
  const int64_t quads_per_row = cols / 4;
  const int64_t total = (int64_t)groups * kRowsPerWave * quads_per_row;
  for (int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x; q < total;
       q += (int64_t)gridDim.x * kThreads) {
    const int row = (int)(q / quads_per_row);
    const int c = (int)(q - (int64_t)row * quads_per_row) * 4;
    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (row < n) v = *(const float4*)(x + (int64_t)row * cols + c);
    const float amax = group8_max(fmaxf(0.0f, max4abs(v)));
    const float scale = q8_scale(amax);
    const float inv = q8_inv(scale);
    const int g = row / kRowsPerWave, r = row % kRowsPerWave, b = c / kBlock, kk = c % kBlock;
    uint8_t* dst = panel + ((int64_t)g * B + b) * kPanelBlock;
    const h4 h = {(_Float16)quant1(v.x, inv), (_Float16)quant1(v.y, inv),
                  (_Float16)quant1(v.z, inv), (_Float16)quant1(v.w, inv)};
    *(uint2*)(dst + (kk >> 4) * 1024 + (((kk >> 3) & 1) * 32 + r) * 16 + (kk & 7) * 2) =
        __builtin_bit_cast(uint2, h);
    if (kk == 0) {
      uint32_t p0, p1, p2;
      split3_bf16(scale, p0, p1, p2);
      *(uint2*)(dst + kPanelA + r * 8) = a_scale_half0(p0, p1, p2);
      *(uint2*)(dst + kPanelA + (32 + r) * 8) = a_scale_half1(p0, p1, p2);
    }
  }
}

// ----------------------------------------------------------------- the GEMM

struct Params {
  const void* qs;
  const void* scales;
  const uint8_t* panel;
  float* y;
  int rows, cols, n;
  int tiles_m, tiles;   // token tiles; all tiles of one K split
  int split_stages;     // K stages per split (blockIdx.y)
  float* part;          // split partials [splits][n][rows], or null
};

// Workgroup: 8 waves, 128 token rows x SN * 32 weight rows. Wave w takes
// the 32-row group w % 4 and the K half w / 4: in each stage of KB = 4
// blocks it computes blocks w / 4 and w / 4 + 2, so two waves share every
// SIMD (one hides the other's LDS, memory and MFMA latencies) while the
// staged weight tile is shared by all eight. The two halves' sums are added
// once at the end, through LDS, in a fixed order.
constexpr int kGemmThreads = 512;
constexpr int kKB = 4;          // blocks per stage
constexpr int kKH = kKB / 2;    // blocks per wave per stage

template <bool kQ4, int SN>
__global__ void __launch_bounds__(kGemmThreads) gemm_f16_kernel(Params p) {
  constexpr int KB = kKB, KH = kKH;
  constexpr int BN = SN * 32;
  constexpr int kPairs = BN * KB;                               // (weight row, block) per stage
  constexpr int PP = (kPairs + kGemmThreads - 1) / kGemmThreads;
  constexpr int kChunk = 2048 + 64;   // one (j, kb): two 1 KB K halves; +64 B spreads banks
  constexpr int kSChunk = 512 + 32;   // one (j, kb) of scale pieces; +32 B spreads banks
  constexpr int kStageBytes = SN * KB * (kChunk + kSChunk);
  // Threads without a (row, block) pair in a stage still convert one and
  // store it here: a branch around the staging makes the compiler spill
  // (values live across a divergent region).
  constexpr int kDummy = 80;
  constexpr int kStaging = 2 * kStageBytes + kDummy;
  constexpr int kRedBytes = kWaves * SN * 16 * 64 * 4;          // the second half's sums
  constexpr int kLds = kStaging > kRedBytes ? kStaging : kRedBytes;
  __shared__ __align__(16) uint8_t lds[kLds];
  auto sb = [&](int buf) { return lds + buf * kStageBytes; };
  auto ss = [&](int buf) { return lds + buf * kStageBytes + SN * KB * kChunk; };

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rg = wave & 3, kh = wave >> 2;
  const int K = p.cols, B = K / kBlock, M = p.n, N = p.rows;
  const int stages = (B + KB - 1) / KB;

  // XCD-aware tile order (see the file comment).
  const int i = blockIdx.x;
  const int t = (p.tiles % 8 == 0) ? (i % 8) * (p.tiles / 8) + i / 8 : i;
  const int mt = t % p.tiles_m, nt = t / p.tiles_m;
  const int n0 = nt * BN;
  const int g = mt * kWaves + rg;                   // this wave's 32-row group
  const int groups = (M + kRowsPerWave - 1) / kRowsPerWave;
  const bool live = g < groups;

  const i32x4 rpanel = buffer_rsrc(p.panel, (uint32_t)((size_t)groups * B * kPanelBlock));
  const i32x4 rqs = buffer_rsrc(p.qs, (uint32_t)((size_t)N * (kQ4 ? K / 2 : K)));
  const i32x4 rws = buffer_rsrc(p.scales, (uint32_t)((size_t)N * B * (kQ4 ? 2 : 4)));

  const int s_begin = blockIdx.y * p.split_stages;
  const int s_end = min(stages, s_begin + p.split_stages);

  // Weight staging: pair q = (row nn, block kb), kb fastest (coalesced rows).
  int offW[PP], offS[PP], cK[PP];
#pragma unroll
  for (int e = 0; e < PP; e++) {
    const int q = e * kGemmThreads + tid;
    const int nn = q / KB, kb = q - nn * KB, r = n0 + nn;
    const bool ok = q < kPairs && r < N;
    offW[e] = r * (kQ4 ? K / 2 : K) + kb * (kQ4 ? 16 : 32);
    offS[e] = (r * B + kb) * (kQ4 ? 2 : 4);
    cK[e] = ok ? kb : (1 << 30);
  }
  // Loaded values stay as loaded (the scale as its raw 16 or 32 bits) until
  // store_w: any operation on a loaded register, even a zero-extension,
  // makes the wave wait for that load where the operation is, which would
  // put the next stage's load latency in front of this stage's MFMAs.
  uint4 rw[PP][kQ4 ? 1 : 2];
  short rsh[PP];
  int rsi[PP];

  // Loads of a stage past this split's last read zeros (the bounded loads
  // make every load unconditional, so the compiler can count them).
  auto load_w = [&](int s) {
    const int b0 = s * KB;
    const int bend = s < s_end ? B : 0;
#pragma unroll
    for (int e = 0; e < PP; e++) {
      const bool ok = b0 + cK[e] < bend;
      const int o = ok ? offW[e] + b0 * (kQ4 ? 16 : 32) : -64;
      rw[e][0] = buffer_load16(rqs, o);
      if (!kQ4) rw[e][1] = buffer_load16(rqs, o + 16);
      if (kQ4) {
        rsh[e] = dnx_raw_buffer_load_i16(rws, ok ? offS[e] + b0 * 2 : -4, 0, 0);
      } else {
        rsi[e] = dnx_raw_buffer_load_i32(rws, ok ? offS[e] + b0 * 4 : -4, 0, 0);
      }
    }
  };

  auto store_w = [&](int buf) {
#pragma unroll
    for (int e = 0; e < PP; e++) {
      const int q = e * kGemmThreads + tid;
      const bool real = q < kPairs;
      const int nn = q / KB, kb = q - nn * KB, j = nn >> 5, c = nn & 31;
      uint8_t* dst = real ? sb(buf) + (j * KB + kb) * kChunk : lds + 2 * kStageBytes;
      uint4 f[4];
      if (kQ4) {
        const uint4 v = rw[e][0];
        const uint32_t m4 = 0x0f0f0f0fu;
        const _Float16 bias = (_Float16)1032.0f;
        f[0] = frag_from_bytes(v.x & m4, v.y & m4, bias);
        f[1] = frag_from_bytes(v.z & m4, v.w & m4, bias);
        f[2] = frag_from_bytes((v.x >> 4) & m4, (v.y >> 4) & m4, bias);
        f[3] = frag_from_bytes((v.z >> 4) & m4, (v.w >> 4) & m4, bias);
      } else {
        const uint4 a = rw[e][0], b = rw[e][1];
        const uint32_t x = 0x80808080u;
        const _Float16 bias = (_Float16)1152.0f;
        f[0] = frag_from_bytes(a.x ^ x, a.y ^ x, bias);
        f[1] = frag_from_bytes(a.z ^ x, a.w ^ x, bias);
        f[2] = frag_from_bytes(b.x ^ x, b.y ^ x, bias);
        f[3] = frag_from_bytes(b.z ^ x, b.w ^ x, bias);
      }
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int h = u >> 1, kg = u & 1;
        *(uint4*)(dst + (real ? h * 1024 + (kg * 32 + c) * 16 : u * 16)) = f[u];
      }
      const float w = kQ4 ? half_bits_to_float((uint16_t)rsh[e]) : __int_as_float(rsi[e]);
      uint32_t p0, p1, p2;
      split3_bf16(w, p0, p1, p2);
      uint8_t* sd = real ? ss(buf) + (j * KB + kb) * kSChunk + c * 8 : lds + 2 * kStageBytes + 64;
      *(uint2*)sd = b_scale_half0(p0, p1, p2);
      *(uint2*)(sd + (real ? 256 : 8)) = b_scale_half1(p0, p1, p2);
    }
  };

  // This wave's activation operands of one stage (its KH blocks), from the
  // panel straight into registers; a block past K, a stage past this split
  // or a group past n reads as zeros.
  struct AStage {
    uint4 a[KH][2];
    uint2 s[KH];
  };
  auto load_a = [&](int s, AStage& r) {
    const int bend = live && s < s_end ? B : 0;
#pragma unroll
    for (int u = 0; u < KH; u++) {
      const int b = s * KB + kh + 2 * u;
      const int base = b < bend ? (g * B + b) * kPanelBlock : -4096;
      r.a[u][0] = buffer_load16(rpanel, base + lane * 16);
      r.a[u][1] = buffer_load16(rpanel, base + 1024 + lane * 16);
      const int so = base + kPanelA + lane * 8;
      r.s[u].x = (uint32_t)dnx_raw_buffer_load_i32(rpanel, so, 0, 0);
      r.s[u].y = (uint32_t)dnx_raw_buffer_load_i32(rpanel, so + 4, 0, 0);
    }
  };

  f32x16 acc[SN];
#pragma unroll
  for (int j = 0; j < SN; j++)
#pragma unroll
    for (int v = 0; v < 16; v++) acc[j][v] = 0.0f;

  // One stage: the wave's KH x SN output-tile steps, software-pipelined.
  // Step t reads the weight fragments of step t + 2 from LDS, issues its
  // three MFMAs, and runs the fmas of step t - 2, whose MFMA results (held
  // in the third of three D/S register sets) completed a whole step
  // earlier: the VALU never waits for the matrix pipe, and the SIMD's other
  // wave fills either pipe while this one waits. Blocks past K contribute
  // exact zeros (their activation fragments and scales read as zeros), so
  // the stage has no branches. The scale outer product uses the K = 8 bf16
  // MFMA: its 2-register operands hold the three used slots and the zero
  // slot of each lane half as loaded, with no zero registers to refill.
  constexpr int T = KH * SN;
  auto compute = [&](int buf, const AStage& r) {
    h8 fb0[3], fb1[3];
    s4 fbs[3];
    auto read_b = [&](int t, int slot) {
      const int u = t / SN, j = t - u * SN, kb = kh + 2 * u;
      const uint8_t* src = sb(buf) + (j * KB + kb) * kChunk;
      fb0[slot] = *(const h8*)(src + lane * 16);
      fb1[slot] = *(const h8*)(src + 1024 + lane * 16);
      fbs[slot] = *(const s4*)(ss(buf) + (j * KB + kb) * kSChunk + lane * 8);
    };
    f32x16 d[3], sc[3];
    auto fold = [&](int t) {
      const int j = t % SN;
#pragma unroll
      for (int v = 0; v < 16; v++) acc[j][v] = fmaf(d[t % 3][v], sc[t % 3][v], acc[j][v]);
    };
    read_b(0, 0);
    if (T > 1) read_b(1, 1);
#pragma unroll
    for (int t = 0; t < T; t++) {
      const int u = t / SN;
      if (t + 2 < T) read_b(t + 2, (t + 2) % 3);
      const h8 a0 = __builtin_bit_cast(h8, r.a[u][0]);
      const h8 a1 = __builtin_bit_cast(h8, r.a[u][1]);
      const s4 as = __builtin_bit_cast(s4, r.s[u]);
      const f32x16 z = {};
      sc[t % 3] = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(as, fbs[t % 3], z, 0, 0, 0);
      d[t % 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, fb0[t % 3], z, 0, 0, 0);
      d[t % 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, fb1[t % 3], d[t % 3], 0, 0, 0);
      if (t >= 2) fold(t - 2);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (T >= 2) fold(T - 2);
    fold(T - 1);
  };

  AStage ra, rb;
  load_w(s_begin);
  load_a(s_begin, ra);
  store_w(0);
  __syncthreads();

  // Two stages per iteration so that the two activation register sets swap
  // roles without copies.
  for (int s = s_begin; s < s_end; s += 2) {
    const int buf = (s - s_begin) & 1;
    load_w(s + 1);
    load_a(s + 1, rb);
    if (live) compute(buf, ra);
    store_w(buf ^ 1);
    __syncthreads();
    if (s + 1 >= s_end) break;
    load_w(s + 2);
    load_a(s + 2, ra);
    if (live) compute(buf ^ 1, rb);
    store_w(buf);
    __syncthreads();
  }

  // The K halves: the second half's sums go through LDS (the staging
  // buffers are free after the last barrier) to the first half's waves.
  float* red = (float*)lds + (size_t)rg * SN * 16 * 64;
  if (kh == 1 && live) {
#pragma unroll
    for (int j = 0; j < SN; j++)
#pragma unroll
      for (int v = 0; v < 16; v++) red[(j * 16 + v) * 64 + lane] = acc[j][v];
  }
  __syncthreads();
  if (kh == 1 || !live) return;
#pragma unroll
  for (int j = 0; j < SN; j++)
#pragma unroll
    for (int v = 0; v < 16; v++) acc[j][v] += red[(j * 16 + v) * 64 + lane];

  float* out = p.part ? p.part + (size_t)blockIdx.y * M * N : p.y;
#pragma unroll
  for (int j = 0; j < SN; j++) {
    const int r = n0 + j * 32 + (lane & 31);
    if (r >= N) continue;
#pragma unroll
    for (int v = 0; v < 16; v++) {
      const int m = g * kRowsPerWave + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
      if (m < M) store_wt(out + (size_t)m * N + r, acc[j][v]);
    }
  }
}

}  // namespace

namespace {

// y = the split partials summed in split order (deterministic).
__global__ void __launch_bounds__(kThreads) f16_splitk_reduce_kernel(const float* __restrict__ part,
                                                                     float* __restrict__ y,
                                                                     int64_t count, int splits) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < count;
       i += (int64_t)gridDim.x * kThreads) {
    float v = part[i];
    for (int z = 1; z < splits; z++) v += part[(size_t)z * count + i];
    store_wt(y + i, v);
  }
}

// Library-owned workspaces (the panel of dnx_gemm_q4/q8 and the split
// partials), grown on demand: a call at a larger shape than any before
// allocates, so such a call must not be the first inside a graph capture.
struct Workspace {
  void* ptr = nullptr;
  size_t bytes = 0;
  void* get(size_t need) {
    if (need <= bytes) return ptr;
    if (ptr != nullptr) {
      if (hipDeviceSynchronize() != hipSuccess) return nullptr;
      (void)hipFree(ptr);
      ptr = nullptr;
      bytes = 0;
    }
    if (hipMalloc(&ptr, need) != hipSuccess) {
      ptr = nullptr;
      return nullptr;
    }
    bytes = need;
    return ptr;
  }
};
Workspace gPanelWs, gPartWs;

int64_t panel_bytes(int64_t n, int64_t cols) {
  return (n + kRowsPerWave - 1) / kRowsPerWave * (cols / kBlock) * kPanelBlock;
}

template <bool kQ4, int SN>
int launch_f16(const void* qs, const void* scales, const uint8_t* panel, float* y, int64_t rows,
               int64_t cols, int64_t n, hipStream_t stream) {
  constexpr int BN = SN * 32;
  Params p{};
  p.qs = qs;
  p.scales = scales;
  p.panel = panel;
  p.y = y;
  p.rows = (int)rows;
  p.cols = (int)cols;
  p.n = (int)n;
  p.tiles_m = (int)((n + kBM - 1) / kBM);
  p.tiles = p.tiles_m * (int)((rows + BN - 1) / BN);
  const int stages = (int)((cols / kBlock + kKB - 1) / kKB);
  int splits = 1;
  if (p.tiles < 192 && stages > 1) {
    splits = (256 + p.tiles - 1) / p.tiles;
    if (splits > stages) splits = stages;
  }
  p.split_stages = (stages + splits - 1) / splits;
  splits = (stages + p.split_stages - 1) / p.split_stages;
  const int64_t count = n * rows;
  p.part = nullptr;
  if (splits > 1) {
    p.part = (float*)gPartWs.get((size_t)splits * count * 4);
    if (p.part == nullptr) return DNX_ENOMEM;
  }
  hipLaunchKernelGGL((gemm_f16_kernel<kQ4, SN>), dim3((unsigned)p.tiles, (unsigned)splits),
                     dim3(kGemmThreads), 0, stream, p);
  if (hipGetLastError() != hipSuccess) return DNX_ELAUNCH;
  if (splits > 1) {
    const int64_t blocks = (count + kThreads - 1) / kThreads;
    hipLaunchKernelGGL(f16_splitk_reduce_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)),
                       dim3(kThreads), 0, stream, p.part, y, count, splits);
    if (hipGetLastError() != hipSuccess) return DNX_ELAUNCH;
  }
  return DNX_OK;
}

bool shape_ok(int64_t rows, int64_t cols, int64_t n, bool q4) {
  if (rows <= 0 || cols <= 0 || n <= 0 || cols % kBlock != 0) return false;
  // 32-bit buffer offsets: each operand below 2 GB.
  return rows * (q4 ? cols / 2 : cols) < (1ll << 31) && panel_bytes(n, cols) < (1ll << 31) &&
         rows * (cols / kBlock) * 4 < (1ll << 31);
}

template <bool kQ4>
int gemm_panel(const void* qs, const void* scales, const uint8_t* panel, float* y, int64_t rows,
               int64_t cols, int64_t n, hipStream_t stream) {
  if (!shape_ok(rows, cols, n, kQ4) || ((uintptr_t)panel & 15) || ((uintptr_t)qs & 15)) {
    return DNX_EINVAL;
  }
  return launch_f16<kQ4, 3>(qs, scales, panel, y, rows, cols, n, stream);
}

}  // namespace

extern "C" {

int64_t dnx_gemm_panel_bytes(int64_t n, int64_t cols) {
  if (n <= 0 || cols <= 0 || cols % kBlock != 0) return -1;
  return panel_bytes(n, cols);
}

int dnx_pack_panel(const int8_t* xq, const float* xsc, void* panel, int64_t n, int64_t cols,
                   dnx_stream_t stream) {
  if (n <= 0 || cols <= 0 || cols % kBlock != 0 || ((uintptr_t)xq & 15) ||
      ((uintptr_t)panel & 15) || panel_bytes(n, cols) >= (1ll << 31)) {
    return DNX_EINVAL;
  }
  const int groups = (int)((n + kRowsPerWave - 1) / kRowsPerWave);
  const int64_t total = (int64_t)groups * kRowsPerWave * (cols / kBlock);
  const int64_t blocks = (total + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(pack_panel_kernel, dim3((unsigned)(blocks < 8192 ? blocks : 8192)),
                     dim3(kThreads), 0, (hipStream_t)stream, xq, xsc, (uint8_t*)panel, (int)n,
                     (int)cols, groups);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int dnx_quantize_q8_panel(const float* x, void* panel, int64_t n, int64_t cols,
                          dnx_stream_t stream) {
  if (n <= 0 || cols <= 0 || cols % kBlock != 0 || ((uintptr_t)x & 15) ||
      ((uintptr_t)panel & 15) || panel_bytes(n, cols) >= (1ll << 31)) {
    return DNX_EINVAL;
  }
  const int groups = (int)((n + kRowsPerWave - 1) / kRowsPerWave);
  const int64_t total = (int64_t)groups * kRowsPerWave * (cols / 4);
  const int64_t blocks = (total + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(quantize_panel_kernel, dim3((unsigned)(blocks < 16384 ? blocks : 16384)),
                     dim3(kThreads), 0, (hipStream_t)stream, x, (uint8_t*)panel, (int)n,
                     (int)cols, groups);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int dnx_gemm_q4_panel(const uint8_t* qs, const uint16_t* scales, const void* panel, float* y,
                      int64_t rows, int64_t cols, int64_t n, dnx_stream_t stream) {
  return gemm_panel<true>(qs, scales, (const uint8_t*)panel, y, rows, cols, n,
                          (hipStream_t)stream);
}

int dnx_gemm_q8_panel(const int8_t* qs, const float* scales, const void* panel, float* y,
                      int64_t rows, int64_t cols, int64_t n, dnx_stream_t stream) {
  return gemm_panel<false>(qs, scales, (const uint8_t*)panel, y, rows, cols, n,
                           (hipStream_t)stream);
}

}  // extern "C"
