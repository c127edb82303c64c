// Prefill / vision-encoder GEMM on gfx950 int8 MFMA with per-32-block
// scales: y[m][r] = sum_b sx[m][b] * sw[r][b] * D_b[m][r], where
// D_b = sum over block b of xq[m][k] * w[r][k] is an exact int32 from one
// v_mfma_i32_32x32x32_i8 (its K of 32 is exactly one Q block). The scale
// epilogue is fp32: cvt, s = sx * sw (rounded, as the CPU's s,
// lab_native.c:509), fma into the accumulator, block after block. The CPU
// keeps four partial lanes per block (lab_native.c:480-512); one lane per
// output here gives a different rounding, within 1e-4 relative.
//
// Roofline: per 32 x 32 output tile and block, one MFMA (32K MACs) against
// 3 x 16 VALU ops per lane for the epilogue (no packed fp32 here): the
// epilogue, not the MFMA, bounds this kernel (about 1/6 of the int8 peak
// when VALU and MFMA overlap perfectly).
//
// Workgroup tile: BM tokens x BN weight rows, 4 waves in a WM x WN grid,
// each wave (BM/WM) x (BN/WN) of 32 x 32 MFMA subtiles. K is staged KB
// blocks at a time in LDS (double buffered through registers): activations
// as int8, weights unpacked to int8 (Q4 nibbles -> q - 8 once per stage,
// shared by all BM tokens), scales as fp32. Small tiles keep enough
// workgroups resident (several waves per SIMD) for MFMA and VALU to overlap.

#include "common.h"
#include "dnx_kernels.h"

using namespace dnx;

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef short s4 __attribute__((ext_vector_type(4)));   // 4 bf16 (bits)

constexpr int kThreads = 256;

struct GemmParams {
  const void* qs;
  const void* scales;
  const int8_t* xq;
  const float* xsc;
  float* y;
  int rows, cols, n;
  int split_stages;  // K stages per split (blockIdx.z); all of K without split
  float* part;       // split partials [splits][n][rows], or null: write y
};

// Q4 byte-dword of 4 nibble pairs -> two dwords of int8 weights q - 8:
// low nibbles (weights k) and high nibbles (weights k + 16).
DNX_DEV void unpack_q4(uint32_t v, uint32_t& lo, uint32_t& hi) {
  const uint32_t m = 0x0f0f0f0fu;
  // (q | 0x80) - 8 never borrows across bytes; ^ 0x80 gives q - 8 as int8.
  lo = (((v & m) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
  hi = ((((v >> 4) & m) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
}

template <bool kQ4, int BM, int BN, int WM, int KB>
__global__ void __launch_bounds__(kThreads) gemm_kernel(GemmParams p) {
  constexpr int WN = 4 / WM;
  constexpr int TM = BM / WM, TN = BN / WN;   // wave tile
  constexpr int SM = TM / 32, SN = TN / 32;   // 32x32 subtiles per wave
  static_assert(SM >= 1 && SN >= 1, "wave tile below one MFMA tile");
  constexpr int RB = KB * 32;                 // bytes of a row per stage
  constexpr int RS = RB + 16;                 // LDS row stride (bank spread)
  __shared__ __align__(16) int8_t sa[2][BM * RS];
  __shared__ __align__(16) int8_t sb[2][BN * RS];
  // Block scales as bf16 pieces of the outer-product MFMA (two 8-byte lane
  // halves per row or column and block).
  __shared__ __align__(16) uint2 sxs[2][KB][BM][2];
  __shared__ __align__(16) uint2 sws[2][KB][BN][2];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave - (wave / WN) * WN;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int K = p.cols, B = K / kBlock, M = p.n, N = p.rows;
  const int stages = (B + KB - 1) / KB;

  // Staging of one stage through registers, with bounded buffer loads
  // (rows past the matrix, blocks past K read as zeros).
  constexpr int A16 = BM * RB / 16;                 // 16-byte pieces of A per stage
  constexpr int B16 = BN * (kQ4 ? RB / 2 : RB) / 16;
  constexpr int AP = (A16 + kThreads - 1) / kThreads;
  constexpr int BP = (B16 + kThreads - 1) / kThreads;
  constexpr int SXP = (KB * BM + kThreads - 1) / kThreads;
  constexpr int SWP = (KB * BN + kThreads - 1) / kThreads;
  // Loaded values stay as loaded (Q4 scales as their raw 16 bits) until
  // store_stage: any operation on a loaded register, even a zero-extension,
  // makes the wave wait for that load where the operation is, which would
  // put the next stage's load latency in front of this stage's MFMAs.
  uint4 ra[AP], rb[BP];
  float rsx[SXP], rsw[SWP];
  short rsh[SWP];
  const i32x4 rxq = buffer_rsrc(p.xq, (uint32_t)((size_t)M * K));
  const i32x4 rqs = buffer_rsrc(p.qs, (uint32_t)((size_t)N * (kQ4 ? K / 2 : K)));
  const i32x4 rxs = buffer_rsrc(p.xsc, (uint32_t)((size_t)M * B * 4));
  const i32x4 rws = buffer_rsrc(p.scales, (uint32_t)((size_t)N * B * (kQ4 ? 2 : 4)));

  // Per-thread offsets at stage 0 and each piece's block within a stage
  // (kNever when its row lies past the matrix): a stage adds b0 blocks'
  // bytes, and a piece whose block is past K reads zeros (offset -16 lies
  // outside the buffer). 32-bit offsets: the launch refuses operands of 2 GB.
  constexpr int kNever = 1 << 30;
  int offA[AP], cA[AP], offB[BP], cB[BP], offX[SXP], cX[SXP], offW[SWP], cW[SWP];
#pragma unroll
  for (int i = 0; i < AP; i++) {
    const int idx = i * kThreads + tid;
    const int row = idx / (RB / 16), seg = idx - row * (RB / 16), m = m0 + row;
    offA[i] = m * K + seg * 16;
    cA[i] = idx < A16 && m < M ? seg / 2 : kNever;
  }
#pragma unroll
  for (int i = 0; i < BP; i++) {
    const int idx = i * kThreads + tid;
    if (kQ4) {
      const int row = idx / KB, kb = idx - row * KB, r = n0 + row;
      offB[i] = r * (K / 2) + kb * 16;
      cB[i] = idx < B16 && r < N ? kb : kNever;
    } else {
      const int row = idx / (RB / 16), seg = idx - row * (RB / 16), r = n0 + row;
      offB[i] = r * K + seg * 16;
      cB[i] = idx < B16 && r < N ? seg / 2 : kNever;
    }
  }
#pragma unroll
  for (int i = 0; i < SXP; i++) {
    const int idx = i * kThreads + tid;
    const int kb = idx / BM, m = m0 + idx - kb * BM;
    offX[i] = (m * B + kb) * 4;
    cX[i] = idx < KB * BM && m < M ? kb : kNever;
  }
#pragma unroll
  for (int i = 0; i < SWP; i++) {
    const int idx = i * kThreads + tid;
    const int kb = idx / BN, r = n0 + idx - kb * BN;
    offW[i] = (r * B + kb) * (kQ4 ? 2 : 4);
    cW[i] = idx < KB * BN && r < N ? kb : kNever;
  }

  auto load_stage = [&](int s) {
    const int b0 = s * KB;
#pragma unroll
    for (int i = 0; i < AP; i++)
      ra[i] = buffer_load16(rxq, b0 + cA[i] < B ? offA[i] + b0 * 32 : -16);
#pragma unroll
    for (int i = 0; i < BP; i++)
      rb[i] = buffer_load16(rqs, b0 + cB[i] < B ? offB[i] + b0 * (kQ4 ? 16 : 32) : -16);
#pragma unroll
    for (int i = 0; i < SXP; i++) {
      rsx[i] = __int_as_float(
          dnx_raw_buffer_load_i32(rxs, b0 + cX[i] < B ? offX[i] + b0 * 4 : -4, 0, 0));
    }
#pragma unroll
    for (int i = 0; i < SWP; i++) {
      if (kQ4) {
        rsh[i] = dnx_raw_buffer_load_i16(rws, b0 + cW[i] < B ? offW[i] + b0 * 2 : -2, 0, 0);
      } else {
        rsw[i] = __int_as_float(
            dnx_raw_buffer_load_i32(rws, b0 + cW[i] < B ? offW[i] + b0 * 4 : -4, 0, 0));
      }
    }
  };

  auto store_stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < AP; i++) {
      const int idx = i * kThreads + tid;
      if (idx < A16) {
        const int row = idx / (RB / 16), seg = idx - row * (RB / 16);
        *(uint4*)(&sa[buf][row * RS + seg * 16]) = ra[i];
      }
    }
#pragma unroll
    for (int i = 0; i < BP; i++) {
      const int idx = i * kThreads + tid;
      if (idx < B16) {
        if (kQ4) {
          const int row = idx / KB, kb = idx - row * KB;
          uint4 lo, hi;
          unpack_q4(rb[i].x, lo.x, hi.x);
          unpack_q4(rb[i].y, lo.y, hi.y);
          unpack_q4(rb[i].z, lo.z, hi.z);
          unpack_q4(rb[i].w, lo.w, hi.w);
          int8_t* dst = &sb[buf][row * RS + kb * 32];
          *(uint4*)dst = lo;
          *(uint4*)(dst + 16) = hi;
        } else {
          const int row = idx / (RB / 16), seg = idx - row * (RB / 16);
          *(uint4*)(&sb[buf][row * RS + seg * 16]) = rb[i];
        }
      }
    }
#pragma unroll
    for (int i = 0; i < SXP; i++) {
      const int idx = i * kThreads + tid;
      if (idx < KB * BM) {
        uint32_t p0, p1, p2;
        split3_bf16(rsx[i], p0, p1, p2);
        uint2* d = sxs[buf][idx / BM][idx % BM];
        d[0] = a_scale_half0(p0, p1, p2);
        d[1] = a_scale_half1(p0, p1, p2);
      }
    }
#pragma unroll
    for (int i = 0; i < SWP; i++) {
      const int idx = i * kThreads + tid;
      if (idx < KB * BN) {
        uint32_t p0, p1, p2;
        split3_bf16(kQ4 ? half_bits_to_float((uint16_t)rsh[i]) : rsw[i], p0, p1, p2);
        uint2* d = sws[buf][idx / BN][idx % BN];
        d[0] = b_scale_half0(p0, p1, p2);
        d[1] = b_scale_half1(p0, p1, p2);
      }
    }
  };

  float acc[SM][SN][16];
#pragma unroll
  for (int i = 0; i < SM; i++)
#pragma unroll
    for (int j = 0; j < SN; j++)
#pragma unroll
      for (int v = 0; v < 16; v++) acc[i][j][v] = 0.0f;

  // This workgroup's K stages: all of them, or split blockIdx.z's share.
  const int s_begin = blockIdx.z * p.split_stages;
  const int s_end = min(stages, s_begin + p.split_stages);
  load_stage(s_begin);
  store_stage(0);
  __syncthreads();

  const int lrow = lane & 31, lk = (lane >> 5) * 16;
  for (int s = s_begin; s < s_end; s++) {
    const int buf = (s - s_begin) & 1;
    if (s + 1 < s_end) load_stage(s + 1);
    const int nkb = min(KB, B - s * KB);
#pragma unroll
    for (int kb = 0; kb < KB; kb++) {
      if (kb >= nkb) break;
      v4i a[SM], b[SN];
#pragma unroll
      for (int i = 0; i < SM; i++)
        a[i] = *(const v4i*)(&sa[buf][(wm * TM + i * 32 + lrow) * RS + kb * 32 + lk]);
#pragma unroll
      for (int j = 0; j < SN; j++)
        b[j] = *(const v4i*)(&sb[buf][(wn * TN + j * 32 + lrow) * RS + kb * 32 + lk]);
      // This lane's outputs: column n = lane % 32 of each N subtile; rows
      // (v / 4) * 8 + (lane / 32) * 4 + v % 4 of each M subtile. The tile's
      // scale products s = sx * sw come from the outer-product MFMA on the
      // staged bf16 pieces; the epilogue is cvt + fma per output.
      s4 bsv[SN];
#pragma unroll
      for (int j = 0; j < SN; j++)
        bsv[j] = __builtin_bit_cast(s4, sws[buf][kb][wn * TN + j * 32 + lrow][lane >> 5]);
#pragma unroll
      for (int i = 0; i < SM; i++) {
        const s4 asv = __builtin_bit_cast(s4, sxs[buf][kb][wm * TM + i * 32 + lrow][lane >> 5]);
#pragma unroll
        for (int j = 0; j < SN; j++) {
          v16i d = {};
          d = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], d, 0, 0, 0);
          const v16f z = {};
          const v16f sc = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(asv, bsv[j], z, 0, 0, 0);
#pragma unroll
          for (int v = 0; v < 16; v++) acc[i][j][v] = fmaf((float)d[v], sc[v], acc[i][j][v]);
        }
      }
    }
    if (s + 1 < s_end) store_stage(buf ^ 1);
    __syncthreads();
  }

  // Store: lane holds column n0 + wn*TN + j*32 + lane%32 for 16 rows.
  float* out = p.part ? p.part + (size_t)blockIdx.z * M * N : p.y;
#pragma unroll
  for (int i = 0; i < SM; i++)
#pragma unroll
    for (int j = 0; j < SN; j++) {
      const int r = n0 + wn * TN + j * 32 + lrow;
      if (r >= N) continue;
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int m = m0 + wm * TM + i * 32 + (v / 4) * 8 + (lane >> 5) * 4 + (v % 4);
        if (m < M) store_wt(out + (size_t)m * N + r, acc[i][j][v]);
      }
    }
}

// ------------------------------------------------------------ skinny (n <= 16)

// Few tokens (n <= 16) and K <= 2048: the weights are read once from HBM and
// the work is too small to hide a memory round trip per stage, so every
// load of the kernel is issued at its start and waited for once. A
// workgroup owns 16 weight rows over the whole K:
// * its 16 rows (Q4 nibbles or Q8 bytes), their scales and the x scales of
//   all tokens arrive with coalesced 16-byte (scales: 4-byte) loads and go
//   to LDS (rows padded by 16 bytes against bank conflicts; x scales
//   transposed [block][token]);
// * its 4 waves split K into 4 runs of at most 16 blocks (wave w: blocks
//   wQ .. wQ + Q - 1, Q = ceil(B / 4)), and each wave loads the int8 tokens
//   of its blocks straight into registers, also at the start.
// A lane holds column c = lane % 16 (weight row r0 + c) and k-group
// g = lane / 16 of a block: v_mfma_i32_16x16x32_i8 takes A = 16 tokens x 32
// (8 int8 of token 16t + c at k = 8g.. per lane), B = 32 x 16 weight rows
// (8 int8 of row r0 + c at k = 8g.., from LDS) and gives the block's exact
// int32 dots, the lane holding tokens 16t + 4g + v (v < 4) of column c.
// Epilogue per output and block: acc = fma(d, sw * sx, acc) (s rounded
// first, as lab_native.c:509). The 4 waves' sums are added through LDS in
// wave order (deterministic), with no split-K pass. Rows past the matrix
// and tokens past n load zeros (bounded buffer loads) and are not stored;
// blocks past a wave's last load zeros and add exact zeros.
constexpr int kSkinnyRows = 16;
constexpr int kSkinnyBlocks = 16;       // blocks per wave: K <= 2048
constexpr int kSkinnyFar = 0x7fffff00;  // a buffer offset past every operand

typedef int v2i_t __attribute__((ext_vector_type(2)));
typedef int v4i_t __attribute__((ext_vector_type(4)));

// LDS of the skinny kernel: padded weight rows, weight scales (fp32), x
// scales [block][token], and waves 1..3's sums.
size_t skinny_row_bytes(bool q4, int cols) { return (size_t)(q4 ? cols / 2 : cols) + 16; }
size_t skinny_lds(bool q4, int cols, int mt) {
  const int blocks = cols / kBlock;
  return kSkinnyRows * skinny_row_bytes(q4, cols) + (size_t)kSkinnyRows * blocks * 4 +
         (size_t)blocks * 16 * mt * 4 + (size_t)3 * mt * 4 * 64 * 4;
}

template <bool kQ4, int MT>
__global__ void __launch_bounds__(kThreads) skinny_kernel(GemmParams p) {
  extern __shared__ __align__(16) uint8_t slds[];
  constexpr int MP = 16 * MT;
  constexpr int NB = kSkinnyBlocks;
  const int K = p.cols, B = K / kBlock, M = p.n, N = p.rows;
  const int RB = kQ4 ? K / 2 : K;            // bytes of a weight row
  const int RS = RB + 16;                    // its LDS stride
  uint8_t* sw_rows = slds;                   // [16][RS]
  float* sws = (float*)(slds + kSkinnyRows * RS);   // [16][B] weight scales
  float* sxT = sws + kSkinnyRows * B;               // [B][MP] x scales
  float* red = sxT + B * MP;                        // [3][MT][4][64]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, c = lane & 15;
  const int r0 = blockIdx.x * kSkinnyRows;

  const i32x4 rq = buffer_rsrc(p.qs, (uint32_t)((size_t)N * RB));
  const i32x4 rs = buffer_rsrc(p.scales, (uint32_t)((size_t)N * B * (kQ4 ? 2 : 4)));
  const i32x4 rx = buffer_rsrc(p.xq, (uint32_t)((size_t)M * K));
  const i32x4 rxs = buffer_rsrc(p.xsc, (uint32_t)((size_t)M * B * 4));

  // 1. Every load, issued together. Weight rows: 16-byte pieces, RB / 16
  // per row, at most 8 per thread (16 rows x 2048 bytes).
  constexpr int WP = 8;
  uint4 wraw[WP];
#pragma unroll
  for (int e = 0; e < WP; e++) {
    const int i = e * kThreads + tid, per = RB / 16;
    const int row = i / per, piece = i - row * per;
    const bool in = i < kSkinnyRows * per && r0 + row < N;
    wraw[e] = buffer_load16(rq, in ? (r0 + row) * RB + piece * 16 : kSkinnyFar);
  }
  // Weight scales: 16 x B (<= 1024) raw values, 4 per thread.
  int sraw[4];
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const int i = e * kThreads + tid, row = i / B, b = i - (i / B) * B;
    const bool in = i < kSkinnyRows * B && r0 + row < N;
    const int off = ((r0 + row) * B + b) * (kQ4 ? 2 : 4);
    sraw[e] = kQ4 ? (int)dnx_raw_buffer_load_i16(rs, in ? off : kSkinnyFar, 0, 0)
                  : dnx_raw_buffer_load_i32(rs, in ? off : kSkinnyFar, 0, 0);
  }
  // x scales: MP x B (<= 4096) floats, token-major, 16 per thread.
  float xraw[16];
#pragma unroll
  for (int e = 0; e < 16; e++) {
    const int i = e * kThreads + tid;
    xraw[e] = __int_as_float(dnx_raw_buffer_load_i32(rxs, i < M * B ? i * 4 : kSkinnyFar, 0, 0));
  }
  // This wave's int8 tokens: block j (= wave * Q + j), token tile t. A
  // lane's consecutive blocks are adjacent 32-byte pieces of its token's
  // row, so the wave's loads reuse each cache line 4 times in a row.
  const int Q = (B + 3) / 4;   // blocks per wave (<= 16)
  v2i_t ra[NB][MT];
#pragma unroll
  for (int j = 0; j < NB; j++) {
    const int b = j < Q ? wave * Q + j : B;
#pragma unroll
    for (int t = 0; t < MT; t++) {
      const int m = 16 * t + c;
      ra[j][t] = dnx_raw_buffer_load_v2i32(
          rx, b < B && m < M ? m * K + b * 32 + 8 * g : kSkinnyFar, 0, 0);
    }
  }

  // 2. Weights, weight scales and x scales to LDS.
#pragma unroll
  for (int e = 0; e < WP; e++) {
    const int i = e * kThreads + tid, per = RB / 16;
    const int row = i / per, piece = i - row * per;
    if (i < kSkinnyRows * per) *(uint4*)(sw_rows + row * RS + piece * 16) = wraw[e];
  }
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const int i = e * kThreads + tid;
    if (i < kSkinnyRows * B) {
      sws[i] = kQ4 ? half_bits_to_float((uint16_t)sraw[e]) : __int_as_float(sraw[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < 16; e++) {
    const int i = e * kThreads + tid;
    if (i < MP * B) {
      const int m = i / B, b = i - (i / B) * B;
      sxT[b * MP + m] = xraw[e];
    }
  }
  __syncthreads();

  // 3. The wave's blocks.
  float acc[MT][4];
#pragma unroll
  for (int t = 0; t < MT; t++)
#pragma unroll
    for (int v = 0; v < 4; v++) acc[t][v] = 0.0f;
#pragma unroll
  for (int j = 0; j < NB; j++) {
    const int b = min(j < Q ? wave * Q + j : B, B - 1);   // past the end: zeros from ra
    uint2 w = *(const uint2*)(sw_rows + c * RS + b * (kQ4 ? 16 : 32) + (kQ4 ? (g & 1) * 8 : 8 * g));
    if (kQ4) {  // bytes 8(g & 1).. : low nibbles (k < 16) or high (k >= 16)
      uint32_t lo0, hi0, lo1, hi1;
      unpack_q4(w.x, lo0, hi0);
      unpack_q4(w.y, lo1, hi1);
      w.x = (g >> 1) ? hi0 : lo0;
      w.y = (g >> 1) ? hi1 : lo1;
    }
    const long bop = (long)(((uint64_t)w.y << 32) | w.x);
    const float swf = sws[c * B + b];
#pragma unroll
    for (int t = 0; t < MT; t++) {
      const long aop = (long)(((uint64_t)(uint32_t)ra[j][t].y << 32) | (uint32_t)ra[j][t].x);
      const v4i_t z = {};
      const v4i_t d = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, bop, z, 0, 0, 0);
      const float4 sx = *(const float4*)(sxT + b * MP + 16 * t + 4 * g);
      acc[t][0] = fmaf((float)d[0], swf * sx.x, acc[t][0]);
      acc[t][1] = fmaf((float)d[1], swf * sx.y, acc[t][1]);
      acc[t][2] = fmaf((float)d[2], swf * sx.z, acc[t][2]);
      acc[t][3] = fmaf((float)d[3], swf * sx.w, acc[t][3]);
    }
  }

  // 4. Waves 1..3 hand their sums to wave 0, which adds them in wave order.
  if (wave > 0) {
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
      for (int v = 0; v < 4; v++) red[(((wave - 1) * MT + t) * 4 + v) * 64 + lane] = acc[t][v];
  }
  __syncthreads();
  const int row = r0 + c;
  if (wave > 0 || row >= N) return;
#pragma unroll
  for (int t = 0; t < MT; t++)
#pragma unroll
    for (int v = 0; v < 4; v++) {
      float s = acc[t][v];
#pragma unroll
      for (int w = 0; w < 3; w++) s += red[((w * MT + t) * 4 + v) * 64 + lane];
      const int m = 16 * t + 4 * g + v;
      if (m < M) store_wt(p.y + (size_t)m * N + row, s);
    }
}

// Whether the skinny kernel takes this shape: n <= 16, K <= 2048 (16
// blocks per wave, 8 row pieces per thread) and the LDS within 64 KB. With
// more tokens it lost to the split-K tile kernel on 6144 x 2048 Q4 (n = 32:
// 13.7 against 11.8 us; n = 16: 9.7 against 10.2; n = 8: 8.5 against 9.4).
bool skinny_fits(bool q4, int64_t cols, int64_t n) {
  if (n > 16 || cols > 2048 || cols % 16 != 0) return false;
  return skinny_lds(q4, (int)cols, 1) <= 64 * 1024;
}

template <bool kQ4, int MT>
int launch_skinny(const GemmParams& p, hipStream_t stream) {
  const size_t lds = skinny_lds(kQ4, p.cols, MT);
  const unsigned grid = (unsigned)((p.rows + kSkinnyRows - 1) / kSkinnyRows);
  hipLaunchKernelGGL((skinny_kernel<kQ4, MT>), dim3(grid), dim3(kThreads), lds, stream, p);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

// y = the split partials summed in split order (deterministic).
__global__ void __launch_bounds__(kThreads) splitk_reduce_kernel(const float* __restrict__ part,
                                                                 float* __restrict__ y,
                                                                 int64_t count, int splits) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < count;
       i += (int64_t)gridDim.x * kThreads) {
    store_wt(y + i, split_sum(part, count, i, splits));
  }
}

// Library-owned split-K workspace (device 0 of this process), grown on
// demand: the first call at a larger small-M shape allocates, so such a
// call must not be the first one inside a graph capture.
float* gSplitWs = nullptr;
size_t gSplitBytes = 0;

float* split_workspace(size_t bytes) {
  if (bytes <= gSplitBytes) return gSplitWs;
  if (gSplitWs != nullptr) {
    if (hipDeviceSynchronize() != hipSuccess) return nullptr;
    (void)hipFree(gSplitWs);
    gSplitWs = nullptr;
    gSplitBytes = 0;
  }
  if (hipMalloc(&gSplitWs, bytes) != hipSuccess) {
    gSplitWs = nullptr;
    return nullptr;
  }
  gSplitBytes = bytes;
  return gSplitWs;
}

template <bool kQ4, int BM, int BN, int WM, int KB>
int launch_tile(GemmParams p, hipStream_t stream) {
  const unsigned gx = (unsigned)((p.rows + BN - 1) / BN), gy = (unsigned)((p.n + BM - 1) / BM);
  const int stages = (p.cols / kBlock + KB - 1) / KB;
  // Split K when the tiles alone would leave CUs idle (small n): enough
  // splits for about 512 workgroups, each with at least one stage. Between
  // one and three workgroups per CU (the resident count of the 64 x 64
  // tiles) a long K (32+ stages) is split too, into runs of at least 8
  // stages, so that the slots fill: the vision fc2 (1152 x 4320 at 1024
  // tokens, 288 tiles) ran one or two workgroups per CU over all 34 stages
  // (47.9 -> 42.6 us with 3 splits). A shorter K loses more to the partials'
  // round trip than it gains (6144 x 2048 at 256 tokens: 24 -> 27 us).
  int splits = 1;
  const int64_t tiles = (int64_t)gx * gy;
  if (tiles < 256 && stages > 1) {
    splits = (int)((512 + tiles - 1) / tiles);
    if (splits > stages) splits = stages;
  } else if (tiles < 768 && stages >= 32) {
    splits = (int)((768 + tiles - 1) / tiles);
    if (splits > stages / 8) splits = stages / 8;
  }
  p.split_stages = (stages + splits - 1) / splits;
  splits = (stages + p.split_stages - 1) / p.split_stages;
  p.part = nullptr;
  const int64_t count = (int64_t)p.n * p.rows;
  if (splits > 1) {
    p.part = split_workspace((size_t)splits * count * 4);
    if (p.part == nullptr) return DNX_ENOMEM;
  }
  hipLaunchKernelGGL((gemm_kernel<kQ4, BM, BN, WM, KB>), dim3(gx, gy, (unsigned)splits),
                     dim3(kThreads), 0, stream, p);
  if (hipGetLastError() != hipSuccess) return DNX_ELAUNCH;
  if (splits > 1) {
    const int64_t blocks = (count + kThreads - 1) / kThreads;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)),
                       dim3(kThreads), 0, stream, p.part, p.y, count, splits);
    if (hipGetLastError() != hipSuccess) return DNX_ELAUNCH;
  }
  return DNX_OK;
}

template <bool kQ4>
int launch_gemm(const void* qs, const void* scales, const int8_t* xq, const float* xsc,
                float* y, int64_t rows, int64_t cols, int64_t n, hipStream_t stream) {
  if (rows <= 0 || cols <= 0 || n <= 0 || cols % kBlock != 0) return DNX_EINVAL;
  // Buffer-load offsets are 32-bit: each operand must stay below 2 GB.
  if (rows * (kQ4 ? cols / 2 : cols) >= (1ll << 31) || n * cols >= (1ll << 31)) return DNX_EINVAL;
  if (((uintptr_t)qs & 15) || ((uintptr_t)xq & 15) || (cols % 16)) return DNX_EINVAL;
  GemmParams p{qs, scales, xq, xsc, y, (int)rows, (int)cols, (int)n, 0, nullptr};
  // Up to 16 tokens and K <= 2048: the skinny kernel (every load at the
  // start, K shared by a workgroup's waves, no split-K pass);
  // 32 tokens: one wave row of 32 x 32 tiles (4 waves across N); else
  // 64 x 64 tiles (2 x 2 waves), which keep ~3 workgroups per CU resident
  // at prefill sizes.
  if (skinny_fits(kQ4, cols, n)) return launch_skinny<kQ4, 1>(p, stream);
  if (n <= 32) return launch_tile<kQ4, 32, 128, 1, 4>(p, stream);
  return launch_tile<kQ4, 64, 64, 2, 4>(p, stream);
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
