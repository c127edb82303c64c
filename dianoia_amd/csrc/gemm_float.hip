// Float-input GEMM (the products of lab_gemm_q8 / lab_gemm_q4 mode 0,
// lab_native.c:489-501 and :1013-1023, for many tokens) on gfx950 bf16 MFMA:
//   y[m][r] = sum_b sw[r][b] * D_b[m][r],   D_b[m][r] = sum_{k in b} x[m][k] * w[r][k]
// with w the Q8 value or q - 8 for Q4, x fp32 as the caller gives it.
//
// Exact operands. Every weight value is an integer of at most 8 significant
// bits (|w| <= 127), exact in bf16. x is split into three bf16 pieces that
// sum to it exactly (split3_bf16: 8 + 8 + 8 significant bits), so every
// product piece * w is exact in fp32 and D_b is the fp32 sum of exact
// products, in the matrix core's order instead of the CPU's fma chain: the
// outputs agree with the CPU kernel to fp32 rounding (the tolerance bar, as
// the reference's own float GPU kernels, lab_metal.m:79-144, :174-258, sum
// in yet another order).
//
// The weight scale sw is the same for all 16 outputs a lane holds (they are
// one weight row r = the lane's column), so the per-block epilogue is one
// fma per output: acc = fma(D_b, sw, acc), blocks in order, as the CPU's
// acc = fmadd(s, sw, acc).
//
// Per 32 x 32 tile and block: six v_mfma_f32_32x32x16_bf16 (three pieces x
// two halves of the block's K) and 16 fma. A wave loads its 32 tokens'
// fp32 x for a block (32 bytes per lane per half, straight from memory,
// a block ahead) and splits it in registers; the weights are converted to
// bf16 B fragments once per workgroup in LDS, with their fp32 scales.
//
// Workgroup: 256 threads, 4 waves along M (32 tokens each), SN x 32 weight
// rows; 4-block stages double-buffered in LDS. When the tiles alone would
// leave CUs idle, K is split over blockIdx.y and a second kernel adds the
// partials in split order (deterministic).

#include "common.h"
#include "dnx_kernels.h"

using namespace dnx;

namespace {

typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kTok = 32;        // tokens per wave (one MFMA tile of rows)
constexpr int kBM = kWaves * kTok;
constexpr int kKB = 4;          // blocks per stage

struct FParams {
  const void* qs;       // Q8 int8 [rows][cols] or Q4 nibbles [rows][cols/2]
  const void* scales;   // Q8 fp32 / Q4 fp16 bits [rows][cols/32]
  const float* x;       // [n][cols]
  float* y;             // [n][rows]
  float* part;          // split partials [splits][n][rows], or null
  int rows, cols, n;
  int tiles_m, tiles;
  int split_blocks;     // blocks per K split, a multiple of kKB
};

// Two small integers as a pair of bf16 (exact: at most 8 significant bits).
DNX_DEV uint32_t bf16x2(int a, int b) {
  const uint32_t fa = __float_as_uint((float)a), fb = __float_as_uint((float)b);
  return (fa >> 16) | (fb & 0xffff0000u);
}

// 8 weights of a block (k = 8c .. 8c + 7 of one K half) as one 16-byte bf16
// fragment, from the block's integer values in w[0..31].
DNX_DEV uint4 weight_frag(const int* w) {
  return make_uint4(bf16x2(w[0], w[1]), bf16x2(w[2], w[3]), bf16x2(w[4], w[5]),
                    bf16x2(w[6], w[7]));
}

// Eight floats -> the three bf16 pieces of each (p0 + p1 + p2 == x), each
// piece as one 16-byte fragment (element j of the fragment = value j). An
// infinity or NaN is carried whole by p0 (a quiet NaN for every NaN) with
// zero pieces after it, so it meets the weights as the CPU's x does.
DNX_DEV void split_frags(const float* x, uint4* p) {
  uint32_t q[3][8];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    split3_bf16(x[j], q[0][j], q[1][j], q[2][j]);
    const uint32_t bits = __float_as_uint(x[j]);
    if ((bits & 0x7f800000u) == 0x7f800000u) {
      q[0][j] = (bits & 0x007fffffu) ? 0x7fc0u : bits >> 16;
      q[1][j] = q[2][j] = 0u;
    }
  }
#pragma unroll
  for (int i = 0; i < 3; i++) {
    p[i] = make_uint4(q[i][0] | (q[i][1] << 16), q[i][2] | (q[i][3] << 16),
                      q[i][4] | (q[i][5] << 16), q[i][6] | (q[i][7] << 16));
  }
}

template <bool kQ4, int SN>
__global__ void __launch_bounds__(kThreads) gemm_float_kernel(FParams p) {
  constexpr int BN = SN * 32;
  // LDS stage: bf16 B fragments [kb][h][khalf][row][16 B], then the fp32
  // scales [kb][row].
  constexpr int kFrag = kKB * 4 * BN * 16;
  constexpr int kStage = kFrag + kKB * BN * 4;
  constexpr int kPairs = BN * kKB;                      // (row, block) per stage
  constexpr int PP = (kPairs + kThreads - 1) / kThreads;
  __shared__ __align__(16) uint8_t lds[2 * kStage];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int K = p.cols, B = K / kBlock, M = p.n, N = p.rows;
  // XCD-aware order (workgroups are dealt round-robin to the 8 XCDs): each
  // XCD walks a contiguous run of tiles, all token tiles of its weight rows.
  const int i = blockIdx.x;
  const int t = (p.tiles % 8 == 0) ? (i % 8) * (p.tiles / 8) + i / 8 : i;
  const int tm = t % p.tiles_m, tn = t / p.tiles_m;
  const int n0 = tn * BN;
  const int m0 = tm * kBM + wave * kTok;
  const int b_begin = blockIdx.y * p.split_blocks;
  const int b_end = min(B, b_begin + p.split_blocks);
  const int stages = (b_end - b_begin + kKB - 1) / kKB;

  const int wbytes = kQ4 ? 16 : 32;
  const i32x4 rq = buffer_rsrc(p.qs, (uint32_t)((size_t)N * B * wbytes));
  const i32x4 rs = buffer_rsrc(p.scales, (uint32_t)((size_t)N * B * (kQ4 ? 2 : 4)));
  const i32x4 rx = buffer_rsrc(p.x, (uint32_t)((size_t)M * K * 4));

  // ---- weight staging: thread q takes (row q / kKB, block q % kKB)
  i32x4 wq[PP][2];
  int ws[PP];
  auto load_w = [&](int s) {
    const int b0 = b_begin + s * kKB;
#pragma unroll
    for (int e = 0; e < PP; e++) {
      const int q = e * kThreads + tid;
      const int row = q / kKB, b = b0 + q % kKB;
      const bool ok = q < kPairs && n0 + row < N && b < b_end;
      const int off = ok ? ((n0 + row) * B + b) * wbytes : -(1 << 20);
      wq[e][0] = dnx_raw_buffer_load_v4i32(rq, off, 0, 0);
      if (!kQ4) wq[e][1] = dnx_raw_buffer_load_v4i32(rq, off + 16, 0, 0);
      ws[e] = kQ4 ? (int)(uint16_t)dnx_raw_buffer_load_i16(rs, ok ? ((n0 + row) * B + b) * 2 : -4, 0, 0)
                  : dnx_raw_buffer_load_i32(rs, ok ? ((n0 + row) * B + b) * 4 : -4, 0, 0);
    }
  };
  auto store_w = [&](int buf) {
    uint8_t* base = lds + buf * kStage;
#pragma unroll
    for (int e = 0; e < PP; e++) {
      const int q = e * kThreads + tid;
      if (q >= kPairs) continue;
      const int row = q / kKB, kb = q % kKB;
      int w[32];
      if (kQ4) {
        const uint32_t v[4] = {(uint32_t)wq[e][0].x, (uint32_t)wq[e][0].y, (uint32_t)wq[e][0].z,
                               (uint32_t)wq[e][0].w};
#pragma unroll
        for (int k = 0; k < 16; k++) {
          const uint32_t byte = (v[k >> 2] >> (8 * (k & 3))) & 0xffu;
          w[k] = (int)(byte & 15u) - 8;
          w[k + 16] = (int)(byte >> 4) - 8;
        }
      } else {
        const uint32_t v[8] = {(uint32_t)wq[e][0].x, (uint32_t)wq[e][0].y, (uint32_t)wq[e][0].z,
                               (uint32_t)wq[e][0].w, (uint32_t)wq[e][1].x, (uint32_t)wq[e][1].y,
                               (uint32_t)wq[e][1].z, (uint32_t)wq[e][1].w};
#pragma unroll
        for (int k = 0; k < 32; k++) w[k] = (int)(int8_t)(v[k >> 2] >> (8 * (k & 3)));
      }
      // Fragment (h, c) holds k = 16 h + 8 c .. + 7.
#pragma unroll
      for (int f = 0; f < 4; f++) {
        *(uint4*)(base + ((kb * 4 + f) * BN + row) * 16) = weight_frag(w + 8 * f);
      }
      const float sw = kQ4 ? half_bits_to_float((uint16_t)ws[e]) : __int_as_float(ws[e]);
      *(float*)(base + kFrag + (kb * BN + row) * 4) = sw;
    }
  };

  // ---- this wave's x: lane l holds token m0 + l % 32, k = 8 (l / 32) + 0..7
  // of each K half (16 h); tokens past n read zeros.
  const int xm = m0 + (lane & 31);
  auto load_x = [&](int b, i32x4* xr) {
    const bool ok = xm < M && b < b_end;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int off = ok ? (xm * K + b * kBlock + 16 * h + 8 * (lane >> 5)) * 4 : -(1 << 20);
      xr[2 * h] = dnx_raw_buffer_load_v4i32(rx, off, 0, 0);
      xr[2 * h + 1] = dnx_raw_buffer_load_v4i32(rx, off + 16, 0, 0);
    }
  };

  v16f acc[SN];
#pragma unroll
  for (int j = 0; j < SN; j++)
#pragma unroll
    for (int v = 0; v < 16; v++) acc[j][v] = 0.0f;

  i32x4 xcur[4], xnext[4];
  load_x(b_begin, xcur);
  load_w(0);
  store_w(0);
  __syncthreads();
  for (int s = 0; s < stages; s++) {
    const int buf = s & 1;
    if (s + 1 < stages) load_w(s + 1);
    const uint8_t* base = lds + buf * kStage;
    const int b0 = b_begin + s * kKB;
#pragma unroll 1
    for (int kb = 0; kb < kKB; kb++) {
      load_x(b0 + kb + 1, xnext);
      // The three bf16 pieces of this lane's 16 x values, per K half.
      uint4 a[2][3];
#pragma unroll
      for (int h = 0; h < 2; h++) {
        float xv[8];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          xv[j] = __int_as_float(xcur[2 * h][j]);
          xv[4 + j] = __int_as_float(xcur[2 * h + 1][j]);
        }
        split_frags(xv, a[h]);
      }
      // The SN tiles' MFMAs interleaved (independent accumulators), then
      // one fma per output with the row's scale.
      v16f d[SN];
#pragma unroll
      for (int j = 0; j < SN; j++)
#pragma unroll
        for (int v = 0; v < 16; v++) d[j][v] = 0.0f;
#pragma unroll
      for (int h = 0; h < 2; h++) {
        bf8 bw[SN];
#pragma unroll
        for (int j = 0; j < SN; j++) {
          const int row = j * 32 + (lane & 31);
          bw[j] = __builtin_bit_cast(
              bf8, *(const uint4*)(base + ((kb * 4 + 2 * h + (lane >> 5)) * BN + row) * 16));
        }
#pragma unroll
        for (int pc = 0; pc < 3; pc++)
#pragma unroll
          for (int j = 0; j < SN; j++) {
            d[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf8, a[h][pc]),
                                                           bw[j], d[j], 0, 0, 0);
          }
      }
#pragma unroll
      for (int j = 0; j < SN; j++) {
        const float sw = *(const float*)(base + kFrag + (kb * BN + j * 32 + (lane & 31)) * 4);
#pragma unroll
        for (int v = 0; v < 16; v++) acc[j][v] = fmaf(d[j][v], sw, acc[j][v]);
      }
#pragma unroll
      for (int r = 0; r < 4; r++) xcur[r] = xnext[r];
    }
    if (s + 1 < stages) store_w(buf ^ 1);
    __syncthreads();
  }

  float* out = p.part ? p.part + (size_t)blockIdx.y * M * N : p.y;
#pragma unroll
  for (int j = 0; j < SN; j++) {
    const int r = n0 + j * 32 + (lane & 31);
    if (r >= N) continue;
#pragma unroll
    for (int v = 0; v < 16; v++) {
      const int m = m0 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
      if (m < M) store_wt(out + (size_t)m * N + r, acc[j][v]);
    }
  }
}

// y = the split partials summed in split order (deterministic).
__global__ void __launch_bounds__(kThreads) float_splitk_reduce_kernel(
    const float* __restrict__ part, float* __restrict__ y, int64_t count, int splits) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < count;
       i += (int64_t)gridDim.x * kThreads) {
    store_wt(y + i, split_sum(part, count, i, splits));
  }
}

// Library-owned split partials, grown on demand (a call at a larger shape
// than any before allocates: not the first call inside a graph capture).
float* gPart = nullptr;
size_t gPartBytes = 0;

float* part_workspace(size_t bytes) {
  if (bytes <= gPartBytes) return gPart;
  if (gPart != nullptr) {
    if (hipDeviceSynchronize() != hipSuccess) return nullptr;
    (void)hipFree(gPart);
    gPart = nullptr;
    gPartBytes = 0;
  }
  if (hipMalloc(&gPart, bytes) != hipSuccess) {
    gPart = nullptr;
    return nullptr;
  }
  gPartBytes = bytes;
  return gPart;
}

template <bool kQ4, int SN>
int launch(const void* qs, const void* scales, const float* x, float* y, int64_t rows,
           int64_t cols, int64_t n, hipStream_t stream) {
  constexpr int BN = SN * 32;
  FParams p{};
  p.qs = qs;
  p.scales = scales;
  p.x = x;
  p.y = y;
  p.rows = (int)rows;
  p.cols = (int)cols;
  p.n = (int)n;
  p.tiles_m = (int)((n + kBM - 1) / kBM);
  p.tiles = p.tiles_m * (int)((rows + BN - 1) / BN);
  const int B = (int)(cols / kBlock);
  const int max_splits = (B + kKB - 1) / kKB;
  int splits = 1;
  if (p.tiles < 256) splits = min((512 + p.tiles - 1) / p.tiles, max_splits);
  p.split_blocks = (B + splits - 1) / splits;
  p.split_blocks = (p.split_blocks + kKB - 1) / kKB * kKB;
  splits = (B + p.split_blocks - 1) / p.split_blocks;
  const int64_t count = n * rows;
  p.part = nullptr;
  if (splits > 1) {
    p.part = part_workspace((size_t)splits * count * 4);
    if (p.part == nullptr) return DNX_ENOMEM;
  }
  hipLaunchKernelGGL((gemm_float_kernel<kQ4, SN>), dim3((unsigned)p.tiles, (unsigned)splits),
                     dim3(kThreads), 0, stream, p);
  if (hipGetLastError() != hipSuccess) return DNX_ELAUNCH;
  if (splits > 1) {
    const int64_t blocks = (count + kThreads - 1) / kThreads;
    hipLaunchKernelGGL(float_splitk_reduce_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)),
                       dim3(kThreads), 0, stream, p.part, y, count, splits);
    if (hipGetLastError() != hipSuccess) return DNX_ELAUNCH;
  }
  return DNX_OK;
}

template <bool kQ4>
int launch_float(const void* qs, const void* scales, const float* x, float* y, int64_t rows,
                 int64_t cols, int64_t n, hipStream_t stream) {
  if (rows <= 0 || cols <= 0 || n <= 0 || cols % kBlock != 0) return DNX_EINVAL;
  // 32-bit buffer offsets: each operand below 2 GB.
  if (rows * (kQ4 ? cols / 2 : cols) >= (1ll << 31) || n * cols * 4 >= (1ll << 31) ||
      n * rows >= (1ll << 31)) {
    return DNX_EINVAL;
  }
  if (((uintptr_t)qs & 15) || ((uintptr_t)x & 3) || ((uintptr_t)y & 3) ||
      ((uintptr_t)scales & (kQ4 ? 1 : 3))) {
    return DNX_EINVAL;
  }
  // 128 weight rows per workgroup while that keeps the CUs busy, else 64.
  const int64_t tiles128 = ((n + kBM - 1) / kBM) * ((rows + 127) / 128);
  if (tiles128 >= 256) return launch<kQ4, 4>(qs, scales, x, y, rows, cols, n, stream);
  return launch<kQ4, 2>(qs, scales, x, y, rows, cols, n, stream);
}

}  // namespace

extern "C" {

int dnx_gemm_q8_float(const int8_t* qs, const float* scales, const float* x, float* y,
                      int64_t rows, int64_t cols, int64_t n, dnx_stream_t stream) {
  return launch_float<false>(qs, scales, x, y, rows, cols, n, (hipStream_t)stream);
}

int dnx_gemm_q4_float(const uint8_t* qs, const uint16_t* scales, const float* x, float* y,
                      int64_t rows, int64_t cols, int64_t n, dnx_stream_t stream) {
  return launch_float<true>(qs, scales, x, y, rows, cols, n, (hipStream_t)stream);
}

}  // extern "C"
