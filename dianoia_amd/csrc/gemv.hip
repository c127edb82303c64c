// Exact-order decode GEMV on gfx950 for the engine's Q8 and Q4 weights.
//
// y[t][r] = (W x[t])[r] for n <= 4 tokens, computed in the float order of
// the reference CPU kernels (dot_q8_sdot lab_native.c:503-512, dot_q4_sdot
// :1025-1034, lane_sum :209-212): per 32-block, four exact int32 lane sums
// d_l over bytes {4l..4l+3, 16+4l..19+4l}; s = sw * sx rounded;
// acc_l = fma(float(d_l), s, acc_l), block after block; y = (acc0 + acc1) +
// (acc2 + acc3). The logits are therefore bit-identical to lab_gemm_q8 /
// lab_gemm_q4 mode 1, and so is their greedy argmax.
//
// Work decomposition (HBM streaming on 256 CUs):
// * A workgroup is 4 independent waves. Each wave owns tiles of R weight
//   rows, taken round-robin over a persistent grid sized to what stays
//   resident, so each workgroup quantizes x once and then streams.
// * A tile is read in 1 KB chunks per row (32 Q8 blocks or 64 Q4 blocks):
//   one wave instruction loads 1 KB of one row with 16-byte lanes, marked
//   non-temporal. Loads go through a ring of row-chunks per wave: tiles of
//   8+ rows keep one tile-chunk (8 KB) in flight and refill each slot as
//   soon as it is turned into lane sums; smaller tiles keep 16 slots and
//   refill a group at a time. The first chunks are requested while the
//   prologue quantizes x, so the two latencies overlap.
// * Outputs are held in one register across the wave's lanes and stored
//   after the loop: loads and stores share one wait counter, and a store in
//   the loop would make every later wait drain the ring.
// * Lane sums (as floats; exact below 2^24) and per-block scales go to the
//   wave's own LDS; lanes (t, row, l) then run the chunk's FMA chains and a
//   DPP lane combine gives each row.
// * Fusions: the gate/up pair of an MLP shares x and finishes with the
//   SiLU(gate) * up glue (shard.dart:457-461); an LM head can finish with
//   the greedy argmax (sampler.dart:137-143): each workgroup folds its best
//   rank into a workspace slot with a 64-bit atomic max, and a
//   one-workgroup kernel after the GEMV reduces the slots to the token.

#include <type_traits>

#include "common.h"
#include "dnx_kernels.h"

using namespace dnx;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
// Weight formats: the engine's Q8 (fp32 scales) and Q4 (fp16 scales), and Q8
// with the GGUF Q8_0 block's own fp16 scale (34 B per 32 weights, not 36).
constexpr int kFmtQ8 = 0, kFmtQ4 = 1, kFmtQ8H = 2;
// Fused argmax. A rank orders (value, lowest index): argmax_key's 32-bit
// value order above the complemented row. Workgroup b folds its waves' best
// rank into workspace slot b % kArgmaxSlots with a 64-bit atomic max that
// nothing waits for (slots are shared only by grids above kArgmaxSlots
// workgroups); a one-workgroup finisher launched after the GEMV on the same
// stream reads and clears the slots with plain loads and stores and writes
// the token. The kernel boundary orders the atomics before those reads, so
// no fence, no arrival count and no atomic retry is needed.
constexpr int kArgmaxSlots = 256;
// Buffer offset of a request that must read zeros: past every matrix range
// (a launch covers less than 2 GB of codes).
constexpr uint32_t kDead = 0x80000000u;
constexpr int64_t kMaxLaunchBytes = ((int64_t)1 << 31) - 4096;
// Blocks per step of the FMA chains (two steps alternate, so a chain runs
// over a multiple of two steps; tiles of one or two rows take steps of
// 2 kChainStep, with registers to spare); each chain row carries kChainPad
// floats past its blocks (keeps the rows 16-byte aligned).
constexpr int kChainStep = 8;
constexpr int kChainPad = 4;

DNX_DEV uint64_t argmax_rank(float v, uint32_t row) {
  // A NaN at index 0 is the answer whatever follows (every comparison with
  // it is false): give it the one rank no value reaches.
  return (row == 0 && v != v) ? ~0ull : argmax_key(v, row);
}

struct GemvParams {
  const void* qs[2];
  const void* scales[2];
  const float* x;              // [n][cols] fp32
  float* y;                    // [n][ldy]; the pair writes SiLU(gate) * up
  float* y2;                   // pair: the up products too, when not null
  int rows, cols, n;           // rows of this launch (qs, scales, y start at its first)
  int ldy;                     // row stride of y and y2 (the matrix's rows)
  int row0;                    // the launch's first row in the matrix (argmax ranks)
  int tiles;                   // ceil(rows / R)
  int full;                    // 1: a tile's whole K goes to LDS before its chains run
  int stride;                  // LDS floats per chain: span of blocks + 4
  unsigned long long* ws;      // argmax: the rank slots, zero between calls
  int grid;                    // set by the launch
  // Segmented launches (kSeg, n = 1): up to kMaxSegs matrices of one format
  // and width over the same x, their tiles laid end to end; seg_end holds
  // the cumulative tile ends (INT_MAX past the last segment).
  int seg_end[4];
  int seg_rows[4];
  const void* seg_qs[4];
  const void* seg_scales[4];
  float* seg_y[4];
  // Residual add (plain launches, n = 1): when not null, each output is also
  // added into resid[row] (resid[row] + y[row], one rounding, as add_kernel).
  float* resid;
  // Fused RMSNorm of x (gemv_norm_kernel, n = 1): the launch quantizes
  // norm_w * (x * r) instead of x, and workgroup 0 writes it to norm_out.
  const float* norm_w;
  float* norm_out;
  float norm_eps;
  int norm_lds;                // LDS byte offset of workgroup 0's staged copy
};
constexpr int kMaxSegs = 4;

// The segment of a uniform tile index, as selects (an indexed read of the
// kernel's argument array would go through private memory).
template <class T>
DNX_DEV T seg_pick(const T (&a)[4], const int s) {
  return s == 0 ? a[0] : s == 1 ? a[1] : s == 2 ? a[2] : a[3];
}
DNX_DEV void seg_of(const GemvParams& p, const int tile, int& s, int& local) {
  s = (tile >= p.seg_end[0]) + (tile >= p.seg_end[1]) + (tile >= p.seg_end[2]);
  local = tile - (s == 0 ? 0 : s == 1 ? p.seg_end[0] : s == 2 ? p.seg_end[1] : p.seg_end[2]);
}

// Orders LDS writes and reads among the lanes of one wave (a wave's LDS
// operations execute in issue order; this keeps the compiler from moving
// them across).
DNX_DEV void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}


// The kernel body; kNorm: RMSNorm of x fused into the prologue (n = 1,
// 4 waves, one batch of quads; the launch checks these).
template <int F, int R, int NT, bool kPair, bool kArgmax, bool kF, int W, bool kSeg, bool kNorm>
__device__ __forceinline__ void gemv_body(const GemvParams p) {
  // kF: float inputs (lab_gemm_q8 / lab_gemm_q4 mode 0): x is not quantized;
  // per block, lane l sums fma(float(w_j), x_j, s) over j = 4k + l, k = 0..7
  // in order (dot_q8_f32 lab_native.c:489-501, dot_q4_f32 :1013-1023), and
  // the chains run acc_l = fma(s_l, sw, acc_l) on the weight scale alone.
  constexpr bool kQ4 = F == kFmtQ4;
  constexpr bool kHalf = F != kFmtQ8;          // fp16 block scales
  constexpr int CB = kQ4 ? 64 : 32;           // blocks per 1 KB chunk of a row
  constexpr int M = kPair ? 2 : 1;            // matrices sharing x
  constexpr int RR = R * M;                   // weight rows per tile
  constexpr int CH = NT * RR * 4;             // chain lanes per tile
  static_assert(CH <= 64, "a tile's chains must fit one wave");
  constexpr int G = RR >= 8 ? 1 : RR >= 2 ? 16 / RR : 8;  // chunk groups per ring batch
  // Tiles of 8+ rows refill each ring slot as soon as it is consumed (one
  // group of RR slots, 4 waves per SIMD); smaller tiles refill a group at a
  // time from a ring of 16 (measured faster for each).
  constexpr int Q = RR * G;                   // ring slots (row-chunks in flight)
  constexpr bool kFine = G == 1;
  constexpr int CS = RR <= 2 ? 2 * kChainStep : kChainStep;  // blocks per chain step
  constexpr int T = 64 * W;                   // threads of the workgroup (W waves)

  extern __shared__ __align__(16) unsigned char lds[];
  const int cols = p.cols, B = cols / kBlock, n = p.n;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar bookkeeping

  // x in LDS. int8 inputs: sxq [NT][cols], sxs [NT][B], Q4 sxsum [NT][B][4].
  // Float inputs: sxf [NT][B][4][8], x[t][32b + 4k + l] at [t][b][l][k], so
  // that one lane-sum chain reads 8 consecutive floats.
  int8_t* sxq = (int8_t*)lds;                              // [NT][cols]
  float* sxs = (float*)(lds + NT * cols);                  // [NT][B]
  int* sxsum = (int*)(sxs + ((NT * B + 3) & ~3));          // Q4: [NT][B][4]
  float* sxf = (float*)lds;
  const int CP = p.stride;  // floats per chain: a chunk (or the whole K) + kChainPad
  float* sf = (kF ? sxf + NT * cols : (float*)(sxsum + (kQ4 ? NT * B * 4 : 0))) +
              wave * (NT * RR * 5 * CP);
  float* ss = sf + NT * RR * 4 * CP;                       // [NT][RR][CP]

  const int chunks = (B + CB - 1) / CB;
  const int stride = gridDim.x * W;
  const int tile0 = blockIdx.x * W + wave;
  const int my_tiles = tile0 < p.tiles ? (p.tiles - 1 - tile0) / stride + 1 : 0;
  const int groups = my_tiles * chunks;                    // chunk groups of this wave
  const int lblk = kQ4 ? lane : (lane >> 1);               // lane's block in a chunk

  // Code and scale bytes per row, and one resource per matrix.
  const uint32_t qrow = kQ4 ? (uint32_t)cols / 2 : (uint32_t)cols;
  const uint32_t srow = (uint32_t)B * (kHalf ? 2 : 4);
  i32x4 rq[M], rs[M];
#pragma unroll
  for (int m = 0; m < M; m++) {
    rq[m] = buffer_rsrc(p.qs[m], (uint32_t)p.rows * qrow);
    rs[m] = buffer_rsrc(p.scales[m], (uint32_t)p.rows * srow);
  }

  uint4 raw[Q];
  // Raw scale bits, converted only when used: any operation on a loaded
  // value (even a zero-extension) makes the wave wait for that load there.
  using ScaleBits = std::conditional_t<kHalf, short, int>;
  ScaleBits swb[Q];

  // Requests row-chunk i of chunk c of this wave's k-th tile into ring slot
  // s0 + i. One buffer resource spans each matrix (the launch keeps a matrix
  // under 2 GB), so a request is an offset: rows past the matrix fall outside
  // the range and read zeros without a memory access, and so does a slot
  // past this wave's last tile (offset kDead); lanes past a row's last block
  // read the next row, and their results are never used. The issue has no
  // branch.
  // A segmented launch builds the resources of the tile's segment per
  // request (scalar selects).
  auto issue1 = [&](const int s0, const int k, const int c, const int i) {
    const int tile = tile0 + k * stride;
    const int blk = c * CB + lblk;
    const int m = i / R, r = i - (i / R) * R;
    int seg = 0, lt = tile;
    if (kSeg) seg_of(p, tile, seg, lt);
    const uint32_t row = (uint32_t)(lt * R + r);
    const bool live = k < my_tiles;
    const uint32_t oq = row * qrow + (kQ4 ? blk * 16 : blk * 32 + (lane & 1) * 16);
    const uint32_t os = row * srow + blk * (kHalf ? 2 : 4);
    i32x4 q = rq[m], sc = rs[m];
    if (kSeg) {
      const uint32_t rows_s = (uint32_t)seg_pick(p.seg_rows, seg);
      q = buffer_rsrc(seg_pick(p.seg_qs, seg), rows_s * qrow);
      sc = buffer_rsrc(seg_pick(p.seg_scales, seg), rows_s * srow);
    }
    raw[s0 + i] = buffer_load16_stream(q, (int)(live ? oq : kDead));
    // fp16 scales with the default cache policy: a Q8 row's 128-byte scale
    // line is read by two requests (half a row each); with the streaming
    // policy the second fetched the line from HBM again (the LM head read
    // 1.05x its bytes; 1.00x this way).
    if (kHalf) {
      swb[s0 + i] = dnx_raw_buffer_load_i16(sc, (int)(live ? os : kDead), 0, 0);
    } else {
      swb[s0 + i] = dnx_raw_buffer_load_i32(sc, (int)(live ? os : kDead), 0, kStream);
    }
  };
  auto issue = [&](const int s0, const int k, const int c) {
#pragma unroll
    for (int i = 0; i < RR; i++) issue1(s0, k, c, i);
  };
  // Next chunk group: the following chunk of the tile, or the next tile.
  auto advance = [&](int& k, int& c) {
    if (++c == chunks) {
      c = 0;
      ++k;
    }
  };

  // Prologue: the n input rows quantized into LDS (lab_quantize_q8, fused).
  // The first batch of x is requested before the first weight chunks (loads
  // complete in order, so x must not queue behind the weights), then the
  // weight ring is filled, then x is quantized while the weights stream.
  // Rows of tokens t >= n are never stored, so their LDS is left as is.
  // A batch is PQ = 8 quads per thread: quad q0 + j T + tid for j < 8, so for
  // each j the 8 lanes of an aligned group hold one 32-value block.
  // The n rows are one flat array of n * cols / 4 quads (x is [n][cols] and
  // the LDS copies are [NT][...] in the same order, and a block never
  // straddles two rows), so the first batch covers up to 2048 quads of all
  // tokens: at n = 4 the tokens no longer wait for each other's loads.
  constexpr int PQ = 8;
  const int quads = n * (cols / 4);
  float4 v[PQ];
  float4 nw[kNorm ? PQ : 1];  // kNorm: the norm weights of the same quads
  const i32x4 rx = buffer_rsrc(p.x, (uint32_t)(n * cols) * 4);
  const i32x4 rnw = buffer_rsrc(kNorm ? p.norm_w : p.x, (uint32_t)cols * 4);
  auto load_x = [&](const int q0) {
#pragma unroll
    for (int j = 0; j < PQ; j++) {
      const int q = q0 + j * T + tid;  // past the rows: zeros, unused
      v[j] = buffer_load_f4(rx, q * 16);
      if constexpr (kNorm) nw[j] = buffer_load_f4(rnw, q * 16);
    }
  };
  // Residual add (plain one-token launches): this lane's deferred result is
  // chain group j of the wave's tile k (lane = k * R + j, the order the loop
  // records results in), so its x[row] is requested now, first of all, and
  // left raw until the end.
  constexpr bool kResid = !kPair && !kArgmax && !kSeg && !kF && !kNorm && NT == 1;
  int resid_bits = 0;
  if (kResid && p.resid != nullptr) {
    const int k = lane / R, j = lane - (lane / R) * R;
    const int row = (tile0 + k * stride) * R + j;
    const bool ok = k < my_tiles && row < p.rows;
    const i32x4 rr = buffer_rsrc(p.resid, (uint32_t)p.rows * 4);
    resid_bits = dnx_raw_buffer_load_i32(rr, (int)(ok ? (uint32_t)row * 4 : kDead), 0, 0);
  }
  int pk = 0, pc = 0;  // position of the next chunk group to request
  auto quantize_x = [&](const int q0) {
    if (kF) {
#pragma unroll
      for (int j = 0; j < PQ; j++) {
        const int q = q0 + j * T + tid;
        if (q >= quads) break;
        // quad q is k = q % 8 of (flat) block q / 8, l = 0..3
        float* d = sxf + (q >> 3) * 32 + (q & 7);
        d[0] = v[j].x;
        d[8] = v[j].y;
        d[16] = v[j].z;
        d[24] = v[j].w;
      }
      return;
    }
    // Each group's 8 block maxima (one per j), then one correctly rounded
    // scale and inverse per lane: lane 8g + k divides for j = k, and the
    // group's lanes fetch the other seven inverses with a swizzle broadcast
    // (every lane is active here: the loop below diverges, this does not).
    float am[PQ];
#pragma unroll
    for (int j = 0; j < PQ; j++) am[j] = group8_max_nonneg(fmaxf(0.0f, max4abs(v[j])));
    const int k = lane & 7;
    float a = am[0];
#pragma unroll
    for (int j = 1; j < PQ; j++) a = k == j ? am[j] : a;
    const float scale = q8_scale(a);
    const float inv_k = q8_inv(scale);
    {
      const int q = q0 + k * T + (tid & ~7);  // first quad of lane k's block
      if (q < quads) sxs[q >> 3] = scale;
    }
    static_assert(PQ == 8, "one division per lane of an 8-lane group");
    const float inv[PQ] = {bcast8<0>(inv_k), bcast8<1>(inv_k), bcast8<2>(inv_k),
                           bcast8<3>(inv_k), bcast8<4>(inv_k), bcast8<5>(inv_k),
                           bcast8<6>(inv_k), bcast8<7>(inv_k)};
#pragma unroll
    for (int j = 0; j < PQ; j++) {
      const int q = q0 + j * T + tid;
      if (q >= quads) break;  // whole 8-lane groups: quads is a multiple of 8
      const int packed = quant4(v[j], inv[j]);
      *(int*)(sxq + q * 4) = packed;
      if (kQ4) {
        // -8 * (sum of the x bytes meeting lane l's low and high nibbles):
        // quads l and l + 4 of the block, so the nibbles enter sdot as 0..15.
        const int jq = q & 7;  // quad within the block
        const int s = sdot4(packed, 0x01010101, 0);
        const int other = dpp<kRowShl4>(s);  // lane + 4: quad jq + 4 of the block
        if (jq < 4) sxsum[(q >> 3) * 4 + jq] = -8 * (s + other);
      }
    }
  };
  load_x(0);
  // Slots past the wave's last tile are not requested (a uniform branch:
  // such requests would read nothing and only cost their instructions).
#pragma unroll
  for (int g = 0; g < G; g++) {
    if (pk < my_tiles) issue(g * RR, pk, pc);
    advance(pk, pc);
  }
  // The first batch straight after the ring is filled (no loop around it,
  // so waiting for x does not wait for the weights behind it). The
  // scheduling barrier keeps every weight request ahead of the first wait
  // for x (the scheduler would otherwise start the block maxima in between).
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (kNorm) {
    // RMSNorm of the one row (rms_norm_vec_kernel's values): thread t holds
    // quads t + 256 j, as there; its sum of squares in that order over the
    // batches that hold quads of the row (the rest are zeros, which would
    // add +0), each wave's DPP sum, then the four waves in order (the
    // arithmetic of norm_row_sum); r = 1 / sqrt(sum / cols + eps);
    // a = w * (x * r).
    __shared__ float nred[4];
    const int live_j = (quads + T - 1) / T;  // uniform
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < PQ; j++) {
      if (j < live_j) {
        sum += v[j].x * v[j].x;
        sum += v[j].y * v[j].y;
        sum += v[j].z * v[j].z;
        sum += v[j].w * v[j].w;
      }
    }
    sum = wave_sum_dpp(sum);
    if (lane == 0) nred[wave] = sum;
    __syncthreads();
    float total = nred[0];
#pragma unroll
    for (int w = 1; w < 4; w++) total += nred[w];
    const float r = 1.0f / sqrtf(total / (float)cols + p.norm_eps);
    float4* staged = (float4*)(lds + p.norm_lds);  // workgroup 0's copy of a
#pragma unroll
    for (int j = 0; j < PQ; j++) {
      if (j < live_j) {
        v[j].x = nw[j].x * (v[j].x * r);
        v[j].y = nw[j].y * (v[j].y * r);
        v[j].z = nw[j].z * (v[j].z * r);
        v[j].w = nw[j].w * (v[j].w * r);
        const int q = j * T + tid;
        if (blockIdx.x == 0 && q < quads) staged[q] = v[j];
      }
    }
  }
  quantize_x(0);
  for (int q0 = T * PQ; q0 < quads; q0 += T * PQ) {
    load_x(q0);
    quantize_x(q0);
  }
  __syncthreads();  // the only workgroup barrier: x is ready

  float acc = 0.0f;
  uint64_t best = 0;
  int ck = 0, cc = 0;  // position of the chunk group being consumed
  // Deferred outputs: lane j holds the j-th result of the wave's tiles (value
  // and destination), stored after the loop. A store among the loads would
  // make every later wait drain all loads in flight (loads and stores share
  // one counter on this GPU, and with a store pending the compiler waits for
  // zero). The launch gives a wave at most 64 / kOut tiles.
  constexpr int kOut = NT * RR;  // results per tile (chain groups)
  float outv = 0.0f;
  float* outp = nullptr;
  int pend = 0;  // uniform: results recorded so far
  for (int base = 0; base < groups; base += G) {
#pragma unroll
    for (int g = 0; g < G; g++) {
      if (base + g >= groups) break;  // uniform across the wave
      const int tile = tile0 + ck * stride;
      // Lanes past the row's last block (ok false) store zeros; their slots
      // up to the next multiple of 4 are read by the chains, the rest are
      // in bounds and never read. Selects, not branches: a branch here makes
      // the compiler wait for every load in flight.
      const int nb = min(CB, B - cc * CB);
      const bool ok = lblk < nb;
      const int blk = cc * CB + (ok ? lblk : 0);
      const int at = p.full ? cc * CB + lblk : lblk;  // block slot in this chain's LDS
      // The chunk's quantized x for this lane's block, read once for all the
      // tile's rows (int8 inputs; read per row, the reads would wait behind
      // each row's LDS writes).
      int4 xfa[NT], xfb[NT], xfc[NT];
      float xfs[NT];
      if (!kF) {
#pragma unroll
        for (int t = 0; t < NT; t++) {
          if (kQ4) {
            xfa[t] = *(const int4*)(sxq + t * cols + blk * 32);
            xfb[t] = *(const int4*)(sxq + t * cols + blk * 32 + 16);
            xfc[t] = *(const int4*)(sxsum + (t * B + blk) * 4);
          } else {
            xfa[t] = *(const int4*)(sxq + t * cols + blk * 32 + (lane & 1) * 16);
          }
          xfs[t] = sxs[t * B + blk];
        }
      }
      // Row-chunks -> lane sums and block scales in LDS.
#pragma unroll
      for (int i = 0; i < RR; i++) {
        const uint4 w = raw[g * RR + i];
        const float swi = kHalf ? half_bits_to_float((uint16_t)swb[g * RR + i])
                                : __int_as_float((int)swb[g * RR + i]);
#pragma unroll
        for (int t = 0; t < NT; t++) {
          float* f = sf + ((t * RR + i) * 4) * CP + at;
          float* sp = ss + (t * RR + i) * CP + at;
          if (kF && kQ4) {
            // Lane = block. Weight 4k + l: low nibble of byte 4k + l for
            // k < 4, high nibble of byte 4(k - 4) + l after.
            const uint32_t lo[4] = {w.x & 0x0f0f0f0fu, w.y & 0x0f0f0f0fu, w.z & 0x0f0f0f0fu,
                                    w.w & 0x0f0f0f0fu};
            const uint32_t hi[4] = {(w.x >> 4) & 0x0f0f0f0fu, (w.y >> 4) & 0x0f0f0f0fu,
                                    (w.z >> 4) & 0x0f0f0f0fu, (w.w >> 4) & 0x0f0f0f0fu};
            const float* xb = sxf + (t * B + blk) * 32;
#pragma unroll
            for (int l = 0; l < 4; l++) {
              const float4 xa = *(const float4*)(xb + l * 8);
              const float4 xc = *(const float4*)(xb + l * 8 + 4);
              const int sh = 8 * l;
              float sl = fmaf((float)((lo[0] >> sh) & 0xffu) - 8.0f, xa.x, 0.0f);
              sl = fmaf((float)((lo[1] >> sh) & 0xffu) - 8.0f, xa.y, sl);
              sl = fmaf((float)((lo[2] >> sh) & 0xffu) - 8.0f, xa.z, sl);
              sl = fmaf((float)((lo[3] >> sh) & 0xffu) - 8.0f, xa.w, sl);
              sl = fmaf((float)((hi[0] >> sh) & 0xffu) - 8.0f, xc.x, sl);
              sl = fmaf((float)((hi[1] >> sh) & 0xffu) - 8.0f, xc.y, sl);
              sl = fmaf((float)((hi[2] >> sh) & 0xffu) - 8.0f, xc.z, sl);
              sl = fmaf((float)((hi[3] >> sh) & 0xffu) - 8.0f, xc.w, sl);
              f[l * CP] = ok ? sl : 0.0f;
            }
            *sp = ok ? swi : 0.0f;
          } else if (kF) {
            // Q8, two lanes per block: lane h holds bytes 16h..16h+15 (k =
            // 4h..4h+3 of every l) and takes lanes l = 2h, 2h + 1. Each lane
            // keeps bytes 2h, 2h + 1 of its dwords and gives the partner the
            // other two, so both end with all 8 k of their two l.
            const int h = lane & 1;
            const uint32_t keep = h ? 0x07060302u : 0x05040100u;
            const uint32_t give = h ? 0x05040100u : 0x07060302u;
            const uint32_t k0 = __builtin_amdgcn_perm(w.y, w.x, keep);
            const uint32_t k1 = __builtin_amdgcn_perm(w.w, w.z, keep);
            const uint32_t r0 = (uint32_t)dpp<kQuadXor1>((int)__builtin_amdgcn_perm(w.y, w.x, give));
            const uint32_t r1 = (uint32_t)dpp<kQuadXor1>((int)__builtin_amdgcn_perm(w.w, w.z, give));
            const uint32_t a0 = h ? r0 : k0, a1 = h ? r1 : k1;  // k = 0..3
            const uint32_t c0 = h ? k0 : r0, c1 = h ? k1 : r1;  // k = 4..7
            const float* xl = sxf + (t * B + blk) * 32 + 2 * h * 8;
            float* fh = f + 2 * h * CP;
#pragma unroll
            for (int e = 0; e < 2; e++) {  // l = 2h + e: bytes e and e + 2 of each word
              const float4 xa = *(const float4*)(xl + e * 8);
              const float4 xc = *(const float4*)(xl + e * 8 + 4);
              const int s0 = 8 * e, s1 = 8 * e + 16;
              float sl = fmaf((float)(int8_t)(a0 >> s0), xa.x, 0.0f);
              sl = fmaf((float)(int8_t)(a0 >> s1), xa.y, sl);
              sl = fmaf((float)(int8_t)(a1 >> s0), xa.z, sl);
              sl = fmaf((float)(int8_t)(a1 >> s1), xa.w, sl);
              sl = fmaf((float)(int8_t)(c0 >> s0), xc.x, sl);
              sl = fmaf((float)(int8_t)(c0 >> s1), xc.y, sl);
              sl = fmaf((float)(int8_t)(c1 >> s0), xc.z, sl);
              sl = fmaf((float)(int8_t)(c1 >> s1), xc.w, sl);
              fh[e * CP] = ok ? sl : 0.0f;
            }
            *sp = ok ? swi : 0.0f;  // both lanes of the block: the same value
          } else if (kQ4) {
            const int4 xa = xfa[t], xb = xfb[t], c8 = xfc[t];
            const int mk = 0x0f0f0f0f;
            const int d0 = sdot4(w.x & mk, xa.x, sdot4((w.x >> 4) & mk, xb.x, c8.x));
            const int d1 = sdot4(w.y & mk, xa.y, sdot4((w.y >> 4) & mk, xb.y, c8.y));
            const int d2 = sdot4(w.z & mk, xa.z, sdot4((w.z >> 4) & mk, xb.z, c8.z));
            const int d3 = sdot4(w.w & mk, xa.w, sdot4((w.w >> 4) & mk, xb.w, c8.w));
            const float sb = swi * xfs[t];
            f[0] = ok ? (float)d0 : 0.0f;
            f[CP] = ok ? (float)d1 : 0.0f;
            f[2 * CP] = ok ? (float)d2 : 0.0f;
            f[3 * CP] = ok ? (float)d3 : 0.0f;
            *sp = ok ? sb : 0.0f;
          } else {
            const int h = lane & 1;
            const int4 xv = xfa[t];
            int p0 = sdot4(w.x, xv.x, 0), p1 = sdot4(w.y, xv.y, 0);
            int p2 = sdot4(w.z, xv.z, 0), p3 = sdot4(w.w, xv.w, 0);
            // Lane l's sum takes 4 bytes of each half: add the partner's.
            p0 += dpp<kQuadXor1>(p0);
            p1 += dpp<kQuadXor1>(p1);
            p2 += dpp<kQuadXor1>(p2);
            p3 += dpp<kQuadXor1>(p3);
            float* fh = f + 2 * h * CP;
            const float sb = swi * xfs[t];
            fh[0] = ok ? (float)(h ? p2 : p0) : 0.0f;
            fh[CP] = ok ? (float)(h ? p3 : p1) : 0.0f;
            *sp = ok ? sb : 0.0f;  // both lanes of the block: the same value
          }
        }
        // The slot is free: refill it now (unconditionally: a branch here
        // makes the compiler wait for every load in flight).
        if (kFine) issue1(g * RR, pk, pc, i);
      }
      // Refill these ring slots with the chunk group one batch ahead.
      if (!kFine && pk < my_tiles) issue(g * RR, pk, pc);
      advance(pk, pc);
      if (!p.full || cc == chunks - 1) {
        // The FMA chains, in block order: over this chunk, or (full-K tiles)
        // over the whole row at its last chunk.
        // Two register buffers of CS blocks alternate: one step's chain
        // runs while the other's LDS reads are in flight. Every slot of a
        // chunk is written (zeros past the row's last block, and
        // fma(0, 0, acc) = acc: acc is never -0), so the chain may run on to
        // a multiple of 2 CS. Buffer a starts as zeros rather than a read:
        // with a read there the compiler folds both buffers' reads back into
        // one read at the top of each step, and the latency returns.
        const int end = (p.full ? cc * CB : 0) + ((nb + 2 * CS - 1) & ~(2 * CS - 1));
        wave_sync();
        if (lane < CH) {
          const float* fp = sf + lane * CP;
          const float* sp = ss + (lane >> 2) * CP;
          float4 fa[CS / 4], sa[CS / 4], fb[CS / 4], sb[CS / 4];
          auto read = [&](float4* f, float4* sv, const int b) {
#pragma unroll
            for (int i = 0; i < CS / 4; i++) {
              f[i] = *(const float4*)(fp + b + 4 * i);
              sv[i] = *(const float4*)(sp + b + 4 * i);
            }
          };
          auto chain = [&](const float4* f, const float4* sv) {
#pragma unroll
            for (int i = 0; i < CS / 4; i++) {
              acc = fmaf(f[i].x, sv[i].x, acc);
              acc = fmaf(f[i].y, sv[i].y, acc);
              acc = fmaf(f[i].z, sv[i].z, acc);
              acc = fmaf(f[i].w, sv[i].w, acc);
            }
          };
#pragma unroll
          for (int i = 0; i < CS / 4; i++) {
            fa[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            sa[i] = fa[i];
          }
          // a: blocks [b - CS, b); b: blocks [b, b + CS).
          for (int b = 0; b < end; b += 2 * CS) {
            read(fb, sb, b);
            chain(fa, sa);
            read(fa, sa, b + CS);
            chain(fb, sb);
          }
          chain(fa, sa);
        }
        wave_sync();
      }
      if (cc == chunks - 1) {
        // (acc0 + acc1) + (acc2 + acc3) over each group of 4 chain lanes.
        float v = acc + dppf<kQuadXor1>(acc);
        v = v + dppf<kQuadXor2>(v);
        acc = 0.0f;
        const int tr = lane >> 2, t = tr / RR, i = tr - (tr / RR) * RR;
        int seg = 0, lt = tile;
        if (kSeg) seg_of(p, tile, seg, lt);
        const int row = lt * R + (i % R);
        const int rows_here = kSeg ? seg_pick(p.seg_rows, seg) : p.rows;
        const bool lead = lane < CH && (lane & 3) == 0 && t < n && row < rows_here;
        float val = v;
        float* dst = nullptr;
        if (kPair) {
          const float up = __shfl(v, lane + R * 4);  // the up row of this gate row
          if (lead && i < R) {
            val = silu_mul_exact(v, up);
            dst = p.y + (size_t)t * p.ldy + row;
          } else if (lead && p.y2 != nullptr) {
            dst = p.y2 + (size_t)t * p.ldy + row;
          }
        } else if (kSeg) {
          if (lead) dst = seg_pick(p.seg_y, seg) + row;  // n = 1
        } else {
          if (lead) dst = p.y + (size_t)t * p.ldy + row;
          if (kArgmax) {
            const uint64_t key = lead ? argmax_rank(v, (uint32_t)(p.row0 + row)) : 0;
            const uint64_t m = wave_max_u64(key);
            best = m > best ? m : best;
          }
        }
        // Result j of this tile (chain group j, lane 4j) -> lane pend + j.
        const int j = lane - pend;
        const bool mine = j >= 0 && j < kOut;
        const int src = mine ? 4 * j : lane;
        const float mv = __shfl(val, src);
        const long long mp = __shfl((long long)(uintptr_t)dst, src);
        if (mine) {
          outv = mv;
          outp = (float*)(uintptr_t)mp;
        }
        pend += kOut;
      }
      advance(ck, cc);
    }
  }
  if (outp != nullptr) *outp = outv;
  if (kResid && p.resid != nullptr && outp != nullptr) {
    float* rp = p.resid + (outp - p.y);  // n = 1: the same row of x
    *rp = __int_as_float(resid_bits) + outv;
  }
  if constexpr (kNorm) {
    // The normed row to its own buffer (each thread its staged quads; the
    // stores wait until here so that none queues among the weight loads).
    if (blockIdx.x == 0) {
      const float4* staged = (const float4*)(lds + p.norm_lds);
#pragma unroll
      for (int j = 0; j < PQ; j++) {
        const int q = j * T + tid;
        if (q < quads) ((float4*)p.norm_out)[q] = staged[q];
      }
    }
  }

  if (kArgmax) {
    // The workgroup's best rank into its group word (the finisher reads it).
    __shared__ uint64_t red[W];
    if (lane == 0) red[wave] = best;
    __syncthreads();
    if (tid == 0) {
      uint64_t b = red[0];
      for (int w = 1; w < W; w++) b = red[w] > b ? red[w] : b;
      if (b != 0) {
        __hip_atomic_fetch_max(&p.ws[blockIdx.x % kArgmaxSlots], (unsigned long long)b,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

template <int F, int R, int NT, bool kPair, bool kArgmax, bool kF, int W, bool kSeg>
__global__ void __launch_bounds__(64 * W) gemv_kernel(GemvParams p) {
  gemv_body<F, R, NT, kPair, kArgmax, kF, W, kSeg, false>(p);
}

// One token whose x is first normed (the standalone RMSNorm's values: the
// same partition of the row over 256 threads and the same reduction), then
// quantized and multiplied: one matrix, a gate/up pair or a segmented
// launch.
template <int F, int R, bool kPair, bool kSeg>
__global__ void __launch_bounds__(256) gemv_norm_kernel(GemvParams p) {
  gemv_body<F, R, 1, kPair, false, false, 4, kSeg, true>(p);
}

// The fused argmax's last step: the best of the first `slots` workspace
// slots (clearing each for the next call) -> the token. Rank 0 means no value
// was a number: index 0.
__global__ void __launch_bounds__(kThreads) argmax_finish_kernel(unsigned long long* ws,
                                                                 int slots, int64_t* out) {
  const int tid = threadIdx.x;
  constexpr int kPer = kArgmaxSlots / kThreads;
  uint64_t v[kPer];
#pragma unroll
  for (int j = 0; j < kPer; j++) {  // all loads in flight at once
    const int i = j * kThreads + tid;
    v[j] = i < slots ? ws[i] : 0;
  }
  uint64_t r = 0;
#pragma unroll
  for (int j = 0; j < kPer; j++) {
    const int i = j * kThreads + tid;
    r = v[j] > r ? v[j] : r;
    if (i < slots) ws[i] = 0;
  }
  __shared__ uint64_t red[kWaves];
  r = wave_max_u64(r);
  if ((tid & 63) == 0) red[tid >> 6] = r;
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kWaves; w++) r = red[w] > r ? red[w] : r;
    *out = r == 0 ? 0 : (int64_t)(0xffffffffu - (uint32_t)(r & 0xffffffffu));
  }
}

// ------------------------------------------------------------ launch

int cu_count() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0) {
      cus = 256;
    }
  }
  return cus;
}

// LDS of one workgroup of W waves for a chain stride (matches the carving in
// gemv_kernel).
size_t lds_for(bool q4, bool fx, int R, int nt, bool pair, int cols, int stride, int W) {
  const int RR = R * (pair ? 2 : 1), B = cols / kBlock;
  const size_t x = fx ? (size_t)nt * cols * 4
                      : (size_t)nt * cols + 4 * (size_t)((nt * B + 3) & ~3) +
                            (q4 ? (size_t)nt * B * 16 : 0);
  return x + (size_t)W * nt * RR * 5 * stride * 4;
}

// Matrices of at most kWideRows rows are "small" (the decode step's
// projections); an x of at least kWideCols columns is "long".
constexpr int kWideRows = 16384;
constexpr int kWideCols = 4096;

// LDS budgets: 4-wave workgroups share a CU with others and keep to 64 KB;
// an 8-wave workgroup runs alone on its CU and may use the CU's 160 KB.
constexpr size_t kLdsShared = 64 * 1024;
constexpr size_t kLdsAlone = 160 * 1024;
size_t lds_budget(int W) { return W >= 8 ? kLdsAlone : kLdsShared; }

// Ring slots per wave (the kernel's Q) for RR rows per tile.
int ring_units(int RR) { return RR >= 8 ? RR : RR >= 2 ? 16 : 8; }

template <int F, int R, int NT, bool kPair, bool kArgmax, bool kF, int W, bool kSeg = false,
          bool kNorm = false>
int launch(GemvParams& p, hipStream_t stream) {
  constexpr bool kQ4 = F == kFmtQ4;
  constexpr int CB = kQ4 ? 64 : 32, RR = R * (kPair ? 2 : 1);
  static_assert(!kNorm || (NT == 1 && W == 4 && !kArgmax && !kF), "the fused norm's shape");
  const int B = p.cols / kBlock, chunks = (B + CB - 1) / CB;
  const size_t budget = lds_budget(W);
  // The fused norm stages workgroup 0's normed row past everything else.
  const size_t extra = kNorm ? (size_t)p.cols * 4 : 0;
  // Full-K tiles when the whole tile fits the ring (small tiles, where the
  // chain per chunk would otherwise serialize with each chunk's latency).
  p.full = RR * chunks <= ring_units(RR) &&
           lds_for(kQ4, kF, R, NT, kPair, p.cols, chunks * CB + kChainPad, W) + extra <= budget;
  p.stride = (p.full ? chunks * CB : CB) + kChainPad;
  const size_t lds0 = lds_for(kQ4, kF, R, NT, kPair, p.cols, p.stride, W);
  const size_t lds = lds0 + extra;
  if (lds > budget) return DNX_EINVAL;  // x too wide for one workgroup's LDS
  p.norm_lds = (int)lds0;  // a multiple of 16 (cols is a multiple of 32)
  void (*kernel)(GemvParams);
  if constexpr (kNorm) {
    kernel = gemv_norm_kernel<F, R, kPair, kSeg>;
  } else {
    kernel = gemv_kernel<F, R, NT, kPair, kArgmax, kF, W, kSeg>;
  }
  // Persistent grid: as many workgroups as stay resident (the occupancy is
  // looked up once per kernel and LDS size).
  static int cached_per_cu = 0;
  static size_t cached_lds = 0;
  if (cached_per_cu == 0 || cached_lds != lds) {
    if (lds > kLdsShared &&
        hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess) {
      return DNX_ELAUNCH;
    }
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 64 * W, lds) !=
            hipSuccess ||
        per_cu < 1) {
      per_cu = 1;
    }
    cached_per_cu = per_cu;
    cached_lds = lds;
  }
  if (kSeg) {
    // Each segment starts on a tile: cumulative tile ends at R rows per tile.
    int end = 0;
    for (int i = 0; i < kMaxSegs; i++) {
      if (p.seg_rows[i] > 0) {
        end += (p.seg_rows[i] + R - 1) / R;
        p.seg_end[i] = end;
      } else {
        p.seg_end[i] = 0x7fffffff;
      }
    }
    p.tiles = end;
  } else {
    p.tiles = (p.rows + R - 1) / R;
  }
  const int need = (p.tiles + W - 1) / W;
  int cap = cached_per_cu * cu_count();
  // A wave defers its results in one register across its 64 lanes: at most
  // 64 / (NT * RR) tiles per wave, so at least this many workgroups.
  const int per_wave = 64 / (NT * RR);
  const int floor_grid = (p.tiles + W * per_wave - 1) / (W * per_wave);
  // Small matrices (a few thousand tiles: the decode step's projections)
  // run 8-wave workgroups, one per CU, so that each CU quantizes x once;
  // 4-wave launches of them keep two workgroups per CU (fewer workgroups
  // quantize x and wait at their one barrier, and the waves left keep
  // enough loads in flight). The LM head keeps the full grid.
  const int per_cu_small = W >= 8 ? 1 : 2;
  if (p.tiles <= 4096 && cap > per_cu_small * cu_count()) cap = per_cu_small * cu_count();
  if (cap < floor_grid) cap = floor_grid;
  const int grid = need < cap ? need : cap;
  p.grid = grid;
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(64 * W), lds, stream, p);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

// Rows per tile: the largest of 8 that still gives at least kMinTiles
// tiles, halving down to 1 for small matrices; bounded so a tile's chains
// fit a wave and a 4-wave workgroup's LDS stays within 64 KB. Single
// matrices with a short x take fewer, larger tiles (fewer workgroups
// quantize x): measured graph-timed, 3072 x 1024 Q8 4.41 -> 4.13 us with
// 4-row tiles, 2048 x 2048 Q4 4.64 -> 4.32 us with 2-row tiles.
constexpr int kMinTiles = 2048, kMinTilesShortX = 768;
int pick_rows(bool q4, bool fx, int rows, int nt, bool pair, int cols, size_t extra = 0) {
  int r = 8;  // 8 rows keep two chunk groups in the ring (measured faster than 16)
  while (r * nt * (pair ? 2 : 1) * 4 > 64) r /= 2;
  const int min_tiles = pair || cols >= kWideCols ? kMinTiles : kMinTilesShortX;
  while (r > 1 && (rows + r - 1) / r < min_tiles) r /= 2;
  while (r > 1 && lds_for(q4, fx, r, nt, pair, cols, (q4 ? 64 : 32) + kChainPad, 4) + extra >
                      kLdsShared) {
    r /= 2;
  }
  return r;
}

// Waves per workgroup: 8 (one workgroup per CU, so each CU quantizes x
// once) for matrices of at most kWideRows rows and at least kWideCols
// columns whose chains fit the CU's LDS, else 4. Measured graph-timed:
// 2048 x 6144 Q4 7.5 -> 6.9 us with 8 waves; a short x does better on two
// 4-wave workgroups per CU (3072 x 1024 Q8 4.6 against 5.0 us, the
// 6144 x 2048 Q4 pair 7.3 against 9.0 us).
int pick_waves(bool q4, bool fx, int rows, int R, int nt, bool pair, int cols) {
  if (rows > kWideRows || cols < kWideCols) return 4;
  return lds_for(q4, fx, R, nt, pair, cols, (q4 ? 64 : 32) + kChainPad, 8) <= kLdsAlone ? 8 : 4;
}

template <int F, int R, int NT, bool kPair, bool kArgmax, bool kF, bool kSeg = false>
int launch_w(GemvParams& p, int W, hipStream_t stream) {
  return W >= 8 ? launch<F, R, NT, kPair, kArgmax, kF, 8, kSeg>(p, stream)
                : launch<F, R, NT, kPair, kArgmax, kF, 4, kSeg>(p, stream);
}

// A segmented launch (one token, int8 inputs), R rows per tile.
template <int F>
int launch_seg(GemvParams& p, int R, int W, hipStream_t stream) {
  switch (R) {
    case 8: return launch_w<F, 8, 1, false, false, false, true>(p, W, stream);
    case 4: return launch_w<F, 4, 1, false, false, false, true>(p, W, stream);
    case 2: return launch_w<F, 2, 1, false, false, false, true>(p, W, stream);
    default: return launch_w<F, 1, 1, false, false, false, true>(p, W, stream);
  }
}

// A fused-norm launch (one token, 4 waves): one matrix, a gate/up pair or a
// segmented launch, R rows per tile.
template <int F, bool kPair, bool kSeg>
int launch_norm(GemvParams& p, int R, hipStream_t stream) {
  switch (R) {
    case 8: return launch<F, 8, 1, kPair, false, false, 4, kSeg, true>(p, stream);
    case 4: return launch<F, 4, 1, kPair, false, false, 4, kSeg, true>(p, stream);
    case 2: return launch<F, 2, 1, kPair, false, false, 4, kSeg, true>(p, stream);
    case 1: return launch<F, 1, 1, kPair, false, false, 4, kSeg, true>(p, stream);
  }
  return DNX_EINVAL;
}

// The fused norm's operands: RMSNorm(x) * w (one row) goes to out, and the
// launch multiplies it.
struct NormArgs {
  const float* w;
  float* out;
  float eps;
};

// Shapes the fused norm takes: one row of cols % 4 == 0 held by 256 threads
// in one batch of 8 quads each (cols <= 8192), 16-byte aligned operands (the
// alignment under which dnx_rms_norm itself runs the register-row kernel
// whose values the fusion reproduces), out disjoint from x.
bool disjoint(const void* a, int64_t abytes, const void* b, int64_t bbytes) {
  const uintptr_t a0 = (uintptr_t)a, b0 = (uintptr_t)b;
  return a0 + (uintptr_t)abytes <= b0 || b0 + (uintptr_t)bbytes <= a0;
}

bool norm_ok(const float* x, const NormArgs& nm, int64_t cols) {
  if (cols <= 0 || cols % 4 != 0 || cols > 4 * 256 * 8) return false;
  if ((((uintptr_t)x | (uintptr_t)nm.w | (uintptr_t)nm.out) & 15) != 0) return false;
  return disjoint(x, cols * 4, nm.out, cols * 4) && disjoint(nm.w, cols * 4, nm.out, cols * 4);
}

template <int F, int NT, bool kPair, bool kArgmax, bool kF>
int launch_nt(GemvParams& p, int R, int W, hipStream_t stream) {
  constexpr int RR_MAX = 16 / (NT * (kPair ? 2 : 1));
  switch (R) {
    case 8:
      if constexpr (RR_MAX >= 8) return launch_w<F, 8, NT, kPair, kArgmax, kF>(p, W, stream);
      break;
    case 4:
      if constexpr (RR_MAX >= 4) return launch_w<F, 4, NT, kPair, kArgmax, kF>(p, W, stream);
      break;
    case 2:
      if constexpr (RR_MAX >= 2) return launch_w<F, 2, NT, kPair, kArgmax, kF>(p, W, stream);
      break;
    case 1:
      return launch_w<F, 1, NT, kPair, kArgmax, kF>(p, W, stream);
  }
  return DNX_EINVAL;
}

template <int F, bool kPair, bool kArgmax, bool kF = false>
int gemv(const void* qs0, const void* sc0, const void* qs1, const void* sc1, const float* x,
         float* y, float* y2, int64_t rows, int64_t cols, int64_t n, unsigned long long* ws,
         int64_t* out, hipStream_t stream, float* resid = nullptr,
         const NormArgs* norm = nullptr) {
  if (rows <= 0 || cols <= 0 || n <= 0 || n > 4 || cols % kBlock != 0) return DNX_EINVAL;
  if (resid != nullptr && (kPair || kArgmax || kF || n != 1 || ((uintptr_t)resid & 3))) {
    return DNX_EINVAL;
  }
  if (norm != nullptr && (kArgmax || kF || n != 1 || !norm_ok(x, *norm, cols))) return DNX_EINVAL;
  if (rows > (1 << 30) || cols > (1 << 20)) return DNX_EINVAL;
  if (((uintptr_t)qs0 & 15) || (kPair && ((uintptr_t)qs1 & 15))) return DNX_EINVAL;
  constexpr bool kQ4 = F == kFmtQ4;
  if (((uintptr_t)x & 3) || ((uintptr_t)sc0 & (F != kFmtQ8 ? 1 : 3))) return DNX_EINVAL;
  if (kPair && ((uintptr_t)sc1 & (F != kFmtQ8 ? 1 : 3))) return DNX_EINVAL;
  if ((int64_t)rows * (kQ4 ? cols / 2 : cols) > ((int64_t)1 << 40)) return DNX_EINVAL;
  if (kArgmax && (n != 1 || ws == nullptr || out == nullptr)) return DNX_EINVAL;
  // Launches over row ranges of under 2 GB of codes each (one buffer
  // resource spans a launch's matrix); the fused argmax folds every range
  // into the same slots, and one finisher follows.
  const int64_t qrow = kQ4 ? cols / 2 : cols;
  const int64_t srow = (cols / kBlock) * (F != kFmtQ8 ? 2 : 4);
  const int64_t range = kMaxLaunchBytes / qrow;
  const int nt = n == 1 ? 1 : n == 2 ? 2 : 4;
  if (norm != nullptr && rows > range) return DNX_EINVAL;  // one launch writes the norm
  int slots = 0;
  for (int64_t r0 = 0; r0 < rows; r0 += range) {
    const int64_t nr = rows - r0 < range ? rows - r0 : range;
    GemvParams p{};
    p.qs[0] = (const uint8_t*)qs0 + r0 * qrow;
    p.scales[0] = (const uint8_t*)sc0 + r0 * srow;
    p.qs[1] = kPair ? (const uint8_t*)qs1 + r0 * qrow : p.qs[0];
    p.scales[1] = kPair ? (const uint8_t*)sc1 + r0 * srow : p.scales[0];
    p.x = x;
    p.y = y + r0;
    p.y2 = y2 != nullptr ? y2 + r0 : nullptr;
    p.rows = (int)nr;
    p.ldy = (int)rows;
    p.row0 = (int)r0;
    p.cols = (int)cols;
    p.n = (int)n;
    p.ws = ws;
    p.resid = resid != nullptr ? resid + r0 : nullptr;
    int rc;
    if (norm != nullptr) {
      if constexpr (!kArgmax && !kF) {
        p.norm_w = norm->w;
        p.norm_out = norm->out;
        p.norm_eps = norm->eps;
        const int R = pick_rows(kQ4, false, (int)nr, 1, kPair, (int)cols, (size_t)cols * 4);
        rc = launch_norm<F, kPair, false>(p, R, stream);
      } else {
        rc = DNX_EINVAL;
      }
      if (rc != DNX_OK) return rc;
      continue;
    }
    const int R = pick_rows(kQ4, kF, (int)nr, nt, kPair, (int)cols);
    const int W = pick_waves(kQ4, kF, (int)nr, R, nt, kPair, (int)cols);
    if (kArgmax) {
      rc = launch_nt<F, 1, false, true, false>(p, R, W, stream);
      slots = p.grid > slots ? p.grid : slots;
    } else {
      switch (nt) {
        case 1: rc = launch_nt<F, 1, kPair, false, kF>(p, R, W, stream); break;
        case 2: rc = launch_nt<F, 2, kPair, false, kF>(p, R, W, stream); break;
        default: rc = launch_nt<F, 4, kPair, false, kF>(p, R, W, stream); break;
      }
    }
    if (rc != DNX_OK) return rc;
  }
  if (kArgmax) {
    if (slots > kArgmaxSlots) slots = kArgmaxSlots;
    hipLaunchKernelGGL(argmax_finish_kernel, dim3(1), dim3(kThreads), 0, stream, ws, slots, out);
    return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
  }
  return DNX_OK;
}

// Up to kMaxSegs matrices of one format and width over the same x (one
// token): y_i = W_i x for each, in one launch that quantizes x once. Each
// matrix keeps its own pointers and rows; the results are bit-identical to
// one gemv per matrix.
template <int F>
int gemv_multi(const void* const* qs, const void* const* scales, float* const* y,
               const int64_t* rows, int segs, const float* x, int64_t cols, hipStream_t stream,
               const NormArgs* norm = nullptr) {
  if (segs < 1 || segs > kMaxSegs || cols <= 0 || cols % kBlock != 0 || cols > (1 << 20)) {
    return DNX_EINVAL;
  }
  if (norm != nullptr && !norm_ok(x, *norm, cols)) return DNX_EINVAL;
  if (qs == nullptr || scales == nullptr || y == nullptr || rows == nullptr) return DNX_EINVAL;
  if (norm != nullptr && segs == 1) {
    // One matrix: the plain launch (no per-request segment selects).
    return gemv<F, false, false>(qs[0], scales[0], nullptr, nullptr, x, y[0], nullptr, rows[0],
                                 cols, 1, nullptr, nullptr, stream, nullptr, norm);
  }
  if ((uintptr_t)x & 3) return DNX_EINVAL;
  constexpr bool kQ4 = F == kFmtQ4;
  const int64_t qrow = kQ4 ? cols / 2 : cols;
  GemvParams p{};
  int64_t total = 0;
  for (int i = 0; i < kMaxSegs; i++) {
    p.seg_rows[i] = 0;
    p.seg_qs[i] = qs[0];
    p.seg_scales[i] = scales[0];
    p.seg_y[i] = y[0];
  }
  for (int i = 0; i < segs; i++) {
    if (rows[i] <= 0 || rows[i] * qrow > kMaxLaunchBytes) return DNX_EINVAL;
    if (((uintptr_t)qs[i] & 15) || ((uintptr_t)scales[i] & (F != kFmtQ8 ? 1 : 3))) {
      return DNX_EINVAL;
    }
    if (y[i] == nullptr) return DNX_EINVAL;
    p.seg_rows[i] = (int)rows[i];
    p.seg_qs[i] = qs[i];
    p.seg_scales[i] = scales[i];
    p.seg_y[i] = y[i];
    total += rows[i];
  }
  if (total > (1 << 30)) return DNX_EINVAL;
  p.qs[0] = p.qs[1] = qs[0];
  p.scales[0] = p.scales[1] = scales[0];
  p.x = x;
  p.y = y[0];
  p.rows = (int)total;
  p.ldy = (int)total;
  p.cols = (int)cols;
  p.n = 1;
  if (norm != nullptr) {
    p.norm_w = norm->w;
    p.norm_out = norm->out;
    p.norm_eps = norm->eps;
    const int R = pick_rows(kQ4, false, (int)total, 1, false, (int)cols, (size_t)cols * 4);
    return launch_norm<F, false, true>(p, R, stream);
  }
  const int R = pick_rows(kQ4, false, (int)total, 1, false, (int)cols);
  const int W = pick_waves(kQ4, false, (int)total, R, 1, false, (int)cols);
  return launch_seg<F>(p, R, W, stream);
}

// Float inputs (mode 0), any n: launches of up to 4 tokens each.
template <int F>
int gemv_float(const void* qs, const void* scales, const float* x, float* y, int64_t rows,
               int64_t cols, int64_t n, hipStream_t stream) {
  if (n <= 0 || cols <= 0 || cols % kBlock != 0 || cols > (1 << 20)) return DNX_EINVAL;
  // Tokens per launch: 4, or fewer when their fp32 x would not fit the LDS.
  constexpr bool kQ4 = F == kFmtQ4;
  int group = 4;
  while (group > 1 &&
         lds_for(kQ4, true, 1, group, false, (int)cols, (kQ4 ? 64 : 32) + kChainPad, 4) >
             kLdsShared) {
    group /= 2;
  }
  for (int64_t t0 = 0; t0 < n; t0 += group) {
    const int64_t nt = n - t0 < group ? n - t0 : group;
    const int rc = gemv<F, false, false, true>(qs, scales, nullptr, nullptr, x + t0 * cols,
                                              y + t0 * rows, nullptr, rows, cols, nt, nullptr,
                                              nullptr, stream);
    if (rc != DNX_OK) return rc;
  }
  return DNX_OK;
}

}  // namespace

extern "C" {

int dnx_gemv_q8(const int8_t* qs, const float* scales, const float* x, float* y, int64_t rows,
                int64_t cols, int64_t n, hipStream_t stream) {
  return gemv<kFmtQ8, false, false>(qs, scales, nullptr, nullptr, x, y, nullptr, rows, cols, n,
                                   nullptr, nullptr, stream);
}

int dnx_gemv_q4(const uint8_t* qs, const uint16_t* scales, const float* x, float* y,
                int64_t rows, int64_t cols, int64_t n, hipStream_t stream) {
  return gemv<kFmtQ4, false, false>(qs, scales, nullptr, nullptr, x, y, nullptr, rows, cols, n,
                                  nullptr, nullptr, stream);
}

int dnx_gemv_q8_argmax(const int8_t* qs, const float* scales, const float* x, float* y,
                       int64_t rows, int64_t cols, int64_t* out, void* workspace,
                       hipStream_t stream) {
  return gemv<kFmtQ8, false, true>(qs, scales, nullptr, nullptr, x, y, nullptr, rows, cols, 1,
                                  (unsigned long long*)workspace, out, stream);
}

int dnx_gemv_q4_argmax(const uint8_t* qs, const uint16_t* scales, const float* x, float* y,
                       int64_t rows, int64_t cols, int64_t* out, void* workspace,
                       hipStream_t stream) {
  return gemv<kFmtQ4, false, true>(qs, scales, nullptr, nullptr, x, y, nullptr, rows, cols, 1,
                                 (unsigned long long*)workspace, out, stream);
}

int dnx_gate_up_q8(const int8_t* gate_qs, const float* gate_scales, const int8_t* up_qs,
                   const float* up_scales, const float* x, float* h, float* u, int64_t rows,
                   int64_t cols, int64_t n, hipStream_t stream) {
  return gemv<kFmtQ8, true, false>(gate_qs, gate_scales, up_qs, up_scales, x, h, u, rows, cols, n,
                                  nullptr, nullptr, stream);
}

int dnx_gate_up_q4(const uint8_t* gate_qs, const uint16_t* gate_scales, const uint8_t* up_qs,
                   const uint16_t* up_scales, const float* x, float* h, float* u, int64_t rows,
                   int64_t cols, int64_t n, hipStream_t stream) {
  return gemv<kFmtQ4, true, false>(gate_qs, gate_scales, up_qs, up_scales, x, h, u, rows, cols, n,
                                 nullptr, nullptr, stream);
}

int dnx_gemv_q8_float(const int8_t* qs, const float* scales, const float* x, float* y,
                      int64_t rows, int64_t cols, int64_t n, hipStream_t stream) {
  return gemv_float<kFmtQ8>(qs, scales, x, y, rows, cols, n, stream);
}

int dnx_gemv_q4_float(const uint8_t* qs, const uint16_t* scales, const float* x, float* y,
                      int64_t rows, int64_t cols, int64_t n, hipStream_t stream) {
  return gemv_float<kFmtQ4>(qs, scales, x, y, rows, cols, n, stream);
}

int dnx_gemv_q8h(const int8_t* qs, const uint16_t* scales, const float* x, float* y,
                 int64_t rows, int64_t cols, int64_t n, hipStream_t stream) {
  return gemv<kFmtQ8H, false, false>(qs, scales, nullptr, nullptr, x, y, nullptr, rows, cols, n,
                                     nullptr, nullptr, stream);
}

int dnx_gemv_q8h_argmax(const int8_t* qs, const uint16_t* scales, const float* x, float* y,
                        int64_t rows, int64_t cols, int64_t* out, void* workspace,
                        hipStream_t stream) {
  return gemv<kFmtQ8H, false, true>(qs, scales, nullptr, nullptr, x, y, nullptr, rows, cols, 1,
                                    (unsigned long long*)workspace, out, stream);
}

int dnx_gate_up_q8h(const int8_t* gate_qs, const uint16_t* gate_scales, const int8_t* up_qs,
                    const uint16_t* up_scales, const float* x, float* h, float* u, int64_t rows,
                    int64_t cols, int64_t n, hipStream_t stream) {
  return gemv<kFmtQ8H, true, false>(gate_qs, gate_scales, up_qs, up_scales, x, h, u, rows, cols,
                                    n, nullptr, nullptr, stream);
}

int64_t dnx_gemv_argmax_workspace_bytes(void) { return (int64_t)kArgmaxSlots * 8; }

int dnx_gemv_multi_q8(const int8_t* const* qs, const float* const* scales, float* const* y,
                      const int64_t* rows, int segs, const float* x, int64_t cols,
                      hipStream_t stream) {
  return gemv_multi<kFmtQ8>((const void* const*)qs, (const void* const*)scales, y, rows, segs,
                            x, cols, stream);
}

int dnx_gemv_multi_q4(const uint8_t* const* qs, const uint16_t* const* scales, float* const* y,
                      const int64_t* rows, int segs, const float* x, int64_t cols,
                      hipStream_t stream) {
  return gemv_multi<kFmtQ4>((const void* const*)qs, (const void* const*)scales, y, rows, segs,
                            x, cols, stream);
}

int dnx_gemv_multi_q8h(const int8_t* const* qs, const uint16_t* const* scales, float* const* y,
                       const int64_t* rows, int segs, const float* x, int64_t cols,
                       hipStream_t stream) {
  return gemv_multi<kFmtQ8H>((const void* const*)qs, (const void* const*)scales, y, rows, segs,
                             x, cols, stream);
}

int dnx_gemv_add_q8(const int8_t* qs, const float* scales, const float* x, float* y,
                    float* resid, int64_t rows, int64_t cols, hipStream_t stream) {
  if (resid == nullptr || !disjoint(resid, rows * 4, x, cols * 4) ||
      !disjoint(resid, rows * 4, y, rows * 4)) {
    return DNX_EINVAL;
  }
  return gemv<kFmtQ8, false, false>(qs, scales, nullptr, nullptr, x, y, nullptr, rows, cols, 1,
                                   nullptr, nullptr, stream, resid);
}

int dnx_gemv_add_q4(const uint8_t* qs, const uint16_t* scales, const float* x, float* y,
                    float* resid, int64_t rows, int64_t cols, hipStream_t stream) {
  if (resid == nullptr || !disjoint(resid, rows * 4, x, cols * 4) ||
      !disjoint(resid, rows * 4, y, rows * 4)) {
    return DNX_EINVAL;
  }
  return gemv<kFmtQ4, false, false>(qs, scales, nullptr, nullptr, x, y, nullptr, rows, cols, 1,
                                  nullptr, nullptr, stream, resid);
}

int dnx_gate_up_norm_q8(const int8_t* gate_qs, const float* gate_scales, const int8_t* up_qs,
                        const float* up_scales, const float* x, const float* norm_w,
                        float* norm_out, float eps, float* h, float* u, int64_t rows,
                        int64_t cols, hipStream_t stream) {
  const NormArgs nm{norm_w, norm_out, eps};
  return gemv<kFmtQ8, true, false>(gate_qs, gate_scales, up_qs, up_scales, x, h, u, rows, cols, 1,
                                  nullptr, nullptr, stream, nullptr, &nm);
}

int dnx_gate_up_norm_q4(const uint8_t* gate_qs, const uint16_t* gate_scales, const uint8_t* up_qs,
                        const uint16_t* up_scales, const float* x, const float* norm_w,
                        float* norm_out, float eps, float* h, float* u, int64_t rows,
                        int64_t cols, hipStream_t stream) {
  const NormArgs nm{norm_w, norm_out, eps};
  return gemv<kFmtQ4, true, false>(gate_qs, gate_scales, up_qs, up_scales, x, h, u, rows, cols, 1,
                                 nullptr, nullptr, stream, nullptr, &nm);
}

int dnx_gemv_multi_norm_q8(const int8_t* const* qs, const float* const* scales, float* const* y,
                           const int64_t* rows, int segs, const float* x, const float* norm_w,
                           float* norm_out, float eps, int64_t cols, hipStream_t stream) {
  const NormArgs nm{norm_w, norm_out, eps};
  return gemv_multi<kFmtQ8>((const void* const*)qs, (const void* const*)scales, y, rows, segs,
                            x, cols, stream, &nm);
}

int dnx_gemv_multi_norm_q4(const uint8_t* const* qs, const uint16_t* const* scales,
                           float* const* y, const int64_t* rows, int segs, const float* x,
                           const float* norm_w, float* norm_out, float eps, int64_t cols,
                           hipStream_t stream) {
  const NormArgs nm{norm_w, norm_out, eps};
  return gemv_multi<kFmtQ4>((const void* const*)qs, (const void* const*)scales, y, rows, segs,
                            x, cols, stream, &nm);
}

}  // extern "C"
