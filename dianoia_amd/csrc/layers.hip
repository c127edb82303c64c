// gfx950 kernels of the decoder's other layer steps, behind the reference's
// lab_gpu_enc_* encoders (lib/src/gpu.dart:179-312; semantics of the Metal
// layer, src/metal/lab_metal.m:321-579): RMSNorm, the per-head norm + RoPE,
// the gated short convolution, causal attention over a KV cache, the
// residual add and copy, and the control-vector steer. All fp32, HBM- or
// latency-bound; none is on the quantized linear layer's path.
//
// Reductions run as a wave butterfly (all lanes end with the total) and then
// a fixed-order sum of the waves' totals, so every result is deterministic.
// Their order differs from the Metal layer's SIMD-group sums, so results
// agree with it (and with the CPU oracle) to fp32 rounding, not bit for bit.
// Built with -ffp-contract=off: no multiply-add is fused unless written as
// fmaf.

#include <type_traits>

#include "common.h"
#include "f6_panel.h"
#include "dnx_kernels.h"

#include <math.h>

using namespace dnx;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

DNX_DEV float wave_sum(float v) { return wave_sum_xor(v); }


DNX_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// Sum over the workgroup: each wave's butterfly, then the waves' totals in
// wave order. `scratch` holds kWaves floats; every thread gets the total.
DNX_DEV float block_sum(float v, float* scratch) {
  v = wave_sum(v);
  __syncthreads();  // scratch may still be read from a previous call
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = scratch[0];
#pragma unroll
  for (int w = 1; w < kWaves; w++) t += scratch[w];
  return t;
}

DNX_DEV float block_max(float v, float* scratch) {
  v = wave_max(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = scratch[0];
#pragma unroll
  for (int w = 1; w < kWaves; w++) t = fmaxf(t, scratch[w]);
  return t;
}

// Row-wise RMS normalisation, semantics of lab_metal.m:327-347. Each
// workgroup owns one row: its threads stride over the row for the sum of
// squares, one block-wide reduction gives the inverse root of (mean square +
// eps), and a second pass writes w[j] * (x[j] * r) with the inner product
// rounded before the weight multiplies it. The `accumulate` flag turns the
// store into out += value, which is how a norm applied after a block feeds
// the residual stream without a separate add launch.
__global__ void __launch_bounds__(kThreads)
rms_norm_kernel(const float* __restrict__ x, const float* __restrict__ w, float* out,
                int cols, float eps, int accumulate) {
  __shared__ float scratch[kWaves];
  const float* xr = x + (size_t)blockIdx.x * cols;
  float* yr = out + (size_t)blockIdx.x * cols;
  float sum = 0.0f;
  for (int j = threadIdx.x; j < cols; j += kThreads) sum += xr[j] * xr[j];
  sum = block_sum(sum, scratch);
  const float r = 1.0f / sqrtf(sum / (float)cols + eps);
  for (int j = threadIdx.x; j < cols; j += kThreads) {
    const float v = w[j] * (xr[j] * r);
    yr[j] = accumulate ? yr[j] + v : v;
  }
}

// The same RMSNorm with a row held in registers (V float4 per thread, rows
// of up to 1024 V floats, 16-byte aligned operands): every load of x, w and
// (accumulating) out is issued at the start, so the row costs one memory
// round trip instead of a dependent walk over it. The decode step's norms
// (one row of the hidden size) are latency, not bandwidth: 6.6 -> ~3 us.
//
// kAdd: the residual add before the norm in the same pass (x += m, as
// add_kernel rounds it, stored back to x, then the norm of the new x): the
// pair dnx_add + dnx_rms_norm in one launch.
// kPanel: also the fp6 GEMMs' activation panel of the normed rows (for the
// prefill matmuls that read them), as dnx_quantize_q8_f6panel would make it
// from out: the row goes through LDS (cols floats, dynamic) to four lanes
// per 32-value block (panel4_lane); row blockIdx.x is token blockIdx.x.
template <int V, bool kAdd = false, bool kPanel = false>
__global__ void __launch_bounds__(kThreads)
rms_norm_vec_kernel(const float* x_in, const float* __restrict__ w, float* out, int cols,
                    float eps, int accumulate, const float* __restrict__ m, float* x_out,
                    uint8_t* __restrict__ panel) {
  __shared__ float scratch[kWaves];
  const int q = cols / 4;
  const float4* xr = (const float4*)(x_in + (size_t)blockIdx.x * cols);
  const float4* mr = (const float4*)(m + (size_t)blockIdx.x * cols);
  float4* xw = (float4*)(x_out + (size_t)blockIdx.x * cols);
  const float4* wr = (const float4*)w;
  float4* yr = (float4*)(out + (size_t)blockIdx.x * cols);
  float4 xv[V], wv[V], ov[V], mv[V];
  const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int e = 0; e < V; e++) {
    const int i = e * kThreads + threadIdx.x;
    const bool ok = i < q;
    xv[e] = ok ? xr[i] : z;
    wv[e] = ok ? wr[i] : z;
    ov[e] = (ok && accumulate) ? yr[i] : z;
    mv[e] = (ok && kAdd) ? mr[i] : z;
  }
  if (kAdd) {
#pragma unroll
    for (int e = 0; e < V; e++) {
      const int i = e * kThreads + threadIdx.x;
      xv[e].x = xv[e].x + mv[e].x;
      xv[e].y = xv[e].y + mv[e].y;
      xv[e].z = xv[e].z + mv[e].z;
      xv[e].w = xv[e].w + mv[e].w;
      if (i < q) xw[i] = xv[e];
    }
  }
  float sum = 0.0f;
#pragma unroll
  for (int e = 0; e < V; e++) {
    sum += xv[e].x * xv[e].x;
    sum += xv[e].y * xv[e].y;
    sum += xv[e].z * xv[e].z;
    sum += xv[e].w * xv[e].w;
  }
  sum = norm_row_sum(sum, scratch);
  const float r = 1.0f / sqrtf(sum / (float)cols + eps);
#pragma unroll
  for (int e = 0; e < V; e++) {
    const int i = e * kThreads + threadIdx.x;
    if (i >= q) break;
    float4 v;
    v.x = wv[e].x * (xv[e].x * r);
    v.y = wv[e].y * (xv[e].y * r);
    v.z = wv[e].z * (xv[e].z * r);
    v.w = wv[e].w * (xv[e].w * r);
    if (accumulate) {
      v.x = ov[e].x + v.x;
      v.y = ov[e].y + v.y;
      v.z = ov[e].z + v.z;
      v.w = ov[e].w + v.w;
    }
    yr[i] = v;
    if constexpr (kPanel) {
      extern __shared__ float4 row_lds[];
      row_lds[i] = v;
    }
  }
  if constexpr (kPanel) {
    extern __shared__ float4 row_lds[];
    __syncthreads();
    const int B = cols / kBlock;
    const int tok = blockIdx.x, r = tok % kTokens;
    uint8_t* recs = panel + (size_t)(tok / kTokens) * B * kRec;
    // Whole quads of lanes (kThreads and 4 B are multiples of 4): the quad
    // reductions inside panel4_lane see their four lanes.
    for (int idx = threadIdx.x; idx < 4 * B; idx += kThreads) {
      const int j = idx & 3, b = idx >> 2;
      const float4 v0 = row_lds[b * 8 + 2 * j], v1 = row_lds[b * 8 + 2 * j + 1];
      panel4_lane(v0, v1, j, r, recs + (size_t)b * kRec);
    }
  }
}

// Per (head, token), one wave (lab_metal.m:357-380): RMSNorm over head_dim
// with weight w, then the half-split RoPE rotation pairing j with
// j + hd / 2, from the token's tables [cos(hd / 2), sin(hd / 2)]. In place;
// each lane reads its pairs before the reduction and writes only them.
//
// Two operands may share a launch (a decode step's q and k heads, one rope
// table): workgroups with blockIdx.x below heads0 take (x, x_stride, w) and
// the rest (xb, xb_stride, wb), head blockIdx.x - heads0.
// One head's RMSNorm over hd with weight w, then the half-split RoPE
// rotation pairing j with j + hd / 2 from the table row [cos(hd / 2),
// sin(hd / 2)], by one wave (lane j holds the pairs j + 64 e, e < P):
// rope_row_load requests a lane's operands, rope_row_finish computes and
// writes dst (which may be src: every lane reads its pairs before it writes
// them). Shared by head_norm_rope_kernel and the attention that folds it in,
// so both give the same bits (pairs past hd / 2 would only add +0 to the
// sum, so any P covering hd / 2 gives the same result).
template <int P>
struct RopeRow {
  float x1[P], x2[P], w1[P], w2[P], c[P], s[P];
};

template <int P>
DNX_DEV RopeRow<P> rope_row_load(const float* src, const float* __restrict__ w,
                                 const float* __restrict__ table, int hd, int lane) {
  const int pair = hd / 2;
  RopeRow<P> r;
#pragma unroll
  for (int e = 0; e < P; e++) {
    const int j = lane + 64 * e;
    const bool ok = j < pair;
    r.x1[e] = ok ? src[j] : 0.0f;
    r.x2[e] = ok ? src[j + pair] : 0.0f;
    r.w1[e] = ok ? w[j] : 0.0f;
    r.w2[e] = ok ? w[j + pair] : 0.0f;
    r.c[e] = ok ? table[j] : 0.0f;
    r.s[e] = ok ? table[pair + j] : 0.0f;
  }
  return r;
}

template <int P>
DNX_DEV void rope_row_finish(const RopeRow<P>& r, int hd, float eps, float* dst, int lane) {
  const int pair = hd / 2;
  float sum = 0.0f;
#pragma unroll
  for (int e = 0; e < P; e++) sum += r.x1[e] * r.x1[e] + r.x2[e] * r.x2[e];
  sum = wave_sum(sum);
  const float rr = 1.0f / sqrtf(sum / (float)hd + eps);
#pragma unroll
  for (int e = 0; e < P; e++) {
    const int j = lane + 64 * e;
    if (j >= pair) break;
    const float n1 = r.w1[e] * (r.x1[e] * rr), n2 = r.w2[e] * (r.x2[e] * rr);
    dst[j] = n1 * r.c[e] - n2 * r.s[e];
    dst[j + pair] = n2 * r.c[e] + n1 * r.s[e];
  }
}

DNX_DEV void head_norm_rope_row(float* x, const float* __restrict__ w,
                                const float* __restrict__ table, int hd, float eps, int lane) {
  constexpr int kPairs = 4;  // hd <= 512
  rope_row_finish<kPairs>(rope_row_load<kPairs>(x, w, table, hd, lane), hd, eps, x, lane);
}

__global__ void __launch_bounds__(64)
head_norm_rope_kernel(float* x, int x_stride, const float* __restrict__ w,
                      const float* __restrict__ rope, int rope_stride, int hd, float eps,
                      int heads0, float* xb, int xb_stride, const float* __restrict__ wb) {
  const int lane = threadIdx.x;
  const bool second = (int)blockIdx.x >= heads0;
  if (second) {
    x = xb;
    x_stride = xb_stride;
    w = wb;
  }
  const int head = second ? (int)blockIdx.x - heads0 : (int)blockIdx.x;
  float* xh = x + (size_t)blockIdx.y * x_stride + (size_t)head * hd;
  const float* table = rope + (size_t)blockIdx.y * rope_stride;
  head_norm_rope_row(xh, w, table, hd, eps, lane);
}

constexpr int kMaxConvK = 16;
constexpr int kConvCh = 64;   // channels per workgroup (one wave's lanes)
constexpr int kConvT = 16;    // tokens per workgroup tile (>= kMaxConvK - 1)

// Gated short convolution (LFM2's conv block; semantics of lab_metal.m:383-412),
// token-parallel. Per channel c the input sequence is z_j = B_j[c] * X_j[c]
// for tokens j >= 0, and the carried state for j < 0: history row k - 1 + j
// (rows oldest first). Output y_t[c] = C_t[c] * a_t with
//   a_t = w[k-1] z_t + w[k-2] z_{t-1} + ... + w[0] z_{t-k+1},
// each product rounded, summed left to right from the newest term. Afterwards
// history row r holds z_{n-k+1+r}.
//
// Workgroup (slab, tile) owns kConvCh consecutive channels and kConvT
// consecutive tokens. It stages z for its tokens and the k - 1 before them in
// LDS (one product per value, coalesced along channels), then each thread
// forms whole outputs from the staged window: no token waits on another.
// Only tile 0 reaches back into the carried state, so tile 0 alone rewrites
// it: every old row it needs is already in its LDS copy, and no other
// workgroup reads the state, so the in-place update cannot race.
__global__ void __launch_bounds__(kThreads)
conv_kernel(const float* __restrict__ bcx, const float* __restrict__ weight, float* history,
            float* __restrict__ y, int width, int k, int n) {
  __shared__ float zs[kConvT + kMaxConvK - 1][kConvCh];
  const int lane = threadIdx.x % kConvCh, part = threadIdx.x / kConvCh;
  constexpr int kParts = kThreads / kConvCh;
  const int c = blockIdx.x * kConvCh + lane;
  const bool live = c < width;
  const int t0 = blockIdx.y * kConvT;
  const int tn = min(kConvT, n - t0);
  const int span = tn + k - 1;  // staged rows: tokens t0 - (k - 1) .. t0 + tn - 1
  const size_t row3 = (size_t)3 * width;

  constexpr int kStageIters = (kConvT + kMaxConvK - 1 + kParts - 1) / kParts;
#pragma unroll
  for (int m = 0; m < kStageIters; m++) {  // all loads of a thread in flight together
    const int i = part + m * kParts;
    if (i < span) {
      const int j = t0 - (k - 1) + i;
      float z = 0.0f;
      if (live) {
        z = j >= 0 ? bcx[(size_t)j * row3 + c] * bcx[(size_t)j * row3 + 2 * (size_t)width + c]
                   : history[(size_t)(k - 1 + j) * width + c];
      }
      zs[i][lane] = z;
    }
  }
  __syncthreads();
  if (!live) return;

  // Taps by lag: wl[s] weights z_{t-s} (register indices stay constant).
  float wl[kMaxConvK];
#pragma unroll
  for (int s = 0; s < kMaxConvK; s++) wl[s] = s < k ? weight[(size_t)c * k + (k - 1 - s)] : 0.0f;
#pragma unroll
  for (int m = 0; m < kConvT / kParts; m++) {
    const int i = part + m * kParts;
    if (i >= tn) break;
    const int t = t0 + i;
    // Row of z_t in the staged window is i + k - 1; z_{t-s} sits s rows up.
    float a = wl[0] * zs[i + k - 1][lane];
#pragma unroll
    for (int s = 1; s < kMaxConvK; s++) {
      if (s < k) a += wl[s] * zs[i + k - 1 - s][lane];
    }
    y[(size_t)t * width + c] = bcx[(size_t)t * row3 + width + c] * a;
  }

  if (blockIdx.y == 0) {
    // New state row r = z_{n-k+1+r}: from the staged window when that token
    // is in it (or is an old state row), else a product of the last tokens.
    for (int r = part; r + 1 < k; r += kParts) {
      const int j = n - (k - 1) + r;
      float z;
      if (j < tn) {
        z = zs[j + k - 1][lane];
      } else {
        z = bcx[(size_t)j * row3 + c] * bcx[(size_t)j * row3 + 2 * (size_t)width + c];
      }
      history[(size_t)r * width + c] = z;
    }
  }
}

// Causal attention of n tokens at positions position.. over their cached
// keys and values (lab_metal.m:414-521), one workgroup per (head, token):
// scores q.k / sqrt(hd) against the keys the token may see (window 0:
// every earlier position; else the last `window`, its own included), a
// softmax, the weighted sum of values, and the per-head output gate
// sigmoid(gate) when `gate` is not null. GQA: query head h reads KV head
// h / (heads / kv_heads). Scores live in LDS (dynamic, sized by the launch
// for the last token's keys). Each thread takes whole keys for the dots
// (one key row per lane: 16-byte loads), and the value sum splits the keys
// over 256 / hd thread groups added in group order.
__global__ void __launch_bounds__(kThreads)
attention_kernel(const float* __restrict__ q, const float* __restrict__ keys,
                 const float* __restrict__ values, const float* __restrict__ gate,
                 float* __restrict__ out, int position, int heads, int kv_dim, int group,
                 int hd, int window, float scale) {
  extern __shared__ __align__(16) float lds[];
  __shared__ float scratch[kWaves];
  const int head = blockIdx.x, token = blockIdx.y, tid = threadIdx.x;
  const int pos = position + token;
  const int start = window > 0 && pos >= window ? pos - window + 1 : 0;
  const int count = pos - start + 1;
  const size_t qo = ((size_t)token * heads + head) * hd;
  const int kvo = head / group * hd;
  float* qs = lds;                      // [hd]
  float* scores = lds + hd;             // [count]
  float* part = scores + ((count + 3) & ~3);   // [groups][hd] value partials
  for (int d = tid; d < hd; d += kThreads) qs[d] = q[qo + d];
  __syncthreads();

  const int hd4 = hd / 4;
  for (int i = tid; i < count; i += kThreads) {
    const float4* k4 = (const float4*)(keys + (size_t)(start + i) * kv_dim + kvo);
    float d = 0.0f;
    for (int c = 0; c < hd4; c++) {
      const float4 kc = k4[c];
      const float4 qc = *(const float4*)(qs + 4 * c);
      d += qc.x * kc.x + qc.y * kc.y + qc.z * kc.z + qc.w * kc.w;
    }
    scores[i] = d * scale;
  }
  __syncthreads();
  float m = -INFINITY;
  for (int i = tid; i < count; i += kThreads) m = fmaxf(m, scores[i]);
  m = block_max(m, scratch);
  float sum = 0.0f;
  for (int i = tid; i < count; i += kThreads) {
    const float e = expf(scores[i] - m);
    scores[i] = e;
    sum += e;
  }
  sum = block_sum(sum, scratch);  // its barriers also publish the exponentials
  const int groups = kThreads / hd;  // >= 1: hd <= 256
  const int gi = tid / hd, d = tid - gi * hd;
  if (gi < groups) {
    const float* v = values + (size_t)start * kv_dim + kvo + d;
    float acc = 0.0f;
    int i = gi;
    for (; i + 3 * groups < count; i += 4 * groups) {  // 4 keys' loads together
      const float v0 = v[(size_t)i * kv_dim], v1 = v[(size_t)(i + groups) * kv_dim];
      const float v2 = v[(size_t)(i + 2 * groups) * kv_dim];
      const float v3 = v[(size_t)(i + 3 * groups) * kv_dim];
      acc += scores[i] * v0;
      acc += scores[i + groups] * v1;
      acc += scores[i + 2 * groups] * v2;
      acc += scores[i + 3 * groups] * v3;
    }
    for (; i < count; i += groups) acc += scores[i] * v[(size_t)i * kv_dim];
    part[gi * hd + d] = acc;
  }
  __syncthreads();
  if (gi == 0) {
    float acc = part[d];
    for (int g2 = 1; g2 < groups; g2++) acc += part[g2 * hd + d];
    if (gate != nullptr) {
      const float g = 1.0f / (1.0f + expf(-gate[(size_t)token * heads + head]));
      out[qo + d] = (acc / sum) * g;
    } else {
      out[qo + d] = acc / sum;
    }
  }
}

// Long contexts with few (head, token) pairs (decode) split the keys: each
// workgroup of attention_split_kernel takes split_keys(hd) keys of one
// token for G query heads that share one KV head, and writes for each head
// its max m, its exponentials' sum l (relative to m) and its unnormalised
// value sums o[hd] (a row of hd + 4 floats: m, l, two unused, o, so o is
// 16-byte aligned); attention_combine_kernel rescales the splits to their
// common max and adds them in split order (deterministic):
// O = sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M). The same softmax as
// attention_kernel, summed in another order.
// A split puts hd / 4 lanes on a key row (one 16-byte piece each,
// coalesced), 256 / (hd / 4) keys per workgroup step, and kSplitSteps
// steps: every key and value load of the split is issued at its start, so
// it waits for memory once, and each row is read once for the G heads
// (GQA). Eight steps (64 keys at hd 128: 512 workgroups at 4096 positions
// of 8 KV heads) read faster than 16 with half the workgroups (Qwen3-1.7B
// at position 4095: 9.0 against 11.0 us; a pure read of the same bytes in
// the two patterns: 7.2 against 8.1-9.5 us).
// Dots end in a butterfly over the key's lanes; wave w takes the softmax
// statistics of heads w, w + 4, ...; value sums go to per-lane float4
// partials added in a fixed order.
constexpr int kSplitSteps = 8;
constexpr int kSplitMaxKeys = 256;

int split_keys(int hd) {
  const int step = kThreads / (hd / 4);   // keys per workgroup step
  const int k = kSplitSteps * step;
  return k < kSplitMaxKeys ? k : kSplitMaxKeys;
}

// Sum over aligned groups of LT lanes (a power of two up to 32); every lane
// of a group gets the group's sum. DPP moves up to 16 lanes (no LDS round
// trip), a swizzle for 32.
template <int LT>
DNX_DEV float group_sum(float v) {
  if constexpr (LT >= 2) v += dppf<kQuadXor1>(v);
  if constexpr (LT >= 4) v += dppf<kQuadXor2>(v);
  if constexpr (LT >= 8) v += dppf<kHalfRowMirror>(v);
  if constexpr (LT >= 16) v += dppf<kRowMirror>(v);
  if constexpr (LT >= 32) v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
  static_assert(LT <= 32, "group_sum: at most 32 lanes");
  return v;
}

// G query heads per workgroup; LT lanes per key when fixed at compile time
// (hd = 4 * LT), 0 for any hd.
// The q and k head norms + RoPE of a decode step folded into its attention
// (one token): the table row of the token, the two norm weights, eps, and
// the cache's keys (written: the new key row, normed in place).
struct RopeArgs {
  const float* table;
  const float* qw;
  const float* kw;
  float* keys;
  float eps;
};
constexpr int kRopeMaxHd = 256;

template <int G, int LT, int STEPS = kSplitSteps, bool kRope = false>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 2)))
attention_split_kernel(const float* __restrict__ q, const float* keys,
                       const float* __restrict__ values, float* __restrict__ ws, int position,
                       int heads, int kv_dim, int group, int hd, int window, float scale,
                       int splits, int keys_per_split, RopeArgs rp) {
  __shared__ float scores[G][kSplitMaxKeys];
  __shared__ float4 part[G][kThreads];
  __shared__ float stat[G][2];
  const int h0 = blockIdx.x * G, token = blockIdx.y, split = blockIdx.z, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int pos = position + token;
  const int start = window > 0 && pos >= window ? pos - window + 1 : 0;
  const int count = pos - start + 1;
  const int k0 = split * keys_per_split;
  const int nk = max(0, min(keys_per_split, count - k0));   // this split's keys
  const int kvo = h0 / group * hd;
  const int L = LT > 0 ? LT : hd / 4;                      // lanes per key
  const int per = 64 / L, step = kWaves * per;               // keys per wave, per step
  const int c = lane % L, kb = wave * per + lane / L;       // this lane's first key
  float4 qr[G];
  if constexpr (!kRope) {
#pragma unroll
    for (int g = 0; g < G; g++)
      qr[g] = *(const float4*)(q + ((size_t)token * heads + h0 + g) * hd + 4 * c);
  }
  // Resources over this split's nk key rows: a row past them lies wholly
  // beyond the range (its offset is at least nk rows) and reads zeros.
  const size_t first = (size_t)(start + k0) * kv_dim + kvo;
  const uint32_t range = (uint32_t)nk * (uint32_t)kv_dim * 4u;
  const i32x4 krs = buffer_rsrc(keys + first, range);
  const i32x4 vrs = buffer_rsrc(values + first, range);
  const float4 zero = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  // Folded head norms (one token): wave w norms and rotates q heads h0 + w,
  // h0 + w + 4, ..., and in the split that holds the token's own key, the
  // wave after the last q head its key row (as stored). Their operands are
  // requested before the keys and values, which return in order after them.
  const int cur = count - 1 - k0;                // the token's key within the split
  const bool has_cur = kRope && cur >= 0 && cur < nk;
  constexpr int kRP = kRopeMaxHd / 128;          // pairs per lane
  constexpr int kRows = kRope ? (G + kWaves) / kWaves : 1;
  RopeRow<kRP> rrow[kRows];
  float dcur[G];  // the token's own key's dots (folded norms)
  if constexpr (kRope) {
#pragma unroll
    for (int r = 0; r < kRows; r++) {
      // Rows a wave does not norm load q's first head (always valid), unused.
      const int g = wave + r * kWaves;
      const bool is_k = g == G && has_cur;
      const float* src = g < G ? q + ((size_t)h0 + g) * hd
                         : is_k ? keys + (size_t)pos * kv_dim + kvo : q + (size_t)h0 * hd;
      rrow[r] = rope_row_load<kRP>(src, is_k ? rp.kw : rp.qw, rp.table, hd, lane);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  float4 kv[STEPS], vv[STEPS];
#pragma unroll
  for (int j = 0; j < STEPS; j++)
    kv[j] = buffer_load_f4(krs, (kb + j * step) * kv_dim * 4 + 16 * c);
#pragma unroll
  for (int j = 0; j < STEPS; j++)
    vv[j] = buffer_load_f4(vrs, (kb + j * step) * kv_dim * 4 + 16 * c);
  // The folded norms' results go through LDS to the lanes that need them;
  // the keys and values are in flight meanwhile.
  if constexpr (kRope) {
    __shared__ float qn[G][kRopeMaxHd];
    __shared__ float kn[kRopeMaxHd];
#pragma unroll
    for (int r = 0; r < kRows; r++) {
      const int g = wave + r * kWaves;
      if (g < G) {
        rope_row_finish<kRP>(rrow[r], hd, rp.eps, qn[g], lane);
      } else if (g == G && has_cur) {
        rope_row_finish<kRP>(rrow[r], hd, rp.eps, kn, lane);
      }
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; g++) qr[g] = *(const float4*)(qn[g] + 4 * c);
    if (has_cur) {
      // The token's own key scores against its normed row (every key group
      // holds all dims, so every lane computes the same dot, reduced as the
      // other keys' dots are); its loaded copy is not used.
      const float4 k4 = *(const float4*)(kn + 4 * c);
#pragma unroll
      for (int g = 0; g < G; g++) {
        float d = qr[g].x * k4.x + qr[g].y * k4.y + qr[g].z * k4.z + qr[g].w * k4.w;
        if constexpr (LT > 0) {
          d = group_sum<LT>(d);
        } else {
          for (int o = L / 2; o > 0; o >>= 1) d += __shfl_xor(d, o);
        }
        dcur[g] = d;
      }
      // The normed key row back into the cache (only this workgroup reads it).
      if (tid < hd / 4) {
        *(float4*)(rp.keys + (size_t)pos * kv_dim + kvo + 4 * tid) = *(const float4*)(kn + 4 * tid);
      }
    }
  }
  // Dots in batches of kBatch steps x G heads: each butterfly stage issues
  // the batch's lane exchanges together and waits once (L is a run-time
  // count, so per-dot loops would wait on every exchange).
  constexpr int kBatch = 4;
#pragma unroll
  for (int j0 = 0; j0 < STEPS; j0 += kBatch) {
    float d[kBatch][G];
#pragma unroll
    for (int u = 0; u < kBatch; u++)
#pragma unroll
      for (int g = 0; g < G; g++) {
        const float4 k4 = kv[j0 + u];
        d[u][g] = qr[g].x * k4.x + qr[g].y * k4.y + qr[g].z * k4.z + qr[g].w * k4.w;
      }
    if constexpr (LT > 0) {
#pragma unroll
      for (int u = 0; u < kBatch; u++)
#pragma unroll
        for (int g = 0; g < G; g++) d[u][g] = group_sum<LT>(d[u][g]);
    } else {
      for (int o = L / 2; o > 0; o >>= 1) {
#pragma unroll
        for (int u = 0; u < kBatch; u++)
#pragma unroll
          for (int g = 0; g < G; g++) d[u][g] += __shfl_xor(d[u][g], o);
      }
    }
#pragma unroll
    for (int u = 0; u < kBatch; u++) {
      const int i = kb + (j0 + u) * step;
      if (i < nk && c == 0) {
#pragma unroll
        for (int g = 0; g < G; g++) scores[g][i] = (has_cur && i == cur ? dcur[g] : d[u][g]) * scale;
      }
    }
  }
  __syncthreads();
  for (int g = wave; g < G; g += kWaves) {  // one wave per head: no block barrier
    constexpr int kPerLane = kSplitMaxKeys / 64;
    float v[kPerLane];
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < kPerLane; u++) {
      const int i = u * 64 + lane;
      v[u] = i < nk ? scores[g][i] : -INFINITY;
      mx = fmaxf(mx, v[u]);
    }
    mx = wave_max_dpp(mx);
    float sum = 0.0f;
#pragma unroll
    for (int u = 0; u < kPerLane; u++) {
      const int i = u * 64 + lane;
      if (i < nk) {
        const float e = expf(v[u] - mx);
        scores[g][i] = e;
        sum += e;
      }
    }
    sum = wave_sum_dpp(sum);
    if (lane == 0) {
      stat[g][0] = mx;   // -inf for a split past the token's keys (l = 0, o = 0)
      stat[g][1] = sum;
    }
  }
  __syncthreads();
  float4 acc[G];
#pragma unroll
  for (int g = 0; g < G; g++) acc[g] = zero;
#pragma unroll
  for (int j = 0; j < STEPS; j++) {
    const int i = kb + j * step;
#pragma unroll
    for (int g = 0; g < G; g++) {
      const float p = i < nk ? scores[g][i] : 0.0f;
      acc[g].x += p * vv[j].x;
      acc[g].y += p * vv[j].y;
      acc[g].z += p * vv[j].z;
      acc[g].w += p * vv[j].w;
    }
  }
#pragma unroll
  for (int g = 0; g < G; g++) part[g][tid] = acc[g];
  __syncthreads();
  for (int e = tid; e < G * L; e += kThreads) {
    // Head g, dimensions 4cc..4cc+3: the (wave, key-in-step) partials in order.
    const int g = e / L, cc = e - g * L;
    float4 t = zero;
    for (int w = 0; w < kWaves; w++)
      for (int s2 = 0; s2 < per; s2++) {
        const float4 p4 = part[g][w * 64 + s2 * L + cc];
        t.x += p4.x;
        t.y += p4.y;
        t.z += p4.z;
        t.w += p4.w;
      }
    float* out = ws + (((size_t)token * heads + h0 + g) * splits + split) * (hd + 4);
    *(float4*)(out + 4 + 4 * cc) = t;
    if (cc == 0) {
      out[0] = stat[g][0];
      out[1] = stat[g][1];
    }
  }
}

template <int G, bool kRope = false>
void launch_split(dim3 grid, hipStream_t stream, const float* q, const float* keys,
                  const float* values, float* ws, int position, int heads, int kv_dim, int group,
                  int hd, int window, float scale, int splits, int kps, RopeArgs rp = {}) {
  auto kernel = hd == 128 ? attention_split_kernel<G, 32, kSplitSteps, kRope>
              : hd == 64  ? attention_split_kernel<G, 16, kSplitSteps, kRope>
                          : attention_split_kernel<G, 0, kSplitSteps, kRope>;
  hipLaunchKernelGGL(kernel, grid, dim3(kThreads), 0, stream, q, keys, values, ws, position,
                     heads, kv_dim, group, hd, window, scale, splits, kps, rp);
}

// The splits of one (head, token). Thread t takes dimension t % hd of the
// splits s = t / hd + P j (P = 256 / hd threads per dimension). Its first
// kChunk value loads and the split statistics are issued together, so a
// short context waits for memory once; the rescaling factors e^(m_s - M)
// go through LDS (dynamic: `splits` floats), and the P partial sums of a
// dimension are added in a fixed order.
// More than 64 splits: each thread takes splits s0, s0 + 256, ...; the max
// and l over the workgroup (the block reductions' barriers also publish fs).
DNX_DEV float combine_stats(const float* w, int splits, int row, int s0, float m0, float l0,
                            float* fs, float* scratch) {
  float mx = s0 < splits ? m0 : -INFINITY;
  for (int s = s0 + kThreads; s < splits; s += kThreads) mx = fmaxf(mx, w[(size_t)s * row]);
  mx = block_max(mx, scratch);
  float lp = 0.0f;
  if (s0 < splits) {
    const float f = m0 != -INFINITY ? expf(m0 - mx) : 0.0f;
    fs[s0] = f;
    lp = l0 * f;
  }
  for (int s = s0 + kThreads; s < splits; s += kThreads) {
    const float ms = w[(size_t)s * row];
    const float f = ms != -INFINITY ? expf(ms - mx) : 0.0f;
    fs[s] = f;
    lp += w[(size_t)s * row + 1] * f;
  }
  return block_sum(lp, scratch);
}

template <bool kRope = false>
__global__ void __launch_bounds__(kThreads)
attention_combine_kernel(const float* __restrict__ ws, const float* __restrict__ gate,
                         float* __restrict__ out, int heads, int hd, int splits,
                         float* qio = nullptr, RopeArgs rp = {}) {
  extern __shared__ float fs[];   // [splits] e^(m_s - M), 0 for empty splits
  __shared__ float scratch[kWaves];
  __shared__ float red[kThreads];
  constexpr int kChunk = 32;
  const int head = blockIdx.x, token = blockIdx.y, tid = threadIdx.x;
  const int row = hd + 4;
  const float* w = ws + ((size_t)token * heads + head) * splits * row;
  // Every offset past the (head, token)'s rows reads zero.
  const i32x4 rs = buffer_rsrc(w, (uint32_t)splits * (uint32_t)row * 4u);
  const int P = kThreads / hd, d = tid % hd, part = tid / hd;
  float v[kChunk];
#pragma unroll
  for (int u = 0; u < kChunk; u++) {
    const int sp = part + u * P;
    v[u] = __int_as_float(dnx_raw_buffer_load_i32(rs, (sp * row + 4 + d) * 4, 0, 0));
  }
  const int s0 = tid;   // the first split whose statistics this thread reads
  const float m0 = __int_as_float(dnx_raw_buffer_load_i32(rs, s0 * row * 4, 0, 0));
  const float l0 = __int_as_float(dnx_raw_buffer_load_i32(rs, (s0 * row + 1) * 4, 0, 0));
  if constexpr (kRope) {
    // The folded q norm of this head, in place (one token): the split
    // kernel normed its own copies; every split has finished reading q.
    // Wave 1, while wave 0 reduces the split statistics.
    if (tid >= 64 && tid < 128) {
      head_norm_rope_row(qio + (size_t)head * hd, rp.qw, rp.table, hd, rp.eps, tid - 64);
    }
  }
  float l;
  if (splits <= 64) {
    // One wave holds every split's statistics (lane s): the max, the
    // factors and l without a block reduction; one barrier publishes them.
    if (tid < 64) {
      const bool live = s0 < splits;
      const float m = live ? m0 : -INFINITY;
      const float mx = wave_max_dpp(m);
      const float f = live && m != -INFINITY ? expf(m - mx) : 0.0f;
      if (live) fs[s0] = f;
      const float lsum = wave_sum_dpp(live ? l0 * f : 0.0f);
      if (tid == 0) scratch[0] = lsum;
    }
    __syncthreads();
    l = scratch[0];
  } else {
    l = combine_stats(w, splits, row, s0, m0, l0, fs, scratch);
  }
  float acc = 0.0f;
#pragma unroll
  for (int u = 0; u < kChunk; u++) {
    const int sp = part + u * P;
    if (sp < splits) acc += v[u] * fs[sp];
  }
  for (int sp = part + kChunk * P; sp < splits; sp += P) acc += w[(size_t)sp * row + 4 + d] * fs[sp];
  red[tid] = acc;
  __syncthreads();
  if (part == 0) {
    float t = red[d];
    for (int p2 = 1; p2 < P; p2++) t += red[p2 * hd + d];
    const size_t qo = ((size_t)token * heads + head) * hd;
    const float g =
        gate != nullptr ? 1.0f / (1.0f + expf(-gate[(size_t)token * heads + head])) : 1.0f;
    out[qo + d] = gate != nullptr ? (t / l) * g : t / l;
  }
}

// Attention of many tokens (prefill) on the fp32 matrix cores. A wave
// takes 16 queries of one head, a workgroup 4 waves sharing one KV head
// (GW heads of a GQA group x 4 / GW query blocks), and the workgroup walks
// its keys in tiles of 32 staged in LDS (K row-major, V transposed), so a
// tile is read once for up to 64 queries. Per tile and wave:
// * S^T = K Q^T on v_mfma_f32_16x16x4f32: A = 16 keys x 4 dims (K from LDS,
//   dims g * hd / 4 + s for lane group g), B = 4 dims x 16 queries (Q held
//   in registers); a lane ends with 8 scores of its query (column), so the
//   online softmax needs two cross-lane exchanges per tile;
// * O^T += V^T P^T: the lane's exponentials are already the B operand of
//   step s (keys (s / 4) * 16 + 4 g + s % 4), V^T tiles come from LDS.
// The running (max, sum) rescale O when the max grows (flash attention).
// With `splits` > 1 a workgroup takes a run of tiles_per_split tiles and
// writes per (token, head) the partial (m, l, o) rows that
// attention_combine_kernel adds (for long contexts with few query blocks);
// otherwise it writes the output, gated. fp32 throughout: the sums run in
// another order than the oracle's, and the softmax exponentials use the
// hardware exp2 (__expf, a few ulp) instead of expf.
constexpr int kPQ = 16;   // queries per wave
constexpr int kPK = 32;   // keys per tile

typedef float v4f __attribute__((ext_vector_type(4)));

// Max / sum over lanes i, i ^ 16, i ^ 32 and i ^ 48 (lane i % 16 of the four
// 16-lane rows), every lane getting the result, on gfx950's VALU lane swaps:
// with both operands v, permlane16_swap pairs each lane with lane ^ 16 and
// permlane32_swap with lane ^ 32. No LDS round trip.
DNX_DEV float rows4_max(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

DNX_DEV float rows4_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

template <int HD, int GW>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 2)))
attention_prefill_kernel(const float* __restrict__ q, const float* __restrict__ keys,
                         const float* __restrict__ values, const float* __restrict__ gate,
                         float* __restrict__ out, float* __restrict__ ws, int position, int n,
                         int heads, int kv_dim, int group, int window, float scale, int splits,
                         int tiles_per_split) {
  constexpr int QW = 4 / GW;
  constexpr int KS = HD + 4;                     // K row stride in LDS (floats)
  constexpr int VS = kPK + 4;                    // V^T row stride
  constexpr int kF4 = HD * kPK / 4 / kThreads;   // float4 per thread per tile and matrix
  constexpr int kLds = kPK * KS + HD * VS;
  static_assert(kLds >= 4 * kPQ * (HD + 4), "the output transpose reuses the tiles' LDS");
  __shared__ __align__(16) float lds[kLds];
  float* Ks = lds;
  float* Vt = lds + kPK * KS;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c16 = lane & 15, g4 = lane >> 4;
  const int head = blockIdx.x * GW + wave % GW;
  const int split = blockIdx.z;
  // Odd splits take the query blocks in reverse: workgroups dispatched
  // together then pair a late block's long key runs with an early block's
  // short ones (causal work grows with the block).
  const int yb = split & 1 ? gridDim.y - 1 - blockIdx.y : blockIdx.y;
  const int t0 = (yb * QW + wave / GW) * kPQ;   // the wave's first token
  // The workgroup's keys: from its first query's window start through its
  // last query.
  const int wq_first = yb * QW * kPQ;
  const int wq_last = min(n, wq_first + QW * kPQ) - 1;
  const int kend = position + wq_last + 1;
  const int kstart = window > 0 ? max(0, position + wq_first - window + 1) : 0;
  const int ntiles = (kend - kstart + kPK - 1) / kPK;
  const int tile_lo = split * tiles_per_split;
  const int tile_hi = min(ntiles, tile_lo + tiles_per_split);
  const size_t kvo = (size_t)(blockIdx.x * GW / group) * HD;

  // B operand of S^T: the lane's query, dims g4 * HD / 4 + s.
  const int tq = t0 + c16;
  const int qpos = position + tq;
  float qr[HD / 4];
  {
    const float* qp = q + ((size_t)min(tq, n - 1) * heads + head) * HD + g4 * (HD / 4);
#pragma unroll
    for (int s4 = 0; s4 < HD / 16; s4++) {
      const float4 v = *(const float4*)(qp + 4 * s4);
      qr[4 * s4] = v.x;
      qr[4 * s4 + 1] = v.y;
      qr[4 * s4 + 2] = v.z;
      qr[4 * s4 + 3] = v.w;
    }
  }
  float m_run = -INFINITY, l_run = 0.0f;
  v4f o[HD / 16];
#pragma unroll
  for (int e = 0; e < HD / 16; e++) o[e] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  // Tile t's keys and values, thread-strided float4s; rows past the keys
  // read zeros (the resource ends with the last key row).
  float4 kp[kF4], vp[kF4];
  auto load_tile = [&](int t) {
    const int kt = kstart + t * kPK;
    const uint32_t range = (uint32_t)min(kPK, kend - kt) * (uint32_t)kv_dim * 4u;
    const i32x4 kr = buffer_rsrc(keys + (size_t)kt * kv_dim + kvo, range);
    const i32x4 vr = buffer_rsrc(values + (size_t)kt * kv_dim + kvo, range);
#pragma unroll
    for (int j = 0; j < kF4; j++) {
      // K: consecutive threads along a row. V: consecutive threads down a
      // column, so that its transposed LDS writes fall in distinct banks.
      const int f = j * kThreads + tid;
      kp[j] = buffer_load_f4(kr, (f / (HD / 4)) * kv_dim * 4 + (f % (HD / 4)) * 16);
      vp[j] = buffer_load_f4(vr, (f % kPK) * kv_dim * 4 + (f / kPK) * 16);
    }
  };
  if (tile_lo < tile_hi) load_tile(tile_lo);
  for (int t = tile_lo; t < tile_hi; t++) {
    __syncthreads();  // every wave is done with the previous tile
#pragma unroll
    for (int j = 0; j < kF4; j++) {
      const int f = j * kThreads + tid;
      *(float4*)(Ks + (f / (HD / 4)) * KS + (f % (HD / 4)) * 4) = kp[j];
      const int row = f % kPK, c4 = f / kPK;
      Vt[(c4 * 4 + 0) * VS + row] = vp[j].x;
      Vt[(c4 * 4 + 1) * VS + row] = vp[j].y;
      Vt[(c4 * 4 + 2) * VS + row] = vp[j].z;
      Vt[(c4 * 4 + 3) * VS + row] = vp[j].w;
    }
    __syncthreads();
    if (t + 1 < tile_hi) load_tile(t + 1);  // in flight during this tile's math
    const int kt = kstart + t * kPK;

    // S^T for the tile's two 16-key halves, each as two chains (even and
    // odd steps) so that dependent MFMAs interleave.
    v4f sa[2][2];
#pragma unroll
    for (int c = 0; c < 2; c++) sa[c][0] = sa[c][1] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s4 = 0; s4 < HD / 16; s4++) {
#pragma unroll
      for (int c = 0; c < 2; c++) {
        const float4 k4 = *(const float4*)(Ks + (c * 16 + c16) * KS + g4 * (HD / 4) + 4 * s4);
        sa[c][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4.x, qr[4 * s4], sa[c][0], 0, 0, 0);
        sa[c][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4.y, qr[4 * s4 + 1], sa[c][1], 0, 0, 0);
        sa[c][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4.z, qr[4 * s4 + 2], sa[c][0], 0, 0, 0);
        sa[c][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4.w, qr[4 * s4 + 3], sa[c][1], 0, 0, 0);
      }
    }
    // Scores of keys kt + 16 c + 4 g4 + v for query tq, masked; online softmax.
    float p[2][4];
    float mt = -INFINITY;
#pragma unroll
    for (int c = 0; c < 2; c++)
#pragma unroll
      for (int v = 0; v < 4; v++) {
        const int kpos = kt + c * 16 + 4 * g4 + v;
        const bool ok = kpos < kend && kpos <= qpos && (window <= 0 || kpos > qpos - window);
        const float x = (sa[c][0][v] + sa[c][1][v]) * scale;
        p[c][v] = ok ? x : -INFINITY;
        mt = fmaxf(mt, p[c][v]);
      }
    mt = rows4_max(mt);
    const float m_new = fmaxf(m_run, mt);
    const float alpha = m_run == -INFINITY ? 0.0f : __expf(m_run - m_new);
    float ps = 0.0f;
#pragma unroll
    for (int c = 0; c < 2; c++)
#pragma unroll
      for (int v = 0; v < 4; v++) {
        p[c][v] = p[c][v] == -INFINITY ? 0.0f : __expf(p[c][v] - m_new);
        ps += p[c][v];
      }
    ps = rows4_sum(ps);
    l_run = l_run * alpha + ps;
    // The running sums change only where a max grew (alpha < 1); once the
    // maxima settle most tiles skip the rescale of the accumulators.
    if (__any(alpha != 1.0f)) {
#pragma unroll
      for (int e = 0; e < HD / 16; e++) o[e] *= alpha;
    }
    m_run = m_new;
    // O^T += V^T P^T: step s takes keys (s / 4) * 16 + 4 g4 + s % 4.
#pragma unroll
    for (int c = 0; c < 2; c++) {
      float4 v4[HD / 16];
#pragma unroll
      for (int e = 0; e < HD / 16; e++)
        v4[e] = *(const float4*)(Vt + (e * 16 + c16) * VS + c * 16 + 4 * g4);
#pragma unroll
      for (int e = 0; e < HD / 16; e++)
        o[e] = __builtin_amdgcn_mfma_f32_16x16x4f32(v4[e].x, p[c][0], o[e], 0, 0, 0);
#pragma unroll
      for (int e = 0; e < HD / 16; e++)
        o[e] = __builtin_amdgcn_mfma_f32_16x16x4f32(v4[e].y, p[c][1], o[e], 0, 0, 0);
#pragma unroll
      for (int e = 0; e < HD / 16; e++)
        o[e] = __builtin_amdgcn_mfma_f32_16x16x4f32(v4[e].z, p[c][2], o[e], 0, 0, 0);
#pragma unroll
      for (int e = 0; e < HD / 16; e++)
        o[e] = __builtin_amdgcn_mfma_f32_16x16x4f32(v4[e].w, p[c][3], o[e], 0, 0, 0);
    }
  }

  // The wave's O^T (dims x 16 queries) through LDS to rows, then out.
  __syncthreads();  // the tiles' LDS is free
  float* tw = lds + wave * kPQ * (HD + 4);
#pragma unroll
  for (int e = 0; e < HD / 16; e++)
#pragma unroll
    for (int v = 0; v < 4; v++) tw[c16 * (HD + 4) + e * 16 + 4 * g4 + v] = o[e][v];
  if (g4 == 0) {
    tw[c16 * (HD + 4) + HD] = m_run;
    tw[c16 * (HD + 4) + HD + 1] = l_run;
  }
  __syncthreads();
  constexpr int kC4 = HD / 4;            // float4 per row
  constexpr int kRows = 64 / kC4;        // rows per pass of the wave
  const int c4 = lane % kC4;
  for (int r = lane / kC4; r < kPQ; r += kRows) {
    const int tok = t0 + r;
    if (tok >= n) break;
    const float* row = tw + r * (HD + 4);
    const float4 val = *(const float4*)(row + 4 * c4);
    const size_t th = (size_t)tok * heads + head;
    if (splits > 1) {
      float* w = ws + (th * splits + split) * (HD + 4);
      *(float4*)(w + 4 + 4 * c4) = val;
      if (c4 == 0) {
        w[0] = row[HD];
        w[1] = row[HD + 1];
      }
    } else {
      const float l = row[HD + 1];
      const float g = gate != nullptr ? 1.0f / (1.0f + expf(-gate[th])) : 1.0f;
      float4 y = make_float4(val.x / l, val.y / l, val.z / l, val.w / l);
      if (gate != nullptr) y = make_float4(y.x * g, y.y * g, y.z * g, y.w * g);
      *(float4*)(out + th * HD + 4 * c4) = y;
    }
  }
}

// The combine for many (token, head) rows and at most 64 splits (prefill):
// one wave per row, four rows per workgroup, no barrier. Lane s holds split
// s's statistics; the value sums run in split order with C splits' loads in
// flight (the fewest of 2, 4, 8 covering the splits), dims lane + 64 i. Rows past the splits read zeros (the resource
// ends with the row's last split), and dims past hd are computed but not
// stored.
//
// With `panel` (hd a multiple of 32, at most 256), each row's values also go
// into the fp6 activation panel of out ([tokens][heads * hd]) for the matmul
// that reads it (a prefill chunk's o projection): the row through the wave's
// LDS, then four lanes per 32-value block (panel4_lane, the panel
// quantizer's bytes). Records of tokens past the last row are not written.
template <int C>  // splits per load batch: 2, 4 or 8
__global__ void __launch_bounds__(kThreads)
attention_combine_rows_kernel(const float* __restrict__ ws, const float* __restrict__ gate,
                              float* __restrict__ out, int heads, int hd, int splits, int rows,
                              uint8_t* __restrict__ panel) {
  __shared__ __align__(16) float row_lds[kWaves][256];
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * kWaves + (threadIdx.x >> 6);   // token * heads + head
  if (r >= rows) return;
  const int row = hd + 4;
  const i32x4 rs = buffer_rsrc(ws + (size_t)r * splits * row, (uint32_t)splits * row * 4u);
  const float m = lane < splits ? __int_as_float(dnx_raw_buffer_load_i32(rs, lane * row * 4, 0, 0))
                                : -INFINITY;
  const float ls = __int_as_float(dnx_raw_buffer_load_i32(rs, (lane * row + 1) * 4, 0, 0));
  constexpr int kND = 4;   // dims per lane: hd <= 256
  const int nd = (hd + 63) / 64;
  float acc[kND] = {0.0f, 0.0f, 0.0f, 0.0f};
  const float mx = wave_max(m);
  const float f = m == -INFINITY ? 0.0f : expf(m - mx);
  const float l = wave_sum(ls * f);
  for (int s0 = 0; s0 < splits; s0 += C) {
    float v[C][kND];
#pragma unroll
    for (int u = 0; u < C; u++)
#pragma unroll
      for (int i = 0; i < kND; i++)
        v[u][i] = i < nd ? __int_as_float(dnx_raw_buffer_load_i32(
                               rs, ((s0 + u) * row + 4 + lane + 64 * i) * 4, 0, 0))
                         : 0.0f;
#pragma unroll
    for (int u = 0; u < C; u++) {
      const float fs = __shfl(f, s0 + u);   // 0 past the last split
#pragma unroll
      for (int i = 0; i < kND; i++) acc[i] += v[u][i] * fs;
    }
  }
  const float g = gate != nullptr ? 1.0f / (1.0f + expf(-gate[r])) : 1.0f;
  float* mine = row_lds[threadIdx.x >> 6];
#pragma unroll
  for (int i = 0; i < kND; i++) {
    const int d = lane + 64 * i;
    const float o = gate != nullptr ? (acc[i] / l) * g : acc[i] / l;
    if (i < nd && d < hd) {
      out[(size_t)r * hd + d] = o;
      mine[d] = o;
    }
  }
  if (panel == nullptr) return;
  // LDS operations of one wave execute in order; the fence keeps the
  // compiler from moving the reads above the writes.
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  if (lane < hd / 8) {
    const int token = r / heads, head = r - token * heads;
    const int B = heads * hd / kBlock;
    const int b = head * (hd / kBlock) + (lane >> 2);
    const float4 v0 = *(const float4*)(mine + lane * 8);
    const float4 v1 = *(const float4*)(mine + lane * 8 + 4);
    panel4_lane(v0, v1, lane & 3, token % kTokens,
                panel + ((size_t)(token / kTokens) * B + b) * kRec);
  }
}

template <int HD>
void launch_prefill(int gw, dim3 grid, hipStream_t st, const float* q, const float* keys,
                    const float* values, const float* gate, float* out, float* ws, int position,
                    int n, int heads, int kv_dim, int group, int window, float scale, int splits,
                    int tps) {
  auto k = gw == 4 ? attention_prefill_kernel<HD, 4>
         : gw == 2 ? attention_prefill_kernel<HD, 2> : attention_prefill_kernel<HD, 1>;
  hipLaunchKernelGGL(k, grid, dim3(kThreads), 0, st, q, keys, values, gate, out, ws, position, n,
                     heads, kv_dim, group, window, scale, splits, tps);
}

// Library-owned workspace of the split attention, grown on demand: a call
// with more (head, token, split) entries than any before allocates, so such
// a call must not be the first inside a graph capture.
float* gAttnWs = nullptr;
size_t gAttnWsBytes = 0;

float* attention_workspace(size_t bytes) {
  if (bytes <= gAttnWsBytes) return gAttnWs;
  if (gAttnWs != nullptr) {
    if (hipDeviceSynchronize() != hipSuccess) return nullptr;
    (void)hipFree(gAttnWs);
    gAttnWs = nullptr;
    gAttnWsBytes = 0;
  }
  if (hipMalloc(&gAttnWs, bytes) != hipSuccess) return nullptr;
  gAttnWsBytes = bytes;
  return gAttnWs;
}

// dst += src (lab_metal.m:560-566) and dst = src (:567-572), element-wise.
__global__ void __launch_bounds__(kThreads)
add_kernel(const float* __restrict__ src, float* __restrict__ dst, int64_t count) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < count;
       i += (int64_t)gridDim.x * kThreads) {
    dst[i] = dst[i] + src[i];
  }
}

__global__ void __launch_bounds__(kThreads)
copy_kernel(const float* __restrict__ src, float* __restrict__ dst, int64_t count) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < count;
       i += (int64_t)gridDim.x * kThreads) {
    dst[i] = src[i];
  }
}

// Activation steering in place, semantics of lab_metal.m:531-557. Each
// workgroup rewrites one row. Mode 0 shifts the row by the vector. Mode 1
// projects out the vector's direction, scaled: the block reduces the row's
// dot product with v (v is expected to have unit length), then every
// element drops (scale * dot) * v[j].
__global__ void __launch_bounds__(kThreads)
steer_kernel(float* x, const float* __restrict__ v, int cols, int mode, float scale) {
  __shared__ float scratch[kWaves];
  float* xr = x + (size_t)blockIdx.x * cols;
  if (mode == 0) {
    for (int j = threadIdx.x; j < cols; j += kThreads) xr[j] = xr[j] + v[j];
    return;
  }
  float along = 0.0f;
  for (int j = threadIdx.x; j < cols; j += kThreads) along += xr[j] * v[j];
  along = block_sum(along, scratch);
  const float c = scale * along;
  for (int j = threadIdx.x; j < cols; j += kThreads) xr[j] = xr[j] - c * v[j];
}

int grid_for(int64_t items) {
  const int64_t g = (items + kThreads - 1) / kThreads;
  return (int)(g < 1 ? 1 : g > 65536 ? 65536 : g);
}

// The split-key attention (few (head, token) pairs, many keys): the split
// kernel, then the combine. DNX_EINVAL when it does not apply (nothing
// launched). rp: the q and k head norms folded in (one token, one
// workgroup per KV head and split), or null.
int attention_split(const float* q, const float* keys, const float* values, const float* gate,
                    float* out, int64_t position, int64_t n, int64_t heads, int64_t kv_heads,
                    int64_t hd, int64_t window, float scale, dnx_stream_t stream,
                    const RopeArgs* rp) {
  const int64_t last = position + n - 1;
  const int64_t keys_of_last = window > 0 && last >= window ? window : last + 1;
  const int kps = split_keys((int)hd);
  const int64_t splits = (keys_of_last + kps - 1) / kps;
  // (Also when the keys exceed the one-workgroup kernel's LDS.) The split
  // kernel's buffer offsets reach 4096 key rows: 32-bit up to 2^17 floats
  // per row.
  const size_t ws_bytes = (size_t)heads * n * splits * (hd + 4) * 4;
  if (!(splits > 1 && (heads * n < 256 || keys_of_last > dnx_attention_max_keys(hd)) &&
        splits <= 16000 && ws_bytes <= ((size_t)1 << 30) && kv_heads * hd <= (1 << 17))) {
    return DNX_EINVAL;
  }
  // G query heads per workgroup: the largest of 8, 4, 2, 1 dividing the
  // heads per KV head.
  const int group = (int)(heads / kv_heads);
  const int G = group % 8 == 0 ? 8 : group % 4 == 0 ? 4 : group % 2 == 0 ? 2 : 1;
  if (rp != nullptr && (n != 1 || G != group || hd > kRopeMaxHd)) return DNX_EINVAL;
  float* ws = attention_workspace(ws_bytes);
  if (ws == nullptr) return DNX_ENOMEM;
  const dim3 grid((unsigned)(heads / G), (unsigned)n, (unsigned)splits);
  const hipStream_t st = (hipStream_t)stream;
  const int kv_dim = (int)(kv_heads * hd);
  const RopeArgs ra = rp != nullptr ? *rp : RopeArgs{};
  auto split = [&](auto g_tag, auto rope_tag) {
    constexpr int kG = decltype(g_tag)::value;
    constexpr bool kR = decltype(rope_tag)::value;
    launch_split<kG, kR>(grid, st, q, keys, values, ws, (int)position, (int)heads, kv_dim, group,
                         (int)hd, (int)window, scale, (int)splits, kps, ra);
  };
  auto by_g = [&](auto rope_tag) {
    switch (G) {
      case 8: split(std::integral_constant<int, 8>{}, rope_tag); break;
      case 4: split(std::integral_constant<int, 4>{}, rope_tag); break;
      case 2: split(std::integral_constant<int, 2>{}, rope_tag); break;
      default: split(std::integral_constant<int, 1>{}, rope_tag); break;
    }
  };
  if (rp != nullptr) {
    by_g(std::true_type{});
  } else {
    by_g(std::false_type{});
  }
  if (hipGetLastError() != hipSuccess) return DNX_ELAUNCH;
  if (rp != nullptr) {
    hipLaunchKernelGGL(attention_combine_kernel<true>, dim3((unsigned)heads, (unsigned)n),
                       dim3(kThreads), (size_t)splits * 4, st, ws, gate, out, (int)heads,
                       (int)hd, (int)splits, const_cast<float*>(q), ra);
  } else {
    hipLaunchKernelGGL(attention_combine_kernel<false>, dim3((unsigned)heads, (unsigned)n),
                       dim3(kThreads), (size_t)splits * 4, st, ws, gate, out, (int)heads,
                       (int)hd, (int)splits, (float*)nullptr, RopeArgs{});
  }
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

// The vector norm with the activation panel of its output (kPanel), with
// or without the residual add before it (kAdd): V float4 per thread as the
// row needs, the row in dynamic LDS.
template <bool kAdd>
int launch_norm_panel(const float* x_in, const float* w, float* out, int64_t rows, int64_t cols,
                      float eps, const float* m, float* x_out, uint8_t* panel, hipStream_t s) {
  const int64_t per = (cols / 4 + kThreads - 1) / kThreads;  // float4 per thread
  const size_t lds = (size_t)cols * 4;
  const dim3 grid((unsigned)rows);
  if (per <= 1) {
    hipLaunchKernelGGL((rms_norm_vec_kernel<1, kAdd, true>), grid, dim3(kThreads), lds, s, x_in, w,
                       out, (int)cols, eps, 0, m, x_out, panel);
  } else if (per <= 2) {
    hipLaunchKernelGGL((rms_norm_vec_kernel<2, kAdd, true>), grid, dim3(kThreads), lds, s, x_in, w,
                       out, (int)cols, eps, 0, m, x_out, panel);
  } else if (per <= 4) {
    hipLaunchKernelGGL((rms_norm_vec_kernel<4, kAdd, true>), grid, dim3(kThreads), lds, s, x_in, w,
                       out, (int)cols, eps, 0, m, x_out, panel);
  } else {
    hipLaunchKernelGGL((rms_norm_vec_kernel<8, kAdd, true>), grid, dim3(kThreads), lds, s, x_in, w,
                       out, (int)cols, eps, 0, m, x_out, panel);
  }
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

bool norm_panel_ok(int64_t rows, int64_t cols, uintptr_t ptrs) {
  return rows > 0 && rows <= 256 && cols > 0 && cols % kBlock == 0 && cols <= 8192 &&
         (ptrs & 15) == 0 && f6_panel_bytes(rows, cols) < (1ll << 31);
}

}  // namespace

extern "C" {

int dnx_rms_norm_f6panel(const float* x, const float* w, float* out, void* panel, int64_t rows,
                         int64_t cols, float eps, dnx_stream_t stream) {
  if (!norm_panel_ok(rows, cols, (uintptr_t)x | (uintptr_t)w | (uintptr_t)out | (uintptr_t)panel)) {
    return DNX_EINVAL;
  }
  return launch_norm_panel<false>(x, w, out, rows, cols, eps, nullptr, nullptr, (uint8_t*)panel,
                                  (hipStream_t)stream);
}

int dnx_add_rms_norm_f6panel(const float* m, float* x, const float* w, float* out, void* panel,
                             int64_t rows, int64_t cols, float eps, dnx_stream_t stream) {
  if (!norm_panel_ok(rows, cols, (uintptr_t)m | (uintptr_t)x | (uintptr_t)w | (uintptr_t)out |
                                     (uintptr_t)panel)) {
    return DNX_EINVAL;
  }
  return launch_norm_panel<true>(x, w, out, rows, cols, eps, m, x, (uint8_t*)panel,
                                 (hipStream_t)stream);
}

int dnx_rms_norm(const float* x, const float* w, float* out, int64_t rows, int64_t cols,
                 float eps, int accumulate, dnx_stream_t stream) {
  if (rows < 0 || cols <= 0 || cols > (1 << 30) || rows > 0x7fffffff) return DNX_EINVAL;
  if (rows == 0) return DNX_OK;
  // Register rows for the latency-bound case (no more rows than CUs, as in a
  // decode step); at prefill sizes the streaming loop keeps more rows in
  // flight (4096 x 2048: 14 against 21 us).
  const bool vec = rows <= 256 && cols % 4 == 0 && cols <= 16 * 4 * kThreads &&
                   (((uintptr_t)x | (uintptr_t)w | (uintptr_t)out) & 15) == 0;
  const unsigned grid = (unsigned)rows;
  const hipStream_t s = (hipStream_t)stream;
  if (vec) {
    const int64_t per = (cols / 4 + kThreads - 1) / kThreads;  // float4 per thread
    if (per <= 1) {
      hipLaunchKernelGGL(rms_norm_vec_kernel<1>, dim3(grid), dim3(kThreads), 0, s, x, w, out,
                         (int)cols, eps, accumulate, nullptr, nullptr, nullptr);
    } else if (per <= 2) {
      hipLaunchKernelGGL(rms_norm_vec_kernel<2>, dim3(grid), dim3(kThreads), 0, s, x, w, out,
                         (int)cols, eps, accumulate, nullptr, nullptr, nullptr);
    } else if (per <= 4) {
      hipLaunchKernelGGL(rms_norm_vec_kernel<4>, dim3(grid), dim3(kThreads), 0, s, x, w, out,
                         (int)cols, eps, accumulate, nullptr, nullptr, nullptr);
    } else if (per <= 8) {
      hipLaunchKernelGGL(rms_norm_vec_kernel<8>, dim3(grid), dim3(kThreads), 0, s, x, w, out,
                         (int)cols, eps, accumulate, nullptr, nullptr, nullptr);
    } else {
      hipLaunchKernelGGL(rms_norm_vec_kernel<16>, dim3(grid), dim3(kThreads), 0, s, x, w, out,
                         (int)cols, eps, accumulate, nullptr, nullptr, nullptr);
    }
  } else {
    hipLaunchKernelGGL(rms_norm_kernel, dim3(grid), dim3(kThreads), 0, s, x, w, out, (int)cols,
                       eps, accumulate);
  }
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int dnx_add_rms_norm(const float* m, float* x, const float* w, float* out, int64_t rows,
                     int64_t cols, float eps, dnx_stream_t stream) {
  if (rows < 0 || cols <= 0 || rows > 256 || cols % 4 != 0 || cols > 16 * 4 * kThreads ||
      (((uintptr_t)m | (uintptr_t)x | (uintptr_t)w | (uintptr_t)out) & 15) != 0) {
    return DNX_EINVAL;
  }
  if (rows == 0) return DNX_OK;
  const unsigned grid = (unsigned)rows;
  const hipStream_t s = (hipStream_t)stream;
  const int64_t per = (cols / 4 + kThreads - 1) / kThreads;  // float4 per thread
  if (per <= 1) {
    hipLaunchKernelGGL((rms_norm_vec_kernel<1, true>), dim3(grid), dim3(kThreads), 0, s, x, w,
                       out, (int)cols, eps, 0, m, x, nullptr);
  } else if (per <= 2) {
    hipLaunchKernelGGL((rms_norm_vec_kernel<2, true>), dim3(grid), dim3(kThreads), 0, s, x, w,
                       out, (int)cols, eps, 0, m, x, nullptr);
  } else if (per <= 4) {
    hipLaunchKernelGGL((rms_norm_vec_kernel<4, true>), dim3(grid), dim3(kThreads), 0, s, x, w,
                       out, (int)cols, eps, 0, m, x, nullptr);
  } else if (per <= 8) {
    hipLaunchKernelGGL((rms_norm_vec_kernel<8, true>), dim3(grid), dim3(kThreads), 0, s, x, w,
                       out, (int)cols, eps, 0, m, x, nullptr);
  } else {
    hipLaunchKernelGGL((rms_norm_vec_kernel<16, true>), dim3(grid), dim3(kThreads), 0, s, x, w,
                       out, (int)cols, eps, 0, m, x, nullptr);
  }
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int dnx_head_norm_rope(float* x, int64_t x_stride, const float* w, const float* rope,
                       int64_t rope_stride, int64_t heads, int64_t hd, int64_t n, float eps,
                       dnx_stream_t stream) {
  if (heads <= 0 || n < 0 || hd <= 0 || hd % 2 != 0 || hd > 512 || x_stride < heads * hd ||
      rope_stride < hd || x_stride > 0x7fffffff || rope_stride > 0x7fffffff ||
      heads > 65535 || n > 65535) {
    return DNX_EINVAL;
  }
  if (n == 0) return DNX_OK;
  hipLaunchKernelGGL(head_norm_rope_kernel, dim3((unsigned)heads, (unsigned)n), dim3(64), 0,
                     (hipStream_t)stream, x, (int)x_stride, w, rope, (int)rope_stride, (int)hd,
                     eps, (int)heads, x, (int)x_stride, w);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int dnx_head_norm_rope2(float* x0, int64_t x0_stride, const float* w0, int64_t heads0,
                        float* x1, int64_t x1_stride, const float* w1, int64_t heads1,
                        const float* rope, int64_t rope_stride, int64_t hd, int64_t n, float eps,
                        dnx_stream_t stream) {
  if (heads0 <= 0 || heads1 <= 0 || n < 0 || hd <= 0 || hd % 2 != 0 || hd > 512 ||
      x0_stride < heads0 * hd || x1_stride < heads1 * hd || rope_stride < hd ||
      x0_stride > 0x7fffffff || x1_stride > 0x7fffffff || rope_stride > 0x7fffffff ||
      heads0 + heads1 > 65535 || n > 65535) {
    return DNX_EINVAL;
  }
  if (n == 0) return DNX_OK;
  hipLaunchKernelGGL(head_norm_rope_kernel, dim3((unsigned)(heads0 + heads1), (unsigned)n),
                     dim3(64), 0, (hipStream_t)stream, x0, (int)x0_stride, w0, rope,
                     (int)rope_stride, (int)hd, eps, (int)heads0, x1, (int)x1_stride, w1);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int dnx_short_conv(const float* bcx, const float* weight, float* history, float* y,
                   int64_t width, int64_t k, int64_t n, dnx_stream_t stream) {
  if (width <= 0 || k < 1 || k > kMaxConvK || n < 0 || width > 0x7fffffff ||
      n > 0x7fffffff) {
    return DNX_EINVAL;
  }
  if (n == 0) return DNX_OK;
  const int64_t slabs = (width + kConvCh - 1) / kConvCh, tiles = (n + kConvT - 1) / kConvT;
  if (slabs > 0x7fffffff || tiles > 65535) return DNX_EINVAL;
  hipLaunchKernelGGL(conv_kernel, dim3((unsigned)slabs, (unsigned)tiles), dim3(kThreads), 0,
                     (hipStream_t)stream, bcx, weight, history, y, (int)width, (int)k, (int)n);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int dnx_attention_rope(float* q, float* keys, const float* values, const float* gate, float* out,
                       int64_t position, int64_t heads, int64_t kv_heads, int64_t hd,
                       int64_t window, const float* q_norm, const float* k_norm,
                       const float* rope, float eps, dnx_stream_t stream) {
  if (position < 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads != 0 || hd <= 0 ||
      hd % 4 != 0 || hd > kRopeMaxHd || kThreads % hd != 0 || window < 0 || heads > 65535 ||
      position + 1 > 0x7fffffff || ((uintptr_t)keys & 15) || ((uintptr_t)q & 15) ||
      q_norm == nullptr || k_norm == nullptr || rope == nullptr) {
    return DNX_EINVAL;
  }
  const RopeArgs rp{rope, q_norm, k_norm, keys, eps};
  return attention_split(q, keys, values, gate, out, position, 1, heads, kv_heads, hd, window,
                         (float)(1.0 / sqrt((double)hd)), stream, &rp);
}

int64_t dnx_attention_max_keys(int64_t hd) {
  if (hd <= 0 || hd > 256 || kThreads % hd != 0) return -1;
  // LDS: q (hd) + scores (rounded up to 4) + value partials ((256 / hd) x
  // hd) + the kernel's 4-float reduction scratch, within 64 KB.
  return (64 * 1024 / 4) - hd - kThreads - 4 - kWaves;
}

// The attention, and with `panel` the fp6 activation panel of out too (only
// where the split matrix-core path and its row combine run; else DNX_EINVAL
// before anything is launched).
static int attention_impl(const float* q, const float* keys, const float* values,
                          const float* gate, float* out, uint8_t* panel, int64_t position,
                          int64_t n, int64_t heads, int64_t kv_heads, int64_t hd, int64_t window,
                          dnx_stream_t stream) {
  if (n < 0 || position < 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads != 0 ||
      hd <= 0 || hd % 4 != 0 || hd > 256 || kThreads % hd != 0 || window < 0 ||
      heads > 65535 || n > 65535 || position + n > 0x7fffffff || ((uintptr_t)keys & 15) ||
      ((uintptr_t)q & 15)) {
    return DNX_EINVAL;
  }
  if (panel != nullptr && (hd % kBlock != 0 || ((uintptr_t)panel & 15) || n == 0)) {
    return DNX_EINVAL;
  }
  if (n == 0) return DNX_OK;
  const int64_t last = position + n - 1;
  const int64_t keys_of_last = window > 0 && last >= window ? window : last + 1;
  const float scale = (float)(1.0 / sqrt((double)hd));
  // 8+ tokens at hd 64 or 128: the matrix-core kernel, its keys split over
  // workgroups while fewer than kTargetWaves waves would run.
  if ((hd == 64 || hd == 128) && n >= 8 && kv_heads * hd <= (1 << 20) &&
      ((uintptr_t)out & 15) == 0) {
    constexpr int64_t kTargetWaves = 2048;
    const int64_t group = heads / kv_heads;
    const int gw = group % 4 == 0 ? 4 : group % 2 == 0 ? 2 : 1;
    const int64_t qb = kPQ * (4 / gw);   // queries per workgroup
    const int64_t by = (n + qb - 1) / qb;
    int64_t tmax = 1;  // tiles of the longest workgroup range
    for (int64_t b = 0; b < by; b++) {
      const int64_t first = b * qb, lastq = (first + qb < n ? first + qb : n) - 1;
      const int64_t ks = window > 0 && position + first - window + 1 > 0
                             ? position + first - window + 1 : 0;
      const int64_t t = (position + lastq + 1 - ks + kPK - 1) / kPK;
      if (t > tmax) tmax = t;
    }
    const int64_t waves = heads / gw * by * 4;
    int64_t splits = 1;
    if (waves < kTargetWaves && tmax >= 4) {
      splits = (kTargetWaves + waves - 1) / waves;
      if (splits > tmax / 2) splits = tmax / 2;
    }
    int64_t tps = (tmax + splits - 1) / splits;
    splits = (tmax + tps - 1) / tps;
    size_t pws = splits > 1 ? (size_t)n * heads * splits * (hd + 4) * 4 : 0;
    if (pws > ((size_t)1 << 30) || splits > 4096) {
      splits = 1;
      tps = tmax;
      pws = 0;
    }
    if (panel != nullptr && !(splits > 1 && splits <= 64)) return DNX_EINVAL;
    float* ws = nullptr;
    if (splits > 1 && (ws = attention_workspace(pws)) == nullptr) return DNX_ENOMEM;
    const dim3 grid((unsigned)(heads / gw), (unsigned)by, (unsigned)splits);
    const hipStream_t st = (hipStream_t)stream;
    if (hd == 128) {
      launch_prefill<128>(gw, grid, st, q, keys, values, gate, out, ws, (int)position, (int)n,
                          (int)heads, (int)(kv_heads * hd), (int)group, (int)window, scale,
                          (int)splits, (int)tps);
    } else {
      launch_prefill<64>(gw, grid, st, q, keys, values, gate, out, ws, (int)position, (int)n,
                         (int)heads, (int)(kv_heads * hd), (int)group, (int)window, scale,
                         (int)splits, (int)tps);
    }
    if (hipGetLastError() != hipSuccess) return DNX_ELAUNCH;
    if (splits > 1 && splits <= 64) {
      const int64_t rows = n * heads;
      auto k = splits <= 2 ? attention_combine_rows_kernel<2>
             : splits <= 4 ? attention_combine_rows_kernel<4> : attention_combine_rows_kernel<8>;
      hipLaunchKernelGGL(k, dim3((unsigned)((rows + kWaves - 1) / kWaves)), dim3(kThreads), 0, st,
                         ws, gate, out, (int)heads, (int)hd, (int)splits, (int)rows, panel);
    } else if (splits > 1) {
      hipLaunchKernelGGL(attention_combine_kernel<false>, dim3((unsigned)heads, (unsigned)n),
                         dim3(kThreads), (size_t)splits * 4, st, ws, gate, out, (int)heads,
                         (int)hd, (int)splits, (float*)nullptr, RopeArgs{});
    }
    return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
  }
  if (panel != nullptr) return DNX_EINVAL;
  // Few (head, token) workgroups for many keys: split the keys.
  const int rc = attention_split(q, keys, values, gate, out, position, n, heads, kv_heads, hd,
                                 window, scale, stream, nullptr);
  if (rc != DNX_EINVAL) return rc;
  if (keys_of_last > dnx_attention_max_keys(hd)) return DNX_EINVAL;
  const size_t lds = (size_t)(hd + ((keys_of_last + 3) & ~3ll) + kThreads) * 4;
  hipLaunchKernelGGL(attention_kernel, dim3((unsigned)heads, (unsigned)n), dim3(kThreads), lds,
                     (hipStream_t)stream, q, keys, values, gate, out, (int)position,
                     (int)heads, (int)(kv_heads * hd), (int)(heads / kv_heads), (int)hd,
                     (int)window, scale);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int dnx_attention(const float* q, const float* keys, const float* values, const float* gate,
                  float* out, int64_t position, int64_t n, int64_t heads, int64_t kv_heads,
                  int64_t hd, int64_t window, dnx_stream_t stream) {
  return attention_impl(q, keys, values, gate, out, nullptr, position, n, heads, kv_heads, hd,
                        window, stream);
}

int dnx_attention_f6panel(const float* q, const float* keys, const float* values,
                          const float* gate, float* out, void* panel, int64_t position, int64_t n,
                          int64_t heads, int64_t kv_heads, int64_t hd, int64_t window,
                          dnx_stream_t stream) {
  if (panel == nullptr) return DNX_EINVAL;
  return attention_impl(q, keys, values, gate, out, (uint8_t*)panel, position, n, heads,
                        kv_heads, hd, window, stream);
}

int dnx_add(const float* src, float* dst, int64_t count, dnx_stream_t stream) {
  if (count < 0) return DNX_EINVAL;
  if (count == 0) return DNX_OK;
  hipLaunchKernelGGL(add_kernel, dim3(grid_for(count)), dim3(kThreads), 0, (hipStream_t)stream,
                     src, dst, count);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int dnx_copy(const float* src, float* dst, int64_t count, dnx_stream_t stream) {
  if (count < 0) return DNX_EINVAL;
  if (count == 0) return DNX_OK;
  hipLaunchKernelGGL(copy_kernel, dim3(grid_for(count)), dim3(kThreads), 0, (hipStream_t)stream,
                     src, dst, count);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

int dnx_steer(float* x, const float* v, int64_t rows, int64_t cols, int64_t mode, float scale,
              dnx_stream_t stream) {
  if (rows < 0 || cols <= 0 || (mode != 0 && mode != 1) || rows > 0x7fffffff ||
      cols > (1 << 30)) {
    return DNX_EINVAL;
  }
  if (rows == 0) return DNX_OK;
  hipLaunchKernelGGL(steer_kernel, dim3((unsigned)rows), dim3(kThreads), 0, (hipStream_t)stream,
                     x, v, (int)cols, (int)mode, scale);
  return hipGetLastError() == hipSuccess ? DNX_OK : DNX_ELAUNCH;
}

}  // extern "C"
