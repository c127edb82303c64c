// CPU oracle for the quantized linear layer. TEST INFRASTRUCTURE ONLY.
//
// This file restates, in scalar C, the arithmetic of the reference's CPU
// kernels (Atrac613/dianoia src/c/lab_native.c) and the Dart glue around
// them, so that the HIP product can be checked against it on identical
// inputs. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
// leg may load it, and only as the checker or the timed CPU baseline; the
// product library never links it.
//
// Every float operation is written out in the reference's order. The file
// is compiled with -ffp-contract=off so that a*b+c stays two roundings and
// only the explicit fmaf() calls fuse, as in the reference, whose x86 twins
// fuse exactly where NEON does (lab_native.c:13-17, hook/build.dart:19-26).
//
// Pinning (tests/test_oracle.py): every function here is checked against
// the compiled reference (oracle/_ref, built from lab_native.c by
// oracle/Makefile) and against the committed golden fixtures in
// tests/golden/, plus closed forms (quantizer edge cases, exhaustive fp16,
// brute-force integer block dots, argmax ties/NaN). The Dart-only glue
// (orc_silu_mul, orc_gelu) has no compiled reference here: it is pinned by
// closed-form values only (see test_oracle.py), not bit-for-bit against Dart.
// So are the Q6_K decoder (by ggml-layout packing) and the layer steps
// (orc_rms_norm .. orc_steer: closed forms and invariants), whose
// reference is a Metal/Vulkan shader.

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define Q_BLOCK 32

// ------------------------------------------------------------ fp16 <-> fp32

// IEEE binary16 bits -> float, exact (lab_native.c:919-921 uses F16C
// vcvtph2ps; NEON widens _Float16, :905-909; Dart halfToDouble,
// native.dart:871-880). Written from the format's definition.
float orc_half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      // Subnormal half: normalise into a float exponent.
      int e = -1;
      do {
        e++;
        man <<= 1;
      } while ((man & 0x400u) == 0);
      man &= 0x3ffu;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);  // inf, or NaN keeping its payload
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, sizeof f);
  return f;
}

// float -> IEEE binary16 bits, round to nearest even (lab_native.c:923-925,
// F16C vcvtps2ph with _MM_FROUND_TO_NEAREST_INT). NaN keeps the top payload
// bits and is made quiet, as vcvtps2ph does.
uint16_t orc_float_to_half(float f) {
  uint32_t x;
  memcpy(&x, &f, sizeof x);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t exp = (x >> 23) & 0xffu;
  const uint32_t man = x & 0x7fffffu;
  if (exp == 0xff) {
    if (man == 0) return sign | 0x7c00u;
    return (uint16_t)(sign | 0x7e00u | (man >> 13));
  }
  const int e = (int)exp - 127 + 15;
  if (e >= 31) return sign | 0x7c00u;  // overflow to inf
  if (e <= 0) {
    // Subnormal or zero half: shift the full significand right.
    if (e < -10) return sign;  // rounds to zero (below half the smallest subnormal)
    const uint32_t full = man | 0x800000u;
    const int shift = 14 - e;  // 24-bit significand down to the 10-bit field
    const uint32_t q = full >> shift;
    const uint32_t rem = full & ((1u << shift) - 1);
    const uint32_t halfway = 1u << (shift - 1);
    uint32_t r = q;
    if (rem > halfway || (rem == halfway && (q & 1u))) r++;
    return (uint16_t)(sign | r);  // r may carry into the exponent field: correct
  }
  uint32_t r = ((uint32_t)e << 10) | (man >> 13);
  const uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;  // carry may reach inf: correct
  return (uint16_t)(sign | r);
}

// bf16 bits -> float: p << 16, exact (safetensors.dart:207-212).
static inline float bf16_to_float(uint16_t p) {
  const uint32_t bits = (uint32_t)p << 16;
  float f;
  memcpy(&f, &bits, sizeof f);
  return f;
}

// ------------------------------------------------------------ quantizers

// One block of the Q8 quantizer (lab_native.c:411-426): amax with a strict
// '>' (NaN never wins), scale = amax / 127 correctly rounded, inv = 1/scale
// (0 for an all-zero block), q = x * inv then +-0.5 in float, truncation,
// clamp to [-127, 127]. `valid` values are read; the rest of the 32 are 0
// (the zero padding of a tail block, an extension for cols % 32 != 0).
static void quantize_block(const float* src, int valid, int8_t* q, float* scale_out) {
  float v[Q_BLOCK];
  for (int k = 0; k < Q_BLOCK; k++) v[k] = k < valid ? src[k] : 0.0f;
  float amax = 0.0f;
  for (int k = 0; k < Q_BLOCK; k++) {
    const float a = v[k] < 0 ? -v[k] : v[k];
    if (a > amax) amax = a;
  }
  const float scale = amax / 127.0f;
  const float inv = scale > 0 ? 1.0f / scale : 0.0f;
  *scale_out = scale;
  for (int k = 0; k < Q_BLOCK; k++) {
    float t = v[k] * inv;
    t = t < 0 ? t - 0.5f : t + 0.5f;
    const int i = (int)t;
    q[k] = (int8_t)(i > 127 ? 127 : i < -127 ? -127 : i);
  }
}

// lab_quantize_q8 (lab_native.c:407-429). cols % 32 == 0 as the reference
// requires (native.dart:634-636); a tail is dropped, as C does (:409).
void orc_quantize_q8(const float* w, int8_t* qs, float* scales, int64_t rows, int64_t cols) {
  const int64_t blocks = cols / Q_BLOCK;
  for (int64_t r = 0; r < rows; r++) {
    for (int64_t b = 0; b < blocks; b++) {
      quantize_block(w + r * cols + b * Q_BLOCK, Q_BLOCK, qs + r * cols + b * Q_BLOCK,
                     scales + r * blocks + b);
    }
  }
}

// The load-time weight quantizer for BF16 checkpoints: _widenBf16
// (safetensors.dart:207-212) then lab_quantize_q8, with cols zero-padded up
// to cols_pad (a multiple of 32) so K = 4304 becomes 4320: the tail block's
// amax covers only the real values and the pads quantize to 0. qs is
// [rows][cols_pad], scales [rows][cols_pad / 32].
void orc_quantize_q8_bf16(const uint16_t* w, int8_t* qs, float* scales, int64_t rows,
                          int64_t cols, int64_t cols_pad) {
  const int64_t blocks = cols_pad / Q_BLOCK;
  float tmp[Q_BLOCK];
  for (int64_t r = 0; r < rows; r++) {
    for (int64_t b = 0; b < blocks; b++) {
      const int64_t c0 = b * Q_BLOCK;
      int valid = 0;
      for (int k = 0; k < Q_BLOCK; k++) {
        if (c0 + k < cols) {
          tmp[k] = bf16_to_float(w[r * cols + c0 + k]);
          valid = k + 1;
        }
      }
      quantize_block(tmp, valid, qs + r * cols_pad + c0, scales + r * blocks + b);
    }
  }
}

// fp32 rows of width cols, zero-padded to cols_pad, quantized per block:
// the activation quantizer of the padded problem (K = 4304 -> 4320).
void orc_quantize_q8_padded(const float* x, int8_t* qs, float* scales, int64_t rows,
                            int64_t cols, int64_t cols_pad) {
  const int64_t blocks = cols_pad / Q_BLOCK;
  for (int64_t r = 0; r < rows; r++) {
    for (int64_t b = 0; b < blocks; b++) {
      const int64_t c0 = b * Q_BLOCK;
      const int valid = (int)(cols - c0 >= Q_BLOCK ? Q_BLOCK : cols - c0 > 0 ? cols - c0 : 0);
      quantize_block(x + r * cols + c0, valid, qs + r * cols_pad + c0, scales + r * blocks + b);
    }
  }
}

// lab_quantize_q4 (lab_native.c:930-955), llama.cpp's Q4_0 rule: the value
// of largest magnitude maps to q = 0, d = max / -8, q = (int8)(x/d + 8.5f)
// clamped to 15, stored low nibble = weight k, high nibble = weight k + 16.
void orc_quantize_q4(const float* w, uint8_t* qs, uint16_t* scales, int64_t rows,
                     int64_t cols) {
  const int64_t blocks = cols / Q_BLOCK;
  for (int64_t r = 0; r < rows; r++) {
    for (int64_t b = 0; b < blocks; b++) {
      const float* src = w + r * cols + b * Q_BLOCK;
      float amax = 0.0f, max = 0.0f;
      for (int k = 0; k < Q_BLOCK; k++) {
        const float a = src[k] < 0 ? -src[k] : src[k];
        if (a > amax) {
          amax = a;
          max = src[k];
        }
      }
      const float d = max / -8.0f;
      const float id = d != 0.0f ? 1.0f / d : 0.0f;
      scales[r * blocks + b] = orc_float_to_half(d);
      uint8_t* q = qs + (r * cols + b * Q_BLOCK) / 2;
      for (int k = 0; k < Q_BLOCK / 2; k++) {
        const int8_t lo = (int8_t)(src[k] * id + 8.5f);
        const int8_t hi = (int8_t)(src[k + 16] * id + 8.5f);
        q[k] = (uint8_t)((lo > 15 ? 15 : lo) | ((hi > 15 ? 15 : hi) << 4));
      }
    }
  }
}

// ------------------------------------------------------------ Q6_K

// dequantizeQ6K (lib/src/gguf.dart:220-254), ggml's dequantize_row_q6_K:
// super-blocks of 256 values in 210 bytes, ql[128] (4 low bits), qh[64]
// (2 high bits each), sc[16] (int8, one per 16 values), then fp16 d. Per
// half of 128 values and l < 32: q1..q4 = values l, l+32, l+64, l+96 from
// the low nibble of ql[l], of ql[l+32], the high nibble of ql[l], of
// ql[l+32], with qh[l] bits 0-1, 2-3, 4-5, 6-7 above; scales sc[l/16 +
// 0, 2, 4, 6]. Each value is d * sc * (q - 32) in double (Dart's
// halfToDouble, native.dart:871-880, is exact), stored to float.
void orc_dequantize_q6k(const uint8_t* data, float* out, int64_t blocks) {
  for (int64_t b = 0; b < blocks; b++) {
    const uint8_t* base = data + b * 210;
    const double d = (double)orc_half_to_float((uint16_t)(base[208] | base[209] << 8));
    float* y = out + b * 256;
    const uint8_t* ql = base;
    const uint8_t* qh = base + 128;
    const int8_t* sc = (const int8_t*)(base + 192);
    for (int half = 0; half < 2; half++) {
      for (int l = 0; l < 32; l++) {
        const int i = l / 16;
        const int h = qh[l];
        const int q1 = ((ql[l] & 15) | ((h & 3) << 4)) - 32;
        const int q2 = ((ql[l + 32] & 15) | (((h >> 2) & 3) << 4)) - 32;
        const int q3 = ((ql[l] >> 4) | (((h >> 4) & 3) << 4)) - 32;
        const int q4 = ((ql[l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32;
        y[l] = (float)(d * sc[i] * q1);
        y[l + 32] = (float)(d * sc[i + 2] * q2);
        y[l + 64] = (float)(d * sc[i + 4] * q3);
        y[l + 96] = (float)(d * sc[i + 6] * q4);
      }
      y += 128;
      ql += 64;
      qh += 32;
      sc += 8;
    }
  }
}

// The Q6_K -> Q8 embedding / LM-head adapter (gguf.dart:402-414): rows x
// cols (cols a multiple of 256) dequantized row by row, then
// lab_quantize_q8 (NativeQ8Matrix.quantizeRows, native.dart:645-672, which
// quantizes chunks of whole rows: the result does not depend on the chunk).
void orc_q6k_to_q8(const uint8_t* data, int8_t* qs, float* scales, int64_t rows, int64_t cols) {
  float* row = (float*)malloc((size_t)(cols > 0 ? cols : 1) * sizeof(float));
  const int64_t per_row = cols / 256;
  for (int64_t r = 0; r < rows; r++) {
    orc_dequantize_q6k(data + r * per_row * 210, row, per_row);
    orc_quantize_q8(row, qs + r * cols, scales + r * (cols / Q_BLOCK), 1, cols);
  }
  free(row);
}

// ------------------------------------------------------------ products

// (v0 + v1) + (v2 + v3): lane_sum (lab_native.c:209-212, NEON :178-181).
static inline float lane_sum(const float a[4]) { return (a[0] + a[1]) + (a[2] + a[3]); }

// Q4 weight k of a block, in -8..7: low nibble of byte k for k < 16, high
// nibble of byte k - 16 otherwise (lab_native.c:893-900, q4_block :1005-1011).
static inline int q4_weight(const uint8_t* block16, int k) {
  const uint8_t byte = block16[k & 15];
  return (k < 16 ? (byte & 15) : (byte >> 4)) - 8;
}

// Mode 1 of one (row, token) for Q8 weights: dot_q8_sdot (x86 :503-512 with
// sdot_block :483-487; NEON :456-466). Lane l of each block takes the exact
// int32 sum over bytes 4l..4l+3 and 16+4l..19+4l; s = sw * sx rounded to
// float; acc_l = fma(float(d_l), s, acc_l), block after block.
static float dot_q8_int8(const int8_t* row, const float* row_scales, const int8_t* xq,
                         const float* xs, int64_t blocks) {
  float acc[4] = {0, 0, 0, 0};
  for (int64_t b = 0; b < blocks; b++) {
    const int8_t* w = row + b * Q_BLOCK;
    const int8_t* x = xq + b * Q_BLOCK;
    const float s = row_scales[b] * xs[b];
    for (int l = 0; l < 4; l++) {
      int32_t d = 0;
      for (int i = 0; i < 4; i++) {
        d += (int32_t)w[4 * l + i] * x[4 * l + i];
        d += (int32_t)w[16 + 4 * l + i] * x[16 + 4 * l + i];
      }
      acc[l] = fmaf((float)d, s, acc[l]);
    }
  }
  return lane_sum(acc);
}

// Mode 0 of one (row, token) for Q8: dot_q8_f32 (x86 :489-501 with fma16_i8
// :470-478; NEON :433-451). Per block, lane l sums fma(float(w_j), x_j, s_l)
// over j = 4k + l for k = 0..7 in order; then acc_l = fma(s_l, scale, acc_l).
static float dot_q8_float(const int8_t* row, const float* row_scales, const float* x,
                          int64_t blocks) {
  float acc[4] = {0, 0, 0, 0};
  for (int64_t b = 0; b < blocks; b++) {
    const int8_t* w = row + b * Q_BLOCK;
    const float* xb = x + b * Q_BLOCK;
    for (int l = 0; l < 4; l++) {
      float s = 0.0f;
      for (int k = 0; k < 8; k++) s = fmaf((float)w[4 * k + l], xb[4 * k + l], s);
      acc[l] = fmaf(s, row_scales[b], acc[l]);
    }
  }
  return lane_sum(acc);
}

// Mode 1 for Q4 weights: dot_q4_sdot (x86 :1025-1034; NEON :987-1002), the
// same lanes with weights q - 8 and s = half_to_float(d) * sx.
static float dot_q4_int8(const uint8_t* row, const uint16_t* row_scales, const int8_t* xq,
                         const float* xs, int64_t blocks) {
  float acc[4] = {0, 0, 0, 0};
  for (int64_t b = 0; b < blocks; b++) {
    const uint8_t* w = row + b * 16;
    const int8_t* x = xq + b * Q_BLOCK;
    const float s = orc_half_to_float(row_scales[b]) * xs[b];
    for (int l = 0; l < 4; l++) {
      int32_t d = 0;
      for (int i = 0; i < 4; i++) {
        d += q4_weight(w, 4 * l + i) * x[4 * l + i];
        d += q4_weight(w, 16 + 4 * l + i) * x[16 + 4 * l + i];
      }
      acc[l] = fmaf((float)d, s, acc[l]);
    }
  }
  return lane_sum(acc);
}

// Mode 0 for Q4: dot_q4_f32 (x86 :1013-1023; NEON :959-983).
static float dot_q4_float(const uint8_t* row, const uint16_t* row_scales, const float* x,
                          int64_t blocks) {
  float acc[4] = {0, 0, 0, 0};
  for (int64_t b = 0; b < blocks; b++) {
    const uint8_t* w = row + b * 16;
    const float* xb = x + b * Q_BLOCK;
    for (int l = 0; l < 4; l++) {
      float s = 0.0f;
      for (int k = 0; k < 8; k++) s = fmaf((float)q4_weight(w, 4 * k + l), xb[4 * k + l], s);
      acc[l] = fmaf(s, orc_half_to_float(row_scales[b]), acc[l]);
    }
  }
  return lane_sum(acc);
}

// Row boundary of chunk t of n, even (lab_native.c:241-246).
static int64_t boundary(int64_t rows, int64_t t, int64_t n) {
  return t == n ? rows : (rows * t / n) & ~(int64_t)1;
}

// lab_gemm_q8 (lab_native.c:553-579): ys[t * rows + r] = (W xs[t])[r].
// Mode 1 quantizes xs into xq / xsc first (single-threaded, as :556), then
// rows go out in threads * 8 chunks under OpenMP schedule(dynamic, 1)
// (:564-577). A row's result does not depend on the split.
void orc_gemm_q8(const int8_t* qs, const float* scales, const float* xs, int8_t* xq,
                 float* xsc, float* ys, int64_t rows, int64_t cols, int64_t n,
                 int64_t threads, int64_t mode) {
  if (mode == 1) orc_quantize_q8(xs, xq, xsc, n, cols);
  const int64_t blocks = cols / Q_BLOCK;
  const int64_t workers = threads < 1 ? 1 : threads;
  const int64_t chunks = workers == 1 ? 1 : workers * 8;
#pragma omp parallel for num_threads((int)workers) schedule(dynamic, 1)
  for (int64_t c = 0; c < chunks; c++) {
    for (int64_t r = boundary(rows, c, chunks); r < boundary(rows, c + 1, chunks); r++) {
      const int8_t* row = qs + r * cols;
      const float* rs = scales + r * blocks;
      for (int64_t t = 0; t < n; t++) {
        ys[t * rows + r] = mode == 1
                               ? dot_q8_int8(row, rs, xq + t * cols, xsc + t * blocks, blocks)
                               : dot_q8_float(row, rs, xs + t * cols, blocks);
      }
    }
  }
}

// lab_gemm_q4 (lab_native.c:1059-1080): the same for Q4 weights.
void orc_gemm_q4(const uint8_t* qs, const uint16_t* scales, const float* xs, int8_t* xq,
                 float* xsc, float* ys, int64_t rows, int64_t cols, int64_t n,
                 int64_t threads, int64_t mode) {
  if (mode == 1) orc_quantize_q8(xs, xq, xsc, n, cols);
  const int64_t blocks = cols / Q_BLOCK;
  const int64_t workers = threads < 1 ? 1 : threads;
  const int64_t chunks = workers == 1 ? 1 : workers * 8;
#pragma omp parallel for num_threads((int)workers) schedule(dynamic, 1)
  for (int64_t c = 0; c < chunks; c++) {
    for (int64_t r = boundary(rows, c, chunks); r < boundary(rows, c + 1, chunks); r++) {
      const uint8_t* row = qs + r * cols / 2;
      const uint16_t* rs = scales + r * blocks;
      for (int64_t t = 0; t < n; t++) {
        ys[t * rows + r] = mode == 1
                               ? dot_q4_int8(row, rs, xq + t * cols, xsc + t * blocks, blocks)
                               : dot_q4_float(row, rs, xs + t * cols, blocks);
      }
    }
  }
}

// Per-block int32 dot products d[t][r][b] = sum over the 32 values of block b
// of w * xq (the sum of the four lane sums above). Integer-exact, so any
// summation order gives the same value; the GEMM's MFMA tiles must match it.
void orc_block_dots_q8(const int8_t* qs, const int8_t* xq, int32_t* d, int64_t rows,
                       int64_t cols, int64_t n) {
  const int64_t blocks = cols / Q_BLOCK;
  for (int64_t t = 0; t < n; t++)
    for (int64_t r = 0; r < rows; r++)
      for (int64_t b = 0; b < blocks; b++) {
        int32_t s = 0;
        for (int k = 0; k < Q_BLOCK; k++)
          s += (int32_t)qs[r * cols + b * Q_BLOCK + k] * xq[t * cols + b * Q_BLOCK + k];
        d[(t * rows + r) * blocks + b] = s;
      }
}

void orc_block_dots_q4(const uint8_t* qs, const int8_t* xq, int32_t* d, int64_t rows,
                       int64_t cols, int64_t n) {
  const int64_t blocks = cols / Q_BLOCK;
  for (int64_t t = 0; t < n; t++)
    for (int64_t r = 0; r < rows; r++)
      for (int64_t b = 0; b < blocks; b++) {
        int32_t s = 0;
        const uint8_t* w = qs + r * cols / 2 + b * 16;
        for (int k = 0; k < Q_BLOCK; k++) s += q4_weight(w, k) * xq[t * cols + b * Q_BLOCK + k];
        d[(t * rows + r) * blocks + b] = s;
      }
}

// ------------------------------------------------------------ glue

// argmaxToken without suppression (lib/src/sampler.dart:137-143): the first
// index of the maximum; strict '>' so ties keep the lower index and a NaN
// never replaces the best (and a NaN at index 0 stays the answer).
int64_t orc_argmax(const float* logits, int64_t n) {
  int64_t best = 0;
  for (int64_t i = 1; i < n; i++) {
    if (logits[i] > logits[best]) best = i;
  }
  return best;
}

// LayerShard.ffn's glue (lib/src/shard.dart:457-461), in Dart's double
// arithmetic: g = g / (1 + exp(-g)) stored to float32, then g * u stored to
// float32. exp is the C library's double exp here; Dart's VM calls its
// platform's, so the last bit of the double may differ (the float result
// almost never does).
void orc_silu_mul(float* g, const float* u, int64_t count) {
  for (int64_t j = 0; j < count; j++) {
    const double a = g[j];
    const float s = (float)(a / (1.0 + exp(-a)));
    g[j] = (float)((double)s * (double)u[j]);
  }
}

// Abramowitz-Stegun 7.1.26 erf in double (lib/src/vision_encoder.dart:496-509).
static double as_erf(double value) {
  const double x = value < 0 ? -value : value;
  const double t = 1 / (1 + 0.3275911 * x);
  const double polynomial =
      (((((1.061405429 * t - 1.453152027) * t) + 1.421413741) * t - 0.284496736) * t +
       0.254829592) *
      t;
  const double result = 1 - polynomial * exp(-x * x);
  return value < 0 ? -result : result;
}

// The projector's exact-erf GELU (lib/src/vision_encoder.dart:260-263):
// v = 0.5 * v * (1 + erf(v / sqrt2)) in double, stored to float32.
void orc_gelu(float* x, int64_t count) {
  for (int64_t i = 0; i < count; i++) {
    const double v = x[i];
    x[i] = (float)(0.5 * v * (1 + as_erf(v / 1.4142135623730951)));
  }
}

// ------------------------------------------------------------ layer steps
//
// The decoder's other GPU steps as the reference's Metal shaders define them
// (src/metal/lab_metal.m:321-579): element values in float, in the shaders'
// order; sums in double (any GPU summation order rounds within a few ulp of
// the double sum, which is what the tests compare against with a tolerance).

// RMSNorm (lab_metal.m:327-347): r = 1 / sqrt(sum(x^2) / cols + eps) in
// float; y = w * (x * r); accumulate adds into out.
void orc_rms_norm(const float* x, const float* w, float* out, int64_t rows, int64_t cols,
                  float eps, int accumulate) {
  for (int64_t r = 0; r < rows; r++) {
    const float* xr = x + r * cols;
    float* yr = out + r * cols;
    double sum = 0.0;
    for (int64_t j = 0; j < cols; j++) sum += (double)(xr[j] * xr[j]);
    const float rr = 1.0f / sqrtf((float)sum / (float)cols + eps);
    for (int64_t j = 0; j < cols; j++) {
      const float v = w[j] * (xr[j] * rr);
      yr[j] = accumulate ? yr[j] + v : v;
    }
  }
}

// Per head and token, in place (lab_metal.m:357-380): RMSNorm over hd, then
// the half-split RoPE: (n1, n2) -> (n1 c - n2 s, n2 c + n1 s).
void orc_head_norm_rope(float* x, int64_t x_stride, const float* w, const float* rope,
                        int64_t rope_stride, int64_t heads, int64_t hd, int64_t n, float eps) {
  const int64_t pair = hd / 2;
  for (int64_t t = 0; t < n; t++) {
    const float* table = rope + t * rope_stride;
    for (int64_t h = 0; h < heads; h++) {
      float* xh = x + t * x_stride + h * hd;
      double sum = 0.0;
      for (int64_t j = 0; j < pair; j++) {
        sum += (double)(xh[j] * xh[j] + xh[j + pair] * xh[j + pair]);
      }
      const float r = 1.0f / sqrtf((float)sum / (float)hd + eps);
      for (int64_t j = 0; j < pair; j++) {
        const float x1 = xh[j], x2 = xh[j + pair];
        const float n1 = w[j] * (x1 * r), n2 = w[j + pair] * (x2 * r);
        const float c = table[j], s = table[pair + j];
        xh[j] = n1 * c - n2 * s;
        xh[j + pair] = n2 * c + n1 * s;
      }
    }
  }
}

// The gated short convolution (lab_metal.m:383-412), exactly the shader's
// per-channel loop (it has no reduction to reorder).
void orc_short_conv(const float* bcx, const float* weight, float* history, float* y,
                    int64_t width, int64_t k, int64_t n) {
  for (int64_t ch = 0; ch < width; ch++) {
    const float* kw = weight + ch * k;
    float past[16];
    for (int64_t r = 0; r + 1 < k; r++) past[r] = history[r * width + ch];
    for (int64_t t = 0; t < n; t++) {
      const float* row = bcx + t * 3 * width;
      const float z = row[ch] * row[2 * width + ch];
      float acc = kw[k - 1] * z;
      for (int64_t s = 1; s < k; s++) acc += kw[k - 1 - s] * past[k - 1 - s];
      y[t * width + ch] = row[width + ch] * acc;
      for (int64_t r = 0; r + 2 < k; r++) past[r] = past[r + 1];
      if (k >= 2) past[k - 2] = z;
    }
    for (int64_t r = 0; r + 1 < k; r++) history[r * width + ch] = past[r];
  }
}

// Causal attention (lab_metal.m:414-521; host side :1100-1127): scale =
// (float)(1 / sqrt(hd)); per (head, token) scores against the visible keys,
// softmax with exp(s - max), the value sum divided by the exponentials'
// sum, times sigmoid(gate) when gate is not null. Dots and sums in double.
void orc_attention(const float* q, const float* keys, const float* values, const float* gate,
                   float* out, int64_t position, int64_t n, int64_t heads, int64_t kv_heads,
                   int64_t hd, int64_t window) {
  const int64_t kv_dim = kv_heads * hd, group = heads / kv_heads;
  const float scale = (float)(1.0 / sqrt((double)hd));
  float* scores = (float*)malloc((size_t)(position + n) * sizeof(float));
  for (int64_t t = 0; t < n; t++) {
    const int64_t pos = position + t;
    const int64_t start = window > 0 && pos >= window ? pos - window + 1 : 0;
    const int64_t count = pos - start + 1;
    for (int64_t h = 0; h < heads; h++) {
      const float* qh = q + (t * heads + h) * hd;
      const int64_t kvo = h / group * hd;
      float m = -INFINITY;
      for (int64_t i = 0; i < count; i++) {
        const float* kr = keys + (start + i) * kv_dim + kvo;
        double d = 0.0;
        for (int64_t c = 0; c < hd; c++) d += (double)qh[c] * (double)kr[c];
        scores[i] = (float)d * scale;
        if (scores[i] > m) m = scores[i];
      }
      double sum = 0.0;
      for (int64_t i = 0; i < count; i++) {
        scores[i] = expf(scores[i] - m);
        sum += scores[i];
      }
      const float g = gate ? 1.0f / (1.0f + expf(-gate[t * heads + h])) : 1.0f;
      for (int64_t d = 0; d < hd; d++) {
        double acc = 0.0;
        for (int64_t i = 0; i < count; i++) {
          acc += (double)scores[i] * (double)values[(start + i) * kv_dim + kvo + d];
        }
        const float o = (float)acc / (float)sum;
        out[(t * heads + h) * hd + d] = gate ? o * g : o;
      }
    }
  }
  free(scores);
}

// The control vector (lab_metal.m:531-557): mode 0 adds v to each row;
// mode 1 computes c = scale * (x . v) and x -= c v.
void orc_steer(float* x, const float* v, int64_t rows, int64_t cols, int64_t mode, float scale) {
  for (int64_t r = 0; r < rows; r++) {
    float* xr = x + r * cols;
    if (mode == 0) {
      for (int64_t j = 0; j < cols; j++) xr[j] = xr[j] + v[j];
      continue;
    }
    double along = 0.0;
    for (int64_t j = 0; j < cols; j++) along += (double)(xr[j] * v[j]);
    const float c = scale * (float)along;
    for (int64_t j = 0; j < cols; j++) xr[j] = xr[j] - c * v[j];
  }
}
