// The product route of one matmul command: which kernels
// lab_gpu_enc_matmul_q8 / _q4 (lib/src/gpu.dart:137-190, encoded by
// GpuLinear.apply :1327-1341) run for its format, input mode, token count
// and shape. Shared by the lab_gpu_* command recorder (lab_gpu.hip) and the
// dnx_matmul_* device-pointer entry points (matmul.hip), so both always take
// the same path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dnx_kernels.h"

namespace dnx {

// Kernel launches of a route, reported to the caller's hook after each one.
enum class MatmulStep { kGemvFloat, kGemmFloat, kGemv, kQuantize, kGemm, kQuantizeF6, kGemmF6 };

inline int64_t align256(int64_t v) { return (v + 255) & ~(int64_t)255; }

// The fp6-MFMA GEMM wins over quantize + int8-MFMA GEMM only at large
// prefill shapes: its 128-token x 96-row tiles and 16-block stages cost a
// fixed ~5 us more (measured, graph-timed: at 768-2304 rows it loses at every
// n <= 512; at 6144 x 2048 it wins from about 375 tokens: 26.0 against 29.6 us,
// 512 tokens 29.2 against 32.6 us).
inline bool matmul_uses_f6(bool q4, int64_t rows, int64_t cols, int64_t n) {
  return q4 && n >= 320 && rows >= 4096 && cols <= 4096;
}

// A prefill chunk (the reference prefills in chunks of up to 64 tokens,
// lib/src/model.dart:91) or another batch of up to 512 tokens of a Q4
// matrix that the tiled fp6 route above does not take (the audio encoder's
// 375 frames, the callers' 128 and 256): with a prepacked copy of the
// weights (the lab_gpu_* command buffer keeps one per weight region) it runs
// as the f6 panel quantizer + dnx_gemm_q4_f6s, one launch over the whole K.
// Measured against quantize + int8 GEMM (graph-timed): 6144 x 2048 at 8..64
// tokens 7.5-9.4 against 11.0-15.1 us, at 128 / 256 tokens 14.7 / 20.7
// against 18.1 / 23.0; the audio shapes at 375 tokens 8.1-16.4 against
// 11.7-19.2.
inline bool matmul_uses_f6_chunk(bool q4, int64_t rows, int64_t cols, int64_t n) {
  return q4 && n >= 5 && n <= 512 && !matmul_uses_f6(q4, rows, cols, n);
}

// Q8 batches (the vision encoder's attention projections, fc1 / fc2 and
// projector at its 1024 patches, lib/src/vision_encoder.dart:252-316) with
// a prepacked copy of the weights (the lab_gpu_* command buffer keeps one
// per weight region): the int8 panel quantizer + dnx_gemm_q8_i8p.
// Measured against quantize + int8 GEMM (graph-timed, weights rotated past
// the MALL): 1152 x 4320 and 4320 x 1152 at 1024 tokens 32.0-33.1 /
// 26.3-27.1 against 41.9-42.6 / 29.3-30.1 us, 4096 x 4096 at 1024 tokens
// 53.1-53.7 against 78.3-84.7, 1152 x 1152 at 1024 tokens 14.5 against
// 17.3, 1024 x 1024 at 256 / 512 / 1024 tokens 11.6 / 13.9 / 13.0-13.9
// against 12.5 / 14.6 / 14.4-14.9, 768 x 768 at 512 tokens 12.3 against
// 13.6. Below 256 tokens or 2^28 multiply-adds the int8 GEMM's smaller
// tiles win or tie (1024 x 1024 and 2048 x 2048 at 128 tokens: 10.2 / 14.0
// against 10.0 / 13.4); one shape inside the bounds measured slower (4096
// x 1024 at 256 tokens, K of 32 blocks: 13.8 against 12.8).
inline bool matmul_uses_i8p(bool q4, int64_t rows, int64_t cols, int64_t n) {
  return !q4 && n >= 256 && rows * cols * n >= (1ll << 28);
}

// Device bytes a route needs for its quantized activations: int8 xq and fp32
// block scales (each 256-byte aligned), or the fp6 activation panel.
inline int64_t matmul_workspace_bytes(int64_t cols, int64_t n) {
  if (cols <= 0 || n <= 0 || cols % 32 != 0) return -1;
  const int64_t q8 = align256(n * cols) + align256(n * (cols / 32) * 4);
  const int64_t f6 = dnx_f6_panel_bytes(n, cols);
  return q8 > f6 ? q8 : f6;
}

// int8_inputs (mode 1, lab_native.c:553-579, :1059-1080): n <= 4 runs the
// exact GEMV (its prologue quantizes x); wider n, or an x too wide for the
// GEMV's LDS, quantizes x into the workspace and runs a GEMM. Float inputs
// (mode 0): n <= 4 the exact float-input GEMV; wider n, or an x too wide for
// the GEMV's LDS, the bf16-MFMA float GEMM (fp32 rounding of the CPU's).
// after(step) follows every successful launch. Returns the first error.
template <class After>
int matmul_route(bool q4, const void* qs, const void* scales, const float* x, float* y,
                 int64_t rows, int64_t cols, int64_t n, bool int8_inputs, void* workspace,
                 int64_t workspace_bytes, hipStream_t stream, After&& after) {
  auto s = (dnx_stream_t)stream;
  int rc;
  if (!int8_inputs) {
    if (n <= 4) {
      rc = q4 ? dnx_gemv_q4_float((const uint8_t*)qs, (const uint16_t*)scales, x, y, rows, cols,
                                  n, s)
              : dnx_gemv_q8_float((const int8_t*)qs, (const float*)scales, x, y, rows, cols, n, s);
      if (rc == DNX_OK) after(MatmulStep::kGemvFloat);
      if (rc != DNX_EINVAL) return rc;  // EINVAL: x too wide for the GEMV, nothing launched
    }
    rc = q4 ? dnx_gemm_q4_float((const uint8_t*)qs, (const uint16_t*)scales, x, y, rows, cols, n, s)
            : dnx_gemm_q8_float((const int8_t*)qs, (const float*)scales, x, y, rows, cols, n, s);
    if (rc == DNX_OK) after(MatmulStep::kGemmFloat);
    return rc;
  }
  if (n <= 4) {
    rc = q4 ? dnx_gemv_q4((const uint8_t*)qs, (const uint16_t*)scales, x, y, rows, cols, n, s)
            : dnx_gemv_q8((const int8_t*)qs, (const float*)scales, x, y, rows, cols, n, s);
    if (rc == DNX_OK) after(MatmulStep::kGemv);
    if (rc != DNX_EINVAL) return rc;  // EINVAL: x too wide for the GEMV, nothing launched
  }
  const int64_t need = matmul_workspace_bytes(cols, n);
  if (need < 0 || workspace == nullptr || workspace_bytes < need) return DNX_EINVAL;
  // The fp6 panel quantizer reads x 16 bytes at a time; an x that is only
  // 4-byte aligned (a float offset into a caller's buffer) takes the int8
  // route below, which reads it a float at a time where it must.
  if (matmul_uses_f6(q4, rows, cols, n) && ((uintptr_t)x & 15) == 0) {
    rc = dnx_quantize_q8_f6panel(x, workspace, n, cols, s);
    if (rc != DNX_OK) return rc;
    after(MatmulStep::kQuantizeF6);
    rc = dnx_gemm_q4_f6((const uint8_t*)qs, (const uint16_t*)scales, workspace, y, rows, cols, n,
                        s);
    if (rc == DNX_OK) after(MatmulStep::kGemmF6);
    return rc;
  }
  int8_t* xq = (int8_t*)workspace;
  float* xs = (float*)((char*)workspace + align256(n * cols));
  rc = dnx_quantize_q8(x, xq, xs, n, cols, cols, s);
  if (rc != DNX_OK) return rc;
  after(MatmulStep::kQuantize);
  rc = q4 ? dnx_gemm_q4((const uint8_t*)qs, (const uint16_t*)scales, xq, xs, y, rows, cols, n, s)
          : dnx_gemm_q8((const int8_t*)qs, (const float*)scales, xq, xs, y, rows, cols, n, s);
  if (rc == DNX_OK) after(MatmulStep::kGemm);
  return rc;
}

}  // namespace dnx
