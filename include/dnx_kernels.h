// Device-pointer launchers of the MI355X (gfx950) quantized-linear kernels.
//
// These are the kernels behind the lab_gpu_* drop-in ABI (lab_gpu.h),
// exported for callers that already hold device memory and a HIP stream
// (the benchmark, the tests, an engine that keeps activations in HBM). All
// pointers are device pointers; every call only enqueues work on `stream`
// and returns DNX_OK or a negative error before anything is launched.
//
// Layouts are the reference engine's (lab_native.c:398-405, :893-902):
//   Q8: qs int8 [rows][cols] row-major, scales fp32 [rows][cols/32]
//   Q4: qs uint8 [rows][cols/2] (weight k of a block = low nibble of byte k,
//       weight k+16 = high nibble), scales IEEE fp16 bits [rows][cols/32]
//   x fp32 [n][cols], y fp32 [n][rows] (ys[t*rows + r], lab_native.c:547-552)
#pragma once

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* dnx_stream_t;  // a hipStream_t

enum {
  DNX_OK = 0,
  DNX_EINVAL = -1,   // shape or argument outside what the kernel supports
  DNX_ELAUNCH = -2,  // the HIP launch failed
  DNX_ENOMEM = -3,   // a scratch allocation failed
  DNX_ESCRATCH = -4, // the call needs more than the fixed scratch array holds
};

// Up to DNX_COPY_MAX byte copies (src[i] -> dst[i], bytes[i] each) in one
// launch on `stream`; a destination may be pinned host memory
// (hipHostMalloc), which the kernel writes directly. No counterpart in the
// reference: the lab_gpu_* recorder copies a commit's written regions back
// to their host views with it (one launch instead of one copy per region).
// Regions are copied concurrently: destinations must not overlap each other
// or any source. The arrays are read on the host at the call.
enum { DNX_COPY_MAX = 96 };
int dnx_copy_regions(const void* const* src, void* const* dst, const int64_t* bytes, int count,
                     dnx_stream_t stream);

// lab_quantize_q8 (lab_native.c:407-429) on the GPU, bit-exact: rows x cols
// fp32 -> int8 [rows][cols_pad] + fp32 scales [rows][cols_pad/32]. cols_pad
// is a multiple of 32 >= cols; the values past cols are zero padding (the
// extension that lets K = 4304 run as 4320).
int dnx_quantize_q8(const float* x, int8_t* qs, float* scales, int64_t rows, int64_t cols,
                    int64_t cols_pad, dnx_stream_t stream);

// The BF16 load-time weight quantizer: _widenBf16 (safetensors.dart:207-212)
// then lab_quantize_q8, fused; bit-exact with that CPU pair. Same padding.
int dnx_quantize_q8_bf16(const uint16_t* w, int8_t* qs, float* scales, int64_t rows,
                         int64_t cols, int64_t cols_pad, dnx_stream_t stream);

// lab_quantize_q4 (lab_native.c:928-955) on the GPU, bit-exact: rows x cols
// fp32 (cols a multiple of 32, as NativeQ4Matrix.quantize requires,
// native.dart:793-796) -> Q4 nibbles
// [rows][cols/2] (byte k: weight k low, weight k + 16 high) + fp16 scale
// bits [rows][cols/32]. The load-time quantizer of Q4 weights.
int dnx_quantize_q4(const float* w, uint8_t* qs, uint16_t* scales, int64_t rows, int64_t cols,
                    dnx_stream_t stream);

// _widenBf16 (safetensors.dart:207-212) then lab_quantize_q4, fused;
// bit-exact with that CPU pair.
int dnx_quantize_q4_bf16(const uint16_t* w, uint8_t* qs, uint16_t* scales, int64_t rows,
                         int64_t cols, dnx_stream_t stream);

// The Q6_K -> Q8 embedding / LM-head adapter (lib/src/gguf.dart:402-414):
// dequantizeQ6K (:220-254) then lab_quantize_q8, fused and bit-exact with
// that pair. `blocks` holds rows x cols/256 Q6_K super-blocks of 210 bytes,
// row after row (cols a multiple of 256); out: int8 [rows][cols] + fp32
// scales [rows][cols/32], the engine's Q8 layout.
int dnx_q6k_to_q8(const void* blocks, int8_t* qs, float* scales, int64_t rows, int64_t cols,
                  dnx_stream_t stream);

// Decode GEMV, n <= 4 tokens, fp32 x quantized in the kernel's prologue:
// lab_gemm_q8 / lab_gemm_q4 mode 1 (lab_native.c:553-579, :1059-1080) with
// the CPU's exact float order, so y is bit-identical to theirs.
int dnx_gemv_q8(const int8_t* qs, const float* scales, const float* x, float* y, int64_t rows,
                int64_t cols, int64_t n, dnx_stream_t stream);
int dnx_gemv_q4(const uint8_t* qs, const uint16_t* scales, const float* x, float* y,
                int64_t rows, int64_t cols, int64_t n, dnx_stream_t stream);

// Float-input products, any n: lab_gemm_q8 / lab_gemm_q4 mode 0
// (dot_q8_f32 lab_native.c:489-501, dot_q4_f32 :1013-1023, lab_gemm_q8
// :553-579), x used as given (not quantized), in the CPU's exact float order:
// y is bit-identical to theirs. One launch per group of up to 4 tokens
// (each reads the weights once); the group shrinks to 2 or 1 token when the
// group's fp32 x would not fit the workgroup's LDS: 160 KB for matrices of
// up to 16384 rows with x of 4096 columns or more (8-wave workgroups, one
// per CU), 64 KB otherwise. DNX_EINVAL when even one row does not fit: cols
// above about 35000 (about 14000 for more than 16384 rows).
int dnx_gemv_q8_float(const int8_t* qs, const float* scales, const float* x, float* y,
                      int64_t rows, int64_t cols, int64_t n, dnx_stream_t stream);
int dnx_gemv_q4_float(const uint8_t* qs, const uint16_t* scales, const float* x, float* y,
                      int64_t rows, int64_t cols, int64_t n, dnx_stream_t stream);

// The decode GEMV with the greedy argmax fused (argmaxToken, lib/src/
// sampler.dart:137-152, over y): writes y and the token index to *out.
// workspace: dnx_gemv_argmax_workspace_bytes() bytes, zero before its first
// use; every completed call leaves it zero again (the call's last kernel
// clears it). Calls sharing one workspace must not overlap. Two launches on
// `stream`: the GEMV, then a one-workgroup kernel that writes *out.
int64_t dnx_gemv_argmax_workspace_bytes(void);
int dnx_gemv_q8_argmax(const int8_t* qs, const float* scales, const float* x, float* y,
                       int64_t rows, int64_t cols, int64_t* out, void* workspace,
                       dnx_stream_t stream);
int dnx_gemv_q4_argmax(const uint8_t* qs, const uint16_t* scales, const float* x, float* y,
                       int64_t rows, int64_t cols, int64_t* out, void* workspace,
                       dnx_stream_t stream);

// An MLP's gate and up products and their glue in one pass over x
// (LayerShard.ffn, lib/src/shard.dart:455-461): h[t][r] = SiLU(g) * u with
// g = (W_gate x[t])[r], u = (W_up x[t])[r], each bit-identical to the GEMV
// above and SiLU in double as the Dart glue computes it. u, when not null,
// also receives the up products. n <= 4.
int dnx_gate_up_q8(const int8_t* gate_qs, const float* gate_scales, const int8_t* up_qs,
                   const float* up_scales, const float* x, float* h, float* u, int64_t rows,
                   int64_t cols, int64_t n, dnx_stream_t stream);
int dnx_gate_up_q4(const uint8_t* gate_qs, const uint16_t* gate_scales, const uint8_t* up_qs,
                   const uint16_t* up_scales, const float* x, float* h, float* u, int64_t rows,
                   int64_t cols, int64_t n, dnx_stream_t stream);

// The same three for Q8 weights whose block scales are kept as the GGUF Q8_0
// block's own fp16 d (gguf.dart:270-282 widens it to fp32 exactly): scales
// uint16 [rows][cols/32]. Bit-identical to the fp32-scale calls on the
// widened scales, with 34 instead of 36 bytes streamed per 32 weights.
int dnx_gemv_q8h(const int8_t* qs, const uint16_t* scales, const float* x, float* y,
                 int64_t rows, int64_t cols, int64_t n, dnx_stream_t stream);
int dnx_gemv_q8h_argmax(const int8_t* qs, const uint16_t* scales, const float* x, float* y,
                        int64_t rows, int64_t cols, int64_t* out, void* workspace,
                        dnx_stream_t stream);
int dnx_gate_up_q8h(const int8_t* gate_qs, const uint16_t* gate_scales, const int8_t* up_qs,
                    const uint16_t* up_scales, const float* x, float* h, float* u, int64_t rows,
                    int64_t cols, int64_t n, dnx_stream_t stream);

// Up to 4 decode GEMVs over the same x in one launch (one token, int8
// inputs): y[i] = W_i x for i < segs, W_i with rows[i] rows of cols columns
// at qs[i] / scales[i], each y[i] bit-identical to dnx_gemv_*(W_i, x) (the
// attention projections q, k, v and gate of GpuForward.forward, lib/src/
// gpu.dart:1148-1156, read the same normed x). x is quantized once for all.
// The pointer arrays are read on the host at the call.
int dnx_gemv_multi_q8(const int8_t* const* qs, const float* const* scales, float* const* y,
                      const int64_t* rows, int segs, const float* x, int64_t cols,
                      dnx_stream_t stream);
int dnx_gemv_multi_q4(const uint8_t* const* qs, const uint16_t* const* scales, float* const* y,
                      const int64_t* rows, int segs, const float* x, int64_t cols,
                      dnx_stream_t stream);
int dnx_gemv_multi_q8h(const int8_t* const* qs, const uint16_t* const* scales, float* const* y,
                       const int64_t* rows, int segs, const float* x, int64_t cols,
                       dnx_stream_t stream);

// One-token GEMV with the residual add of its output in the epilogue
// (GpuForward adds each block's output into x, gpu.dart:1180-1187): y is
// dnx_gemv_*'s output and then resid[r] = resid[r] + y[r] (the bits of
// dnx_add(y, resid, rows) after the GEMV). resid must not overlap x or y
// (DNX_EINVAL, nothing launched).
int dnx_gemv_add_q8(const int8_t* qs, const float* scales, const float* x, float* y,
                    float* resid, int64_t rows, int64_t cols, dnx_stream_t stream);
int dnx_gemv_add_q4(const uint8_t* qs, const uint16_t* scales, const float* x, float* y,
                    float* resid, int64_t rows, int64_t cols, dnx_stream_t stream);

// One-token GEMVs over the RMSNorm of x (GpuForward norms x before each
// block, gpu.dart:1145-1156, :1180-1185): norm_out = dnx_rms_norm(x, norm_w,
// eps) of the one row, bit for bit, and the products are those of the GEMVs
// on norm_out: the gate/up pair and glue of dnx_gate_up_* (h, u), or the
// segmented launch of dnx_gemv_multi_* (y[i]). Every workgroup norms x in its
// prologue; workgroup 0 writes norm_out at its end. cols % 32 == 0 and
// cols <= 8192; x, norm_w and norm_out 16-byte aligned; norm_out disjoint
// from x and norm_w (DNX_EINVAL otherwise, nothing launched). The outputs
// must not overlap x, norm_w or norm_out.
int dnx_gate_up_norm_q8(const int8_t* gate_qs, const float* gate_scales, const int8_t* up_qs,
                        const float* up_scales, const float* x, const float* norm_w,
                        float* norm_out, float eps, float* h, float* u, int64_t rows,
                        int64_t cols, dnx_stream_t stream);
int dnx_gate_up_norm_q4(const uint8_t* gate_qs, const uint16_t* gate_scales, const uint8_t* up_qs,
                        const uint16_t* up_scales, const float* x, const float* norm_w,
                        float* norm_out, float eps, float* h, float* u, int64_t rows,
                        int64_t cols, dnx_stream_t stream);
int dnx_gemv_multi_norm_q8(const int8_t* const* qs, const float* const* scales, float* const* y,
                           const int64_t* rows, int segs, const float* x, const float* norm_w,
                           float* norm_out, float eps, int64_t cols, dnx_stream_t stream);
int dnx_gemv_multi_norm_q4(const uint8_t* const* qs, const uint16_t* const* scales,
                           float* const* y, const int64_t* rows, int segs, const float* x,
                           const float* norm_w, float* norm_out, float eps, int64_t cols,
                           dnx_stream_t stream);

// Float-input GEMM (lab_gemm_q8 / lab_gemm_q4 mode 0 for many tokens,
// lab_native.c:489-501, :1013-1023; the reference's float GPU GEMMs,
// lab_metal.m:79-144, :174-258) on bf16 MFMA: x (fp32 [n][cols]) split
// exactly into three bf16 pieces, weights exact in bf16, so every product
// is exact and only the fp32 summation order differs from the CPU's (within
// 1e-4 relative, not bit-identical; the same inputs always give the same
// bits). Any n and cols % 32 == 0; qs 16-byte aligned. When the tiles alone
// would leave CUs idle, K is split and a second kernel sums the partials in
// a fixed order, in a workspace the library owns (grown on the first call
// at a larger shape: not the first call inside a graph capture).
int dnx_gemm_q8_float(const int8_t* qs, const float* scales, const float* x, float* y,
                      int64_t rows, int64_t cols, int64_t n, dnx_stream_t stream);
int dnx_gemm_q4_float(const uint8_t* qs, const uint16_t* scales, const float* x, float* y,
                      int64_t rows, int64_t cols, int64_t n, dnx_stream_t stream);

// Prefill / encoder GEMM on int8 MFMA, any n, inputs already quantized
// (xq int8 [n][cols], xsc fp32 [n][cols/32], e.g. by dnx_quantize_q8):
// the per-32-block int32 dots are exact, the per-block scaling is fp32
// (within 1e-4 relative of the CPU kernels, not bit-identical; the same
// inputs always give the same bits). When n is small (fewer than 256 output
// tiles) K is split across workgroups and a second kernel sums the partials
// in a fixed order; their workspace is the library's own, allocated on the
// first such call at a larger shape (so that call must not be captured into
// a graph).
int dnx_gemm_q8(const int8_t* qs, const float* scales, const int8_t* xq, const float* xsc,
                float* y, int64_t rows, int64_t cols, int64_t n, dnx_stream_t stream);
int dnx_gemm_q4(const uint8_t* qs, const uint16_t* scales, const int8_t* xq, const float* xsc,
                float* y, int64_t rows, int64_t cols, int64_t n, dnx_stream_t stream);

// The large-n GEMM on fp16/bf16 MFMA (exact int block dots, scale products
// from an outer-product MFMA, one fma per output per block), on activations
// laid out as a "panel": per 32 token rows and per 32-block, 2048 bytes of
// fp16 MFMA fragments of xq and 512 bytes of bf16 pieces of xsc.
// dnx_gemm_panel_bytes(n, cols) is its size; dnx_pack_panel writes it from
// xq int8 [n][cols] and xsc fp32 [n][cols/32]. The products are within 1e-4
// relative of the CPU kernels (the same inputs always give the same bits).
// With fewer than 192 output tiles K is split across workgroups and summed
// in a fixed order in the library's own workspace, allocated on the first
// such call at a larger shape (so that call must not be captured into a
// graph).
int64_t dnx_gemm_panel_bytes(int64_t n, int64_t cols);
int dnx_pack_panel(const int8_t* xq, const float* xsc, void* panel, int64_t n, int64_t cols,
                   dnx_stream_t stream);
// lab_quantize_q8 of fp32 x [n][cols] written straight into the panel (the
// same quantized values as dnx_quantize_q8; x 16-byte aligned).
int dnx_quantize_q8_panel(const float* x, void* panel, int64_t n, int64_t cols,
                          dnx_stream_t stream);
int dnx_gemm_q8_panel(const int8_t* qs, const float* scales, const void* panel, float* y,
                      int64_t rows, int64_t cols, int64_t n, dnx_stream_t stream);
int dnx_gemm_q4_panel(const uint8_t* qs, const uint16_t* scales, const void* panel, float* y,
                      int64_t rows, int64_t cols, int64_t n, dnx_stream_t stream);

// The large-n Q4 GEMM on the fp6 matrix cores (lab_gemm_q4 mode 1,
// lab_native.c:1059-1080): each block's exact int dot from one scaled
// v_mfma_scale_f32_32x32x64_f8f6f4 (weights as the E2M3 codes of q / 8,
// activations as two E2M3 pieces of xq with power-of-two scales, the -8 of
// q - 8 as the MFMA's C input), the scale products from an fp16
// outer-product MFMA, one fma per output per block. The activations arrive
// as an "f6 panel" (per 32 tokens and block, the MFMA operands in lane
// order); dnx_f6_panel_bytes(n, cols) is its size. dnx_quantize_q8_f6panel
// writes it from fp32 x [n][cols] (lab_quantize_q8's values, bit-exact with
// dnx_quantize_q8; x 16-byte aligned), dnx_pack_f6panel from xq int8
// [n][cols] + xsc fp32 [n][cols/32]. The products are within 1e-4 relative
// of the CPU kernels; the same inputs always give the same bits. With 128
// workgroup tiles (128 tokens x 96 rows) or fewer K is split across
// workgroups and summed in a fixed order in a library-owned workspace,
// allocated on the first such call at a larger shape (so that call must not
// be captured into a graph).
int64_t dnx_f6_panel_bytes(int64_t n, int64_t cols);
int dnx_quantize_q8_f6panel(const float* x, void* panel, int64_t n, int64_t cols,
                            dnx_stream_t stream);
int dnx_pack_f6panel(const int8_t* xq, const float* xsc, void* panel, int64_t n, int64_t cols,
                     dnx_stream_t stream);
int dnx_gemm_q4_f6(const uint8_t* qs, const uint16_t* scales, const void* panel, float* y,
                   int64_t rows, int64_t cols, int64_t n, dnx_stream_t stream);

// The same GEMM on a load-time re-encoding of the Q4 weights: per (row,
// block) 32 bytes holding the E2M3 codes of the signed weights q - 8 and the
// scale MFMA's operand, laid out tile-major (per 32-row group and block one
// 1 KB chunk; dnx_q4_f6pack_bytes(rows, cols) bytes, written once by
// dnx_pack_q4_f6 from the engine's Q4 layout; weights are immutable after
// upload, as GpuLinear.upload treats them, gpu.dart:1295-1323). The GEMM
// moves the chunks into LDS by DMA and needs no per-call conversion of the
// weights; results are bit-identical to dnx_gemm_q4_f6's (the same K split
// and order).
int64_t dnx_q4_f6pack_bytes(int64_t rows, int64_t cols);
int dnx_pack_q4_f6(const uint8_t* qs, const uint16_t* scales, void* packed, int64_t rows,
                   int64_t cols, dnx_stream_t stream);
int dnx_gemm_q4_f6p(const void* packed, const void* panel, float* y, int64_t rows, int64_t cols,
                    int64_t n, dnx_stream_t stream);

// The same GEMM for Q8 weights (lab_gemm_q8 mode 1, lab_native.c:553-579):
// a load-time re-encoding of the engine's Q8 layout (int8 + fp32 scale per
// block) into two fp6 digit planes, |w| = 8 wh + wl, and the scale split into
// its E8M0 exponent and two fp16 mantissa pieces, tile-major
// (dnx_q8_f6pack_bytes(rows, cols) bytes, 2.5 KB per 32-row group and block,
// written once by dnx_pack_q8_f6). Two dot MFMAs per block, chained exactly;
// the same activation panel as the Q4 GEMMs (dnx_quantize_q8_f6panel).
// Exact block dots (int8 weights including -128), fp32 within 1e-4 relative
// (1e-5 absolute near zero) of the CPU kernel, for finite weight scales
// (an infinite or NaN scale has no E8M0 + mantissa form; the int8 GEMM,
// dnx_gemm_q8, propagates them as the CPU does). Not the matmul route's
// choice for Q8: measured slower than the int8 GEMM at the vision shapes.
int64_t dnx_q8_f6pack_bytes(int64_t rows, int64_t cols);
int dnx_pack_q8_f6(const int8_t* qs, const float* scales, void* packed, int64_t rows,
                   int64_t cols, dnx_stream_t stream);
int dnx_gemm_q8_f6p(const void* packed, const void* panel, float* y, int64_t rows, int64_t cols,
                    int64_t n, dnx_stream_t stream);

// The Q8 GEMM (lab_gemm_q8 mode 1, lab_native.c:553-579, :1059-1080; the
// vision encoder's fc1 / fc2, lib/src/vision_encoder.dart:275-316) on the
// int8 matrix cores, one v_mfma_i32_32x32x32_i8 per block (exact int32 block
// dots), the scale products from a bf16 outer-product MFMA, cvt + fma per
// output and block. Both operands in fragment order, 1536 bytes per 32 rows
// (or tokens) and block: the weights re-encoded once at load
// (dnx_q8_i8pack_bytes, dnx_pack_q8_i8), the activations quantized from fp32
// x with lab_quantize_q8's xq and scale bits (dnx_i8_panel_bytes,
// dnx_quantize_q8_i8panel; x and the panel 16-byte aligned). fp32 within
// 1e-4 relative (1e-5 absolute near zero) of the CPU kernel; the scales are
// applied as by dnx_gemm_q8. Tiles of 128 tokens x 96, 128 or 160 rows or
// 64 tokens x 96 or 128 rows (dnx_gemm_q8_i8p_tile: the choice for a shape,
// DNX_EINVAL for a shape the GEMM refuses); at 128 tiles or fewer K is split, the partials added in a
// fixed order in a second launch, from the fp6 GEMMs' library-owned
// workspace, grown on demand (the first call at a larger split shape
// allocates, so it must not be captured into a graph; calls share it:
// serialize them on one GPU).
int64_t dnx_i8_panel_bytes(int64_t n, int64_t cols);
int dnx_quantize_q8_i8panel(const float* x, void* panel, int64_t n, int64_t cols,
                            dnx_stream_t stream);
int64_t dnx_q8_i8pack_bytes(int64_t rows, int64_t cols);
int dnx_pack_q8_i8(const int8_t* qs, const float* scales, void* packed, int64_t rows,
                   int64_t cols, dnx_stream_t stream);
int dnx_gemm_q8_i8p(const void* packed, const void* panel, float* y, int64_t rows, int64_t cols,
                    int64_t n, dnx_stream_t stream);
int dnx_gemm_q8_i8p_tile(int64_t rows, int64_t cols, int64_t n, int* tile_rows,
                         int* tile_tokens);

// The prefill chunk GEMM (lab_gemm_q4 mode 1, lab_native.c:1059-1080, at
// the reference's prefill chunks of up to 64 tokens, lib/src/model.dart:91,
// and other batches of a few hundred tokens) on prepacked weights: one
// launch over the whole K (no split partials, no reduce launch), a
// workgroup per 32 rows and 32 to 96 tokens (more tokens, more
// workgroups); exact block dots, fp32 within 1e-4 relative (1e-5 absolute
// near zero) of the CPU kernel. Deterministic (a fixed order of the K
// parts, whatever the workgroup shape).
int dnx_gemm_q4_f6s(const void* packed, const void* panel, float* y, int64_t rows, int64_t cols,
                    int64_t n, dnx_stream_t stream);

// The same chunk GEMM over 1..4 prepacked matrices of one width that read
// the same panel (a prefill chunk's q, k and v projections, or its gate and
// up), in one launch: y[k] = x W[k]^T, each bit-identical to its own
// dnx_gemm_q4_f6s. No reference counterpart (the reference encodes one
// dispatch per matmul); the lab_gpu_* command buffer uses it for
// consecutive prefill matmuls of one x.
int dnx_gemm_q4_f6s_multi(const void* const* packed, float* const* y, const int64_t* rows,
                          int count, const void* panel, int64_t cols, int64_t n,
                          dnx_stream_t stream);

// dnx_gemm_q4_f6p without any allocation. No counterpart in the reference:
// for callers that cannot allocate device memory (code under HIP graph
// capture, serving loops, harnesses that forbid hipMalloc). Same kernels and
// the same bits as dnx_gemm_q4_f6p; its split-K partials live in a fixed
// 21 MiB array in the library's code object (one per GPU, held until the
// process ends) instead of the grown-on-demand workspace. A shape whose
// partials, splits x n x rows floats, exceed dnx_gemm_q4_f6p_noalloc_max_floats()
// returns DNX_ESCRATCH before anything is launched; with the current split
// policy (K split only below 192 tiles of 128 tokens x 96 rows) every valid
// shape fits. The
// first call on a device looks up that device's array address (make it
// outside a graph capture). Every call on one GPU shares its array: calls
// that overlap on one GPU race, so serialize them (one stream, or events).
int64_t dnx_gemm_q4_f6p_noalloc_max_floats(void);
int dnx_gemm_q4_f6p_noalloc(const void* packed, const void* panel, float* y, int64_t rows,
                            int64_t cols, int64_t n, dnx_stream_t stream);

// One matmul command's product route on device pointers: the kernels
// lab_gpu_enc_matmul_q8 / _q4 (lib/src/gpu.dart:137-190) run at commit, for
// engines that call the ABI's products without its command buffer.
// int8_inputs 1 (mode 1): n <= 4 the exact GEMV above (bit-identical to
// lab_gemm_* mode 1), else x quantized into `workspace` and a GEMM (the
// int8-MFMA GEMM; for Q4 at >= 320 tokens, >= 4096 rows and K <= 4096 the
// fp6-MFMA GEMM, which is faster there). int8_inputs 0 (mode 0): for n <= 4
// and x narrow enough for its LDS the exact float-input GEMV (bit-identical
// to lab_gemm_* mode 0), else the bf16-MFMA float GEMM (any width; within
// 1e-4 + 1e-5 |y| of mode 0). workspace: at least
// dnx_matmul_workspace_bytes(cols, n) bytes of device memory for the
// quantized activations (unused by the GEMV routes; may be null there).
// Split-K partials are not in it: when a GEMM splits K (few output tiles),
// its partials go to a buffer the library owns per GEMM kind and grows on
// demand (a hipMalloc after a device synchronize). So calls share library
// state: serialize them (one stream, or events between streams), and do
// not make the first call of a new, larger split shape inside a graph
// capture.
int64_t dnx_matmul_workspace_bytes(int64_t cols, int64_t n);
int dnx_matmul_q8(const int8_t* qs, const float* scales, const float* x, float* y, int64_t rows,
                  int64_t cols, int64_t n, int int8_inputs, void* workspace,
                  int64_t workspace_bytes, dnx_stream_t stream);
int dnx_matmul_q4(const uint8_t* qs, const uint16_t* scales, const float* x, float* y,
                  int64_t rows, int64_t cols, int64_t n, int int8_inputs, void* workspace,
                  int64_t workspace_bytes, dnx_stream_t stream);

// GGUF Q8_0 / Q4_0 blocks split into the engine's layout on the GPU, bit
// for bit as splitQ8_0 (lib/src/gguf.dart:270-282: int8 values and the fp16
// d widened to fp32) and splitQ4_0 (:208-218: nibble bytes and the fp16
// bits) do on the CPU. count = rows * cols / 32 blocks of 34 (Q8_0) or 18
// (Q4_0) bytes; blocks 4-byte aligned, qs 16-byte aligned.
int dnx_split_q8_0(const void* blocks, int8_t* qs, float* scales, int64_t count,
                   dnx_stream_t stream);
int dnx_split_q4_0(const void* blocks, uint8_t* qs, uint16_t* scales, int64_t count,
                   dnx_stream_t stream);

// Greedy argmax of v[0..n) (argmaxToken, lib/src/sampler.dart:137-152):
// the first index of the maximum; a NaN at index 0 wins, other NaNs never.
// Writes one int64 to *out. workspace: dnx_argmax_workspace_bytes(n) bytes.
int64_t dnx_argmax_workspace_bytes(int64_t n);
int dnx_argmax(const float* v, int64_t n, int64_t* out, void* workspace, dnx_stream_t stream);

// g = SiLU(g) * u in place (the glue of lib/src/shard.dart:457-461 and
// lab_gpu_enc_swiglu), SiLU in double as the Dart glue computes it.
int dnx_swiglu(float* g, const float* u, int64_t count, dnx_stream_t stream);

// Producers that also write the fp6 GEMMs' activation panel of their output
// (the bytes dnx_quantize_q8_f6panel would make from it: dnx_f6_panel_bytes(
// rows, cols), records of tokens past `rows` not written), so that the
// prefill matmuls reading that output skip the quantize launch. No
// reference counterpart; the lab_gpu_* command buffer uses them when the
// next commands are such matmuls. Outputs bit-identical to dnx_swiglu,
// dnx_rms_norm (accumulate 0) and dnx_add_rms_norm. The norms take up to 256
// rows of up to 8192 columns, a multiple of 32; every pointer 16-byte
// aligned.
int dnx_swiglu_f6panel(float* g, const float* u, void* panel, int64_t rows, int64_t cols,
                       dnx_stream_t stream);
int dnx_rms_norm_f6panel(const float* x, const float* w, float* out, void* panel, int64_t rows,
                         int64_t cols, float eps, dnx_stream_t stream);
int dnx_add_rms_norm_f6panel(const float* m, float* x, const float* w, float* out, void* panel,
                             int64_t rows, int64_t cols, float eps, dnx_stream_t stream);

// Exact-erf GELU in place with the Abramowitz-Stegun erf in double
// (lib/src/vision_encoder.dart:260-263, :496-509). x 4-byte aligned; any
// count and offset.
int dnx_gelu(float* x, int64_t count, dnx_stream_t stream);

// The decoder's other layer steps (the lab_gpu_enc_* encoders of
// lib/src/gpu.dart:179-312, semantics of src/metal/lab_metal.m:321-579),
// fp32, deterministic, equal to the reference's to fp32 rounding (their
// reductions run in another order). Pointers are device pointers.
//
// RMSNorm of `rows` rows of `cols` (lab_metal.m:327-347): out = w * (x * r),
// r = 1 / sqrt(mean(x^2) + eps); accumulate != 0 adds into out instead.
int dnx_rms_norm(const float* x, const float* w, float* out, int64_t rows, int64_t cols,
                 float eps, int accumulate, dnx_stream_t stream);
// Per head and token, in place: RMSNorm over hd (weight w), then the
// half-split RoPE from the token's tables [cos(hd/2), sin(hd/2)]
// (lab_metal.m:357-380). Strides in floats between tokens; hd even, <= 512.
int dnx_head_norm_rope(float* x, int64_t x_stride, const float* w, const float* rope,
                       int64_t rope_stride, int64_t heads, int64_t hd, int64_t n, float eps,
                       dnx_stream_t stream);
// Two dnx_head_norm_rope calls that share the rope table, hd, n and eps (a
// decode step's q and k, gpu.dart:1162-1163) in one launch; the two operands
// must not overlap. Bit-identical to the two calls.
int dnx_head_norm_rope2(float* x0, int64_t x0_stride, const float* w0, int64_t heads0,
                        float* x1, int64_t x1_stride, const float* w1, int64_t heads1,
                        const float* rope, int64_t rope_stride, int64_t hd, int64_t n, float eps,
                        dnx_stream_t stream);
// dnx_add(m, x, rows * cols) then dnx_rms_norm(x, w, out, rows, cols, eps, 0)
// in one launch (the residual add and the next norm of GpuForward.forward,
// gpu.dart:1180-1187): bit-identical to the pair. rows <= 256, cols a
// multiple of 4 up to 16384, 16-byte aligned operands, out not overlapping
// x or m (DNX_EINVAL otherwise, nothing launched).
int dnx_add_rms_norm(const float* m, float* x, const float* w, float* out, int64_t rows,
                     int64_t cols, float eps, dnx_stream_t stream);
// The gated short convolution over n tokens (lab_metal.m:383-412): bcx rows
// [B | C | X] of `width` each, weight [width][k] (k <= 16), history
// [k - 1][width] (oldest first, updated), y [n][width].
int dnx_short_conv(const float* bcx, const float* weight, float* history, float* y,
                   int64_t width, int64_t k, int64_t n, dnx_stream_t stream);
// Causal attention of n tokens at positions position.. over cached keys and
// values [positions][kv_heads * hd] (lab_metal.m:414-521), q and out
// [n][heads][hd], gate [n][heads] or null (ungated); window 0: every earlier
// position, else the last `window`. hd a multiple of 4 dividing 256; q and
// keys 16-byte aligned. 8+ tokens at hd 64 or 128 with a 16-byte aligned
// out run on the fp32 matrix cores; decode-shaped calls (fewer than 256
// head-token pairs, more than 256 keys) split the keys over workgroups.
// Both may add a combine pass over a library-owned workspace grown on
// demand: a first call at a larger shape allocates (not inside a graph
// capture), and calls that overlap (other streams, other threads) must not
// share the library. Otherwise at most dnx_attention_max_keys(hd) keys per
// token.
int64_t dnx_attention_max_keys(int64_t hd);
int dnx_attention(const float* q, const float* keys, const float* values, const float* gate,
                  float* out, int64_t position, int64_t n, int64_t heads, int64_t kv_heads,
                  int64_t hd, int64_t window, dnx_stream_t stream);
// dnx_attention, and the fp6 activation panel of out ([n][heads * hd], as
// dnx_quantize_q8_f6panel would write it from out) into `panel` (16-byte
// aligned, f6_panel_bytes(n, heads * hd) bytes) for the prefill matmul that
// reads out (the o projection, lab_gpu commit peephole; no counterpart in
// the reference). Only where the call takes the matrix-core path with its
// keys split over 2..64 workgroups (the row combine writes the panel) and hd
// is a multiple of 32; else DNX_EINVAL and nothing launched. Records of the
// panel's padding tokens (past n in its last group of 32) are left as they
// are: the chunk GEMM never reads them.
int dnx_attention_f6panel(const float* q, const float* keys, const float* values,
                          const float* gate, float* out, void* panel, int64_t position, int64_t n,
                          int64_t heads, int64_t kv_heads, int64_t hd, int64_t window,
                          dnx_stream_t stream);
// One decode token's q and k head norms + RoPE folded into its attention
// (gpu.dart:1157-1175: dnx_head_norm_rope of q with q_norm, of the token's
// key row keys[position] with k_norm, both with the table row `rope`
// [cos(hd / 2), sin(hd / 2)], then dnx_attention with n = 1): the same bits
// in out, in q (normed in place) and in keys[position] (normed in place).
// The split-key path only, with one workgroup per KV head (the query heads
// per KV head a power of two up to 8) and hd <= 256: DNX_EINVAL otherwise,
// nothing launched. out must not overlap q, keys or values.
int dnx_attention_rope(float* q, float* keys, const float* values, const float* gate, float* out,
                       int64_t position, int64_t heads, int64_t kv_heads, int64_t hd,
                       int64_t window, const float* q_norm, const float* k_norm,
                       const float* rope, float eps, dnx_stream_t stream);
// dst += src and dst = src over `count` floats (lab_metal.m:560-572).
int dnx_add(const float* src, float* dst, int64_t count, dnx_stream_t stream);
int dnx_copy(const float* src, float* dst, int64_t count, dnx_stream_t stream);
// A control vector on `rows` rows of `cols` (lab_metal.m:531-557): mode 0
// adds v; mode 1 removes scale * (x . v) v (v a unit direction).
int dnx_steer(float* x, const float* v, int64_t rows, int64_t cols, int64_t mode, float scale,
              dnx_stream_t stream);

#ifdef __cplusplus
}
#endif
