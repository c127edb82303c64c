// The reference's GPU C ABI (lab_gpu_*), implemented for one MI355X (gfx950)
// by libdianoia_amd.so. Dart binds these names with @Native in
// lib/src/gpu.dart:36-312 of the reference (Atrac613/dianoia); the Vulkan
// (src/vulkan/lab_vulkan.c) and Metal (src/metal/lab_metal.m) layers export
// the same signatures. Every handle, offset, size and count is int64_t.
//
// Model (as in the reference): one process-wide command buffer. Buffers have
// a host view (lab_gpu_contents) that the caller writes inputs into and reads
// outputs from. lab_gpu_enc_* record work; lab_gpu_commit submits it; each
// recorded dispatch sees every earlier one's writes. On this discrete GPU a
// buffer is a device allocation plus a pinned host shadow: commit uploads the
// host regions a dispatch reads (unless an earlier dispatch of the same
// command buffer wrote them; with host-write tracking, only their pages the
// host wrote since HBM last matched them), uploads a weight buffer once on
// its first use as weights (weights are immutable, as in GpuLinear.upload,
// gpu.dart:1295-1323), and copies every region a dispatch wrote back to the
// host before the commit completes. Tracking write-protects clean host pages
// and installs a SIGSEGV handler at lab_gpu_init that chains to the one
// installed before it.
//
// Not re-entrant: one thread drives the GPU layer at a time (gpu.dart:
// 1277-1278).
#pragma once

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// lab_gpu_init (lab_vulkan.c:295-296; gpu.dart:36-37): 1 when the GPU is
// ready, 0 when there is none (logged to stderr). Idempotent.
int64_t lab_gpu_init(void);

// lab_gpu_buffer (lab_vulkan.c:582-586; gpu.dart:63-64): a zeroed buffer of
// `bytes`, returning its handle (>= 0) or -1. Handles freed by
// lab_gpu_release are handed out again first; at most 4096 live.
int64_t lab_gpu_buffer(int64_t bytes);

// lab_gpu_readback_buffer (lab_vulkan.c:590-594; gpu.dart:66-67): the same,
// for buffers the host reads after every command buffer (logits).
int64_t lab_gpu_readback_buffer(int64_t bytes);

// lab_gpu_wrap (lab_vulkan.c:598-602; gpu.dart:69-73): a buffer holding a
// copy of `bytes` at `address` (the mapped weight cache), placed in HBM now.
// lab_gpu_wrap_copies (lab_vulkan.c:605; gpu.dart:75-76) returns 1: the
// wrapped memory may be evicted afterwards.
int64_t lab_gpu_wrap(void* address, int64_t bytes);
int64_t lab_gpu_wrap_copies(void);

// lab_gpu_contents (lab_vulkan.c:607; gpu.dart:78-79): the buffer's stable
// host pointer for its lifetime.
void* lab_gpu_contents(int64_t handle);

// lab_gpu_release / lab_gpu_live_buffers (lab_vulkan.c:637-652;
// gpu.dart:81-85): release waits for submitted work, then frees the handle.
// Internal scratch is not counted as a live buffer.
void lab_gpu_release(int64_t handle);
int64_t lab_gpu_live_buffers(void);

// lab_gpu_begin / commit / wait / last_ms (lab_vulkan.c:655-665, 737-767,
// 610; gpu.dart:111-123). commit(1) blocks until done; commit(0) returns
// at once and lab_gpu_wait blocks later. Both return 1 on success, 0 on
// failure (logged); a dispatch recorded with invalid arguments fails its
// commit. last_ms is the GPU time of the last waited command buffer.
void lab_gpu_begin(void);
int64_t lab_gpu_commit(int64_t wait);
int64_t lab_gpu_wait(void);
double lab_gpu_last_ms(void);

// Host-write tracking of the host views. No counterpart in the reference,
// whose host-visible memory needs no copies: the bytes this library has
// copied host -> HBM (commit uploads and first weight uploads) and HBM ->
// host (copy-backs) since lab_gpu_init, for callers that measure the PCIe
// cost of a command buffer (a decode step). lab_gpu_tracking_writes is 1
// while page-granular tracking is on (a commit then uploads only the pages
// the host wrote since HBM last matched them), 0 when it is off
// (DIANOIA_GPU_TRACK_WRITES=0, or another SIGSEGV handler replaced this
// library's; every read region is then uploaded).
void lab_gpu_transfer_bytes(int64_t* up, int64_t* down);
int64_t lab_gpu_tracking_writes(void);

// lab_gpu_enc_matmul_q8 / _q4 (lab_vulkan.c:877-890; gpu.dart:125-177):
// Y[n][rows] = X[n][cols] W^T, W inside buffer w at qsOffset / scalesOffset
// in the engine's Q8 (int8 + fp32 scales) or Q4 (nibbles + fp16 scales)
// layout, X at x + xOffset (fp32), Y at y + yOffset (fp32). By default the
// inputs are quantized to Q8 per block as lab_native.c does (mode 1): for
// n <= 4 (and x narrow enough for the GEMV's LDS) the products are
// bit-identical to lab_gemm_q8 / lab_gemm_q4 mode 1; otherwise a GEMM with
// exact per-block integer dots computes them within 1e-4 relative (1e-5
// absolute near zero). With float inputs (lab_gpu_set_int8_inputs below):
// for n <= 4 and x narrow enough for the GEMV (one token's fp32 x fits its
// LDS up to about 35000 columns; 14000 above 16384 rows), bit-identical to
// mode 0; otherwise the bf16-MFMA float GEMM, any width, within
// 1e-4 + 1e-5 |y| of mode 0 (the reference GPU test's bar). qs must be
// 16-byte aligned.
void lab_gpu_enc_matmul_q8(int64_t w, int64_t qsOffset, int64_t scalesOffset, int64_t x,
                           int64_t xOffset, int64_t y, int64_t yOffset, int64_t rows,
                           int64_t cols, int64_t n);
void lab_gpu_enc_matmul_q4(int64_t w, int64_t qsOffset, int64_t scalesOffset, int64_t x,
                           int64_t xOffset, int64_t y, int64_t yOffset, int64_t rows,
                           int64_t cols, int64_t n);

// Input mode of the matmuls recorded from now on; returns the previous mode
// (1 int8, 0 float). No counterpart in the reference's ABI, where the layer
// decides: the Vulkan layer quantizes the inputs per block on a device with
// integer dot products (lab_vulkan.c:842-858), the Metal layer multiplies
// float inputs (lab_metal.m:1025-1038). 1 (the default) is the Vulkan
// behaviour above; 0 is the Metal one: lab_gemm_q8 / lab_gemm_q4 mode 0's
// products (what GpuLinear documents, gpu.dart:1271-1275), bit-identical
// for n <= 4 with x narrow enough for the exact float GEMV (its LDS takes
// the tokens of a weight pass, 4 down to 1 as x widens, up to about 35000
// fp32 columns; 14000 for more than 16384 rows), and within
// 1e-4 + 1e-5 |y| otherwise (the bf16-MFMA float GEMM, any width).
// The environment variable DIANOIA_GPU_INT8_INPUTS=0 sets 0 at
// lab_gpu_init, for callers that cannot call this.
int64_t lab_gpu_set_int8_inputs(int64_t on);

// The decoder's other layer steps, as the reference binds them
// (lib/src/gpu.dart:179-312; Vulkan lab_vulkan.c:899-1023, Metal
// lab_metal.m:1046-1196) and with the Metal shaders' semantics
// (lab_metal.m:321-579); fp32, equal to the reference's to fp32 rounding.
// Offsets are bytes; strides are floats. An argument the kernel cannot take
// (a region outside its buffer, hd not a multiple of 4 dividing 256 for
// attention, conv k above 16) fails the command buffer (commit returns 0),
// as the reference's kernels would read out of bounds instead.
void lab_gpu_enc_rms_norm(int64_t x, int64_t xOffset, int64_t w, int64_t wOffset, int64_t out,
                          int64_t outOffset, int64_t rows, int64_t cols, double eps,
                          int64_t accumulate);
void lab_gpu_enc_head_norm_rope(int64_t x, int64_t xOffset, int64_t xStride, int64_t w,
                                int64_t wOffset, int64_t rope, int64_t ropeOffset,
                                int64_t ropeStride, int64_t heads, int64_t hd, int64_t n,
                                double eps);
void lab_gpu_enc_conv(int64_t bcx, int64_t weight, int64_t weightOffset, int64_t history,
                      int64_t y, int64_t width, int64_t k, int64_t n);
// A negative `gate` leaves the heads ungated; `keys` and `values` hold rows
// of kvHeads * hd floats for positions 0 .. position + n - 1.
void lab_gpu_enc_attention(int64_t q, int64_t keys, int64_t values, int64_t gate, int64_t out,
                           int64_t position, int64_t n, int64_t heads, int64_t kvHeads,
                           int64_t hd, int64_t window);
void lab_gpu_enc_copy(int64_t src, int64_t srcOffset, int64_t dst, int64_t dstOffset,
                      int64_t count);
void lab_gpu_enc_add(int64_t src, int64_t srcOffset, int64_t dst, int64_t dstOffset,
                     int64_t count);
void lab_gpu_enc_steer(int64_t x, int64_t xOffset, int64_t v, int64_t vOffset, int64_t rows,
                       int64_t cols, int64_t mode, double scale);

// lab_gpu_enc_swiglu (lab_vulkan.c:974-978; gpu.dart:179-312): g = SiLU(g)
// * u over `count` floats from offset 0 of each buffer, SiLU in double as
// the CPU glue computes it (shard.dart:457-461).
void lab_gpu_enc_swiglu(int64_t g, int64_t u, int64_t count);

// Load-time Q8 quantization on the GPU. No GPU counterpart in the
// reference, which quantizes on the CPU: lab_quantize_q8 (lab_native.c:
// 407-429, bound at native.dart:138-147) for fp32 weights, after
// SafetensorsFile._widenBf16 (safetensors.dart:207-212) for BF16 ones
// (vision_encoder.dart:36-66). rows x cols values (fp32, or bf16 bits) at
// src + srcOffset become int8 [rows][colsPad] at qs + qsOffset and fp32
// scales [rows][colsPad/32] at scales + scalesOffset, bit-exact with that
// CPU path. colsPad is a multiple of 32 >= cols; the tail is zero padding
// (the reference refuses cols % 32 != 0, native.dart:634-636; padding is
// this library's defined extension).
void lab_gpu_enc_quantize_q8(int64_t src, int64_t srcOffset, int64_t qs, int64_t qsOffset,
                             int64_t scales, int64_t scalesOffset, int64_t rows, int64_t cols,
                             int64_t colsPad);
void lab_gpu_enc_quantize_q8_bf16(int64_t src, int64_t srcOffset, int64_t qs, int64_t qsOffset,
                                  int64_t scales, int64_t scalesOffset, int64_t rows,
                                  int64_t cols, int64_t colsPad);

// Load-time Q4 quantization on the GPU, the Q4 twin of the above: rows x
// cols values (fp32, or bf16 bits) at src + srcOffset become nibbles
// [rows][cols/2] at qs + qsOffset and fp16 scale bits [rows][cols/32] at
// scales + scalesOffset, bit-exact with lab_quantize_q4 (lab_native.c:
// 928-955, bound at native.dart:178-187) after _widenBf16 for BF16. cols
// must be a multiple of 32, as NativeQ4Matrix.quantize requires
// (native.dart:793-796); otherwise the command buffer fails.
void lab_gpu_enc_quantize_q4(int64_t src, int64_t srcOffset, int64_t qs, int64_t qsOffset,
                             int64_t scales, int64_t scalesOffset, int64_t rows, int64_t cols);
void lab_gpu_enc_quantize_q4_bf16(int64_t src, int64_t srcOffset, int64_t qs, int64_t qsOffset,
                                  int64_t scales, int64_t scalesOffset, int64_t rows,
                                  int64_t cols);

// The Q6_K -> Q8 embedding / LM-head adapter on the GPU (importGguf's tied
// embedding, lib/src/gguf.dart:402-414, which dequantizes with
// dequantizeQ6K :220-254 and quantizes with NativeQ8Matrix.quantizeRows,
// native.dart:645-672, on the CPU): rows x cols/256 super-blocks of 210
// bytes at src + srcOffset become int8 [rows][cols] at qs + qsOffset and
// fp32 scales [rows][cols/32] at scales + scalesOffset, bit-exact. cols
// must be a multiple of 256; otherwise the command buffer fails.
void lab_gpu_enc_q6k_to_q8(int64_t src, int64_t srcOffset, int64_t qs, int64_t qsOffset,
                           int64_t scales, int64_t scalesOffset, int64_t rows, int64_t cols);

// GGUF Q8_0 / Q4_0 blocks split into the engine's layout on the GPU. No
// counterpart in the reference's GPU ABI: its loader splits on the CPU
// (splitQ8_0, lib/src/gguf.dart:270-282; splitQ4_0, :208-218) before the
// upload; here the raw blocks are uploaded and split in HBM, bit for bit.
// rows x cols/32 blocks of 34 (Q8_0) or 18 (Q4_0) bytes at src + srcOffset
// become the values at qs + qsOffset and the scales at scales +
// scalesOffset (Q8: fp32, the fp16 d widened exactly; Q4: the fp16 bits).
// cols must be a multiple of 32, srcOffset a multiple of 4 and qsOffset of
// 16; otherwise the command buffer fails.
void lab_gpu_enc_split_q8_0(int64_t src, int64_t srcOffset, int64_t qs, int64_t qsOffset,
                            int64_t scales, int64_t scalesOffset, int64_t rows, int64_t cols);
void lab_gpu_enc_split_q4_0(int64_t src, int64_t srcOffset, int64_t qs, int64_t qsOffset,
                            int64_t scales, int64_t scalesOffset, int64_t rows, int64_t cols);

// Greedy token on the GPU: argmaxToken (sampler.dart:137-152, no
// suppression) over n floats at x + xOffset, the index written as one int64
// at out + outOffset. Replaces the logits copy + host argmax of
// ChatSession.greedyToken (chat_session.dart:267-270, gpu.dart:785-793).
void lab_gpu_enc_argmax(int64_t x, int64_t xOffset, int64_t n, int64_t out, int64_t outOffset);

// The projector's exact-erf GELU in place over count floats at x + xOffset
// (vision_encoder.dart:260-263): the glue between the vision encoder's fc1
// and fc2. No GPU counterpart in the reference (done in Dart there).
void lab_gpu_enc_gelu(int64_t x, int64_t xOffset, int64_t count);

// lab_gpu_set_profiling / lab_gpu_profile (lab_vulkan.c:720-733;
// gpu.dart:102-109, 545-564): per-kind GPU ms and dispatch counts since the
// last call, in the reference's 18-kind order, followed here by three kinds
// of this library's own (18 argmax, 19 weight quantization, 20 gelu). Copies
// at most `kinds` entries and returns the number of kinds (21). A fused
// launch (several encoded commands in one kernel) books its time under its
// main kernel's kind and counts each other command under that command's own
// kind with no time, so the counts equal those of one launch per command.
// Q4 prefill routes that run a load-time prepack book it once as weight
// quantization (19) and the activation panel as quantize (10).
void lab_gpu_set_profiling(int64_t on);
int64_t lab_gpu_profile(double* ms, int64_t* counts, int64_t kinds);

// Tuning knobs and device queries (lab_vulkan.c:506-530, 670-717;
// gpu.dart:39-61, 87-100). The decode kernel here has one shape chosen per
// matrix, so the knobs are accepted and have no effect: set_decode_rows is a
// no-op, set_q8_group / set_q8_vector / register_q8_head return 0 (not
// available), as the Metal layer does (lab_metal.m:757-766).
void lab_gpu_set_decode_rows(int64_t rows);
int64_t lab_gpu_set_q8_group(int64_t invocations);
int64_t lab_gpu_set_q8_vector(int64_t on);
int64_t lab_gpu_register_q8_head(int64_t w, int64_t qs, int64_t rows, int64_t cols,
                                 int64_t q4Body);
void lab_gpu_device_name(char* out, int64_t capacity);
int64_t lab_gpu_max_buffer_length(void);
int64_t lab_gpu_max_shared_memory(void);
int64_t lab_gpu_recommended_working_set(void);
int64_t lab_gpu_thermal_state(void);
int64_t lab_gpu_physical_memory(void);

#ifdef __cplusplus
}
#endif
