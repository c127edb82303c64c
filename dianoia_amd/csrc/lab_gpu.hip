// The lab_gpu_* C ABI of the reference (src/vulkan/lab_vulkan.c,
// src/metal/lab_metal.m), on one MI355X through HIP.
//
// Design for a discrete GPU (the reference assumes host-visible coherent
// buffers, lab_vulkan.c:7-10):
//
// * A buffer is an HBM allocation plus a pinned host shadow; the shadow is
//   what lab_gpu_contents returns. Wrapped weights get no shadow until a
//   caller asks for their contents.
// * lab_gpu_enc_* only record commands. lab_gpu_commit runs them in order
//   on one HIP stream: before a command, the host regions it reads are
//   uploaded unless an earlier command of this command buffer wrote them
//   (the host may have rewritten any input since, lab_vulkan.c:664); a
//   weight buffer is uploaded once, on its first use as weights, and is
//   immutable afterwards. After the last command, every region a command
//   wrote is copied back to the shadow. Stream order gives each dispatch
//   the previous one's writes (the reference's barrier after each
//   dispatch, lab_vulkan.c:769-787).
// * Host writes are tracked per page, so that a commit uploads only what
//   the host changed: a shadow page whose bytes equal HBM's is "clean" and
//   write-protected (mprotect). The host's first write to it faults; the
//   SIGSEGV handler installed by lab_gpu_init marks the page dirty, lifts
//   the protection and returns, and the write proceeds. A read region
//   uploads its dirty pages whole (protected again before the copy is
//   queued, so a later write faults again), and a copy-back makes the
//   pages it covers whole clean. Faults the handler does not own go to the
//   handler installed before it. DIANOIA_GPU_TRACK_WRITES=0 turns tracking
//   off (every read region is uploaded, as the reference's coherent
//   memory implies); so does a buffer whose shadow cannot be protected.
// * Scratch (quantized activations, argmax partials) is internal device
//   memory: it does not count as a live buffer.

#include <hip/hip_runtime.h>
#include <signal.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <thread>
#include <utility>
#include <vector>

#include "dnx_kernels.h"
#include "matmul_route.h"
#include "lab_gpu.h"

#define LOG(...) fprintf(stderr, "lab_gpu: " __VA_ARGS__)

namespace {

constexpr int64_t kMaxBuffers = 4096;
constexpr int kMaxProfiled = 1024;

// Kernel kinds in the reference's lab_gpu_profile order (lab_vulkan.c:
// 174-177, names in gpu.dart:545-564), then this library's own.
enum Kind {
  kKindGemvQ8, kKindGemmQ8, kKindGemvQ4, kKindGemmQ4, kKindRmsNorm, kKindHeadNormRope,
  kKindConv, kKindAttention, kKindSwiglu, kKindCopy, kKindQuantize, kKindGemmQ8I8,
  kKindGemmQ4I8, kKindGemvQ8I8, kKindGemvQ4I8, kKindGemvQ8I8Vec, kKindSteer, kKindAdd,
  kKindArgmax, kKindQuantizeWeights, kKindGelu, kKinds
};

struct Buffer {
  void* host = nullptr;   // pinned shadow (lazily made for wrapped buffers)
  void* dev = nullptr;
  int64_t size = 0;
  bool live = false;
  bool weights = false;   // HBM copy is authoritative and immutable
  bool tracked = false;   // host writes tracked per page (see Tracked below)
};

// Page tracking of a shadow, read by the SIGSEGV handler: [start, end) is the
// shadow (whole pages), clean[p] = 1 while page p equals HBM and is
// write-protected. start is published last on creation and cleared first on
// release, so the handler never sees a half-made entry.
struct Tracked {
  std::atomic<uintptr_t> start{0};
  uintptr_t end = 0;
  uint8_t* clean = nullptr;
};

enum Op {
  kOpMatmulQ8, kOpMatmulQ4, kOpSwiglu, kOpQuantize, kOpQuantizeBf16, kOpQuantizeQ4,
  kOpQuantizeQ4Bf16, kOpQ6kToQ8, kOpSplitQ8, kOpSplitQ4, kOpArgmax, kOpGelu, kOpRmsNorm,
  kOpHeadNormRope, kOpConv, kOpAttention, kOpCopy, kOpAdd, kOpSteer
};

struct Cmd {
  Op op;
  int64_t a[12];
  bool int8_inputs;  // matmuls: the input mode when the command was recorded
};

struct Region {
  int64_t handle, offset, bytes;
};

bool gReady = false;
// Matmul input mode. Int8 inputs (the default): x quantized per block as
// lab_quantize_q8 does, as the Vulkan layer does on a device with integer
// dot products (lab_vulkan.c:842-858) and lab_gemm_* mode 1. Float inputs:
// x used as given, as the Metal layer does and lab_gemm_* mode 0.
bool gInt8Inputs = true;
hipStream_t gStream;
hipEvent_t gStart, gStop;
hipEvent_t gProfEvents[kMaxProfiled];
int gProfKinds[kMaxProfiled];
int gProfiled = 0;
bool gProfiling = false;
double gKindMs[kKinds];
int64_t gKindCount[kKinds];
double gLastMs = 0;
bool gPending = false;
bool gFailed = false;   // a recorded command was invalid
std::vector<Cmd> gCmds;
std::vector<Region> gWritten;

Buffer gBuffers[kMaxBuffers];
int64_t gBufferCount = 0, gFree[kMaxBuffers], gFreeCount = 0, gLive = 0;

// Host-write tracking (see the header comment).
Tracked gTracked[kMaxBuffers];
std::atomic<int64_t> gTrackedSpan{0};  // entries [0, span) may be in use
bool gTrack = false;                    // tracking enabled and handler installed
int64_t gPage = 4096;
struct sigaction gPrevSegv;
// Bytes moved over PCIe by commits and first weight uploads (cumulative).
int64_t gUpBytes = 0, gDownBytes = 0;

// Quantized-activation workspace of the GEMM routes, and argmax partials.
void* gWs = nullptr;
int64_t gWsBytes = 0;

// The activation panel the prepacked route last made in the matmul
// workspace, and from which x: the next prepacked matmul of the same x in
// the command buffer (a prefill chunk's q, k and v projections, or its gate
// and up, all read one normed x) runs on it without quantizing again. It is
// forgotten when a command writes that x, when another route uses the
// workspace, when the workspace is re-made, and at every commit (the host
// may have written x since).
struct PanelKey {
  int64_t handle = -1, offset = 0, n = 0, cols = 0;
  bool i8 = false;  // the int8 GEMM's panel (dnx_quantize_q8_i8panel), else the fp6 one
};
PanelKey gPanel;
void* gArgmaxWs = nullptr;
void* gGemvArgmaxWs = nullptr;  // zeroed once; each fused argmax leaves it zero

bool valid(int64_t h) { return h >= 0 && h < gBufferCount && gBuffers[h].live; }

bool in_bounds(int64_t h, int64_t offset, int64_t bytes) {
  return valid(h) && offset >= 0 && bytes >= 0 && offset + bytes <= gBuffers[h].size;
}

char* dev_at(int64_t h, int64_t offset) { return (char*)gBuffers[h].dev + offset; }

// ---------------------------------------------------------------- host-write tracking

// A write to a write-protected shadow page: that page becomes dirty and
// writable again, and the write is retried. Anything else goes to the
// handler that was installed before lab_gpu_init.
void on_segv(int sig, siginfo_t* info, void* ctx) {
  const uintptr_t a = (uintptr_t)info->si_addr;
  if (info->si_code == SEGV_ACCERR) {
    const int64_t span = gTrackedSpan.load(std::memory_order_acquire);
    for (int64_t i = 0; i < span; i++) {
      const uintptr_t start = gTracked[i].start.load(std::memory_order_acquire);
      if (start == 0 || a < start || a >= gTracked[i].end) continue;
      const uintptr_t page = (a - start) / (uintptr_t)gPage;
      __atomic_store_n(&gTracked[i].clean[page], (uint8_t)0, __ATOMIC_RELEASE);
      if (mprotect((void*)(start + page * (uintptr_t)gPage), (size_t)gPage,
                   PROT_READ | PROT_WRITE) == 0) {
        return;
      }
      break;
    }
  }
  if (gPrevSegv.sa_flags & SA_SIGINFO) {
    if (gPrevSegv.sa_sigaction != nullptr) {
      gPrevSegv.sa_sigaction(sig, info, ctx);
      return;
    }
  } else if (gPrevSegv.sa_handler != SIG_DFL && gPrevSegv.sa_handler != SIG_IGN) {
    gPrevSegv.sa_handler(sig);
    return;
  }
  // The default action: restored, the access repeats and ends the process
  // as it would have without this handler.
  signal(SIGSEGV, SIG_DFL);
}

int64_t shadow_pages(int64_t bytes) { return (bytes + gPage - 1) / gPage; }

// Stops tracking h: every page counts as dirty from now on.
void untrack(int64_t h) {
  Buffer& b = gBuffers[h];
  if (!b.tracked) return;
  gTracked[h].start.store(0, std::memory_order_release);
  (void)mprotect(b.host, (size_t)(shadow_pages(b.size) * gPage), PROT_READ | PROT_WRITE);
  b.tracked = false;
}

// Marks pages [p0, p1) of h clean, then write-protects them: a host write
// before the protection lands before any copy queued after this call reads
// the page, and one after it faults and marks the page dirty again.
void make_clean(int64_t h, int64_t p0, int64_t p1) {
  Buffer& b = gBuffers[h];
  if (!b.tracked || p1 <= p0) return;
  uint8_t* c = gTracked[h].clean;
  for (int64_t p = p0; p < p1; p++) __atomic_store_n(&c[p], (uint8_t)1, __ATOMIC_RELEASE);
  if (mprotect((char*)b.host + p0 * gPage, (size_t)((p1 - p0) * gPage), PROT_READ) != 0) {
    LOG("write-protecting a host view failed; buffer %ld is uploaded whole from now on\n",
        (long)h);
    untrack(h);
  }
}

bool page_clean(int64_t h, int64_t p) {
  return __atomic_load_n(&gTracked[h].clean[p], __ATOMIC_ACQUIRE) != 0;
}

// Starts tracking a new shadow whose bytes equal HBM: every page clean.
void track(int64_t h) {
  Buffer& b = gBuffers[h];
  b.tracked = false;
  if (!gTrack || b.host == nullptr || ((uintptr_t)b.host % (uintptr_t)gPage) != 0) return;
  const int64_t pages = shadow_pages(b.size);
  Tracked& t = gTracked[h];
  uint8_t* c = (uint8_t*)realloc(t.clean, (size_t)pages);
  if (c == nullptr) return;
  memset(c, 0, (size_t)pages);
  t.clean = c;
  t.end = (uintptr_t)b.host + (uintptr_t)(pages * gPage);
  t.start.store((uintptr_t)b.host, std::memory_order_release);
  int64_t span = gTrackedSpan.load(std::memory_order_relaxed);
  while (span < h + 1 && !gTrackedSpan.compare_exchange_weak(span, h + 1)) {
  }
  b.tracked = true;
  make_clean(h, 0, pages);
}

// The handler stays ours only while nobody replaced it; otherwise tracking
// stops (a write fault would no longer reach it).
void check_handler() {
  if (!gTrack) return;
  struct sigaction cur;
  if (sigaction(SIGSEGV, nullptr, &cur) == 0 && (cur.sa_flags & SA_SIGINFO) &&
      cur.sa_sigaction == on_segv) {
    return;
  }
  LOG("another SIGSEGV handler replaced this library's; host-write tracking is off\n");
  for (int64_t h = 0; h < gBufferCount; h++) {
    if (gBuffers[h].live) untrack(h);
  }
  gTrack = false;
}

int64_t create(int64_t bytes, bool shadow) {
  if (!gReady || bytes <= 0) return -1;
  int64_t handle;
  if (gFreeCount > 0) {
    handle = gFree[gFreeCount - 1];
  } else if (gBufferCount < kMaxBuffers) {
    handle = gBufferCount;
  } else {
    return -1;
  }
  Buffer b;
  if (hipMalloc(&b.dev, (size_t)bytes) != hipSuccess) return -1;
  if (shadow && hipHostMalloc(&b.host, (size_t)(shadow_pages(bytes) * gPage),
                              hipHostMallocDefault) != hipSuccess) {
    (void)hipFree(b.dev);
    return -1;
  }
  b.size = bytes;
  b.live = true;
  gBuffers[handle] = b;
  if (handle == gBufferCount) {
    gBufferCount++;
  } else {
    gFreeCount--;
  }
  gLive++;
  return handle;
}

// Uploads the parts of [offset, offset + bytes) of h that no command of
// this command buffer has written (those are current in HBM already).
void upload_gaps(int64_t h, int64_t offset, int64_t bytes) {
  Buffer& b = gBuffers[h];
  std::vector<std::pair<int64_t, int64_t>> cover;
  for (const Region& r : gWritten) {
    if (r.handle == h && offset < r.offset + r.bytes && r.offset < offset + bytes) {
      cover.push_back({r.offset, r.offset + r.bytes});
    }
  }
  std::sort(cover.begin(), cover.end());
  int64_t at = offset;
  const int64_t end = offset + bytes;
  for (const auto& c : cover) {
    if (c.first > at) {
      (void)hipMemcpyAsync(dev_at(h, at), (char*)b.host + at, (size_t)(c.first - at),
                           hipMemcpyHostToDevice, gStream);
      gUpBytes += c.first - at;
    }
    if (c.second > at) at = c.second;
  }
  if (at < end) {
    (void)hipMemcpyAsync(dev_at(h, at), (char*)b.host + at, (size_t)(end - at),
                         hipMemcpyHostToDevice, gStream);
    gUpBytes += end - at;
  }
}

// Makes the device copy of [offset, offset + bytes) of h current: with
// tracking, each run of dirty pages it touches is uploaded whole (and made
// clean first); without, the whole region.
void read_region(int64_t h, int64_t offset, int64_t bytes) {
  Buffer& b = gBuffers[h];
  if (b.weights || b.host == nullptr || bytes <= 0) return;
  if (!b.tracked) {
    upload_gaps(h, offset, bytes);
    return;
  }
  const int64_t last = (offset + bytes - 1) / gPage;
  for (int64_t p = offset / gPage; p <= last;) {
    if (page_clean(h, p)) {
      p++;
      continue;
    }
    int64_t q = p + 1;
    while (q <= last && !page_clean(h, q)) q++;
    make_clean(h, p, q);
    const int64_t end = std::min(q * gPage, b.size);
    upload_gaps(h, p * gPage, end - p * gPage);
    p = q;
  }
}

// First use of h as weights: its host content goes to HBM once (except what
// this command buffer already produced there); afterwards HBM is
// authoritative and the buffer is treated as immutable.
void use_as_weights(int64_t h) {
  Buffer& b = gBuffers[h];
  if (b.weights) return;
  if (b.host != nullptr) {
    if (b.tracked) {
      read_region(h, 0, b.size);
    } else {
      upload_gaps(h, 0, b.size);
    }
  }
  b.weights = true;
}

void stale_prepacks(int64_t h, int64_t offset, int64_t bytes);
void stale_panel(int64_t h, int64_t offset, int64_t bytes);

// A command wrote [offset, offset + bytes) of h: recorded for the copy-back
// and the upload gaps; a prepacked copy of weights it overwrote is re-made
// at its next use, and an activation panel made from it is not reused.
void wrote_region(int64_t h, int64_t offset, int64_t bytes) {
  gWritten.push_back({h, offset, bytes});
  stale_prepacks(h, offset, bytes);
  stale_panel(h, offset, bytes);
}

void after_dispatch(int kind) {
  if (gProfiling && gProfiled < kMaxProfiled) {
    (void)hipEventRecord(gProfEvents[gProfiled], gStream);
    gProfKinds[gProfiled++] = kind;
  }
}

// A fused launch (the commit peepholes below) runs several encoded
// commands: its time goes to the kind of its main kernel (after_dispatch),
// and every other command it ran is counted under its own kind with no time
// of its own, so the profile counts the same dispatches per kind as one
// launch per command would.
void also_ran(int kind, int times = 1) {
  if (gProfiling) gKindCount[kind] += times;
}

// Grows the matmul workspace to what a command of this shape needs (at
// encode time: outside the commit that launches it).
bool grow_scratch(int64_t cols, int64_t n) {
  const int64_t need = dnx_matmul_workspace_bytes(cols, n);
  if (need < 0) return false;
  if (need <= gWsBytes) return true;
  const int64_t cap = need > (4 << 20) ? need : (4 << 20);
  gPanel = PanelKey{};
  if (gWs) (void)hipFree(gWs);
  gWs = nullptr;
  gWsBytes = 0;
  if (hipMalloc(&gWs, (size_t)cap) != hipSuccess) return false;
  gWsBytes = cap;
  return true;
}

bool wait_pending() {
  if (!gPending) return true;
  gPending = false;
  if (hipEventSynchronize(gStop) != hipSuccess) return false;
  float ms = 0;
  if (hipEventElapsedTime(&ms, gStart, gStop) == hipSuccess) gLastMs = ms;
  for (int i = 0; i < gProfiled; i++) {
    float e = 0;
    // Each dispatch's share runs from the previous mark to its own, which
    // includes the uploads it waited for (as the reference's includes its
    // barrier, lab_vulkan.c:623-629).
    if (hipEventElapsedTime(&e, i == 0 ? gStart : gProfEvents[i - 1], gProfEvents[i]) ==
        hipSuccess) {
      gKindMs[gProfKinds[i]] += e;
      gKindCount[gProfKinds[i]]++;
    }
  }
  gProfiled = 0;
  return hipStreamQuery(gStream) == hipSuccess;
}

void record(Op op, std::initializer_list<int64_t> args) {
  Cmd c;
  c.op = op;
  c.int8_inputs = gInt8Inputs;
  int i = 0;
  for (int64_t v : args) c.a[i++] = v;
  gCmds.push_back(c);
}

// Prepacked copies of weight matrices: Q4 for the fp6 GEMMs (the routes of
// prefill chunks, dnx::matmul_uses_f6_chunk, and of large prefill shapes,
// dnx::matmul_uses_f6), Q8 for the int8 GEMM on prepacked operands (large
// batches, dnx::matmul_uses_i8p). The host cannot change weights once used
// (use_as_weights), so a matrix region is re-encoded on its first such
// matmul into the GEMM's layout (dnx_pack_q4_f6, dnx_pack_q8_i8), and later
// products of it run on the prepack. A command that writes into the region
// (a load-time quantizer, a copy, a GGUF split run again into the same
// buffer) marks the prepack stale, and the next matmul re-makes it. The
// copy's memory is reserved when the command is encoded (no allocation
// inside a commit); it is freed with the buffer. Not a live buffer:
// lab_gpu_live_buffers does not count it.
constexpr size_t kMaxChunkSegs = 4;   // matrices per dnx_gemm_q4_f6s_multi launch

struct Prepack {
  int64_t handle, qs_off, sc_off, rows, cols;
  void* dev;
  bool packed;
  bool q8;
};
std::vector<Prepack> gPrepacks;

Prepack* find_prepack(int64_t h, int64_t qs_off, int64_t sc_off, int64_t rows, int64_t cols,
                      bool q8 = false) {
  for (Prepack& p : gPrepacks) {
    if (p.handle == h && p.qs_off == qs_off && p.sc_off == sc_off && p.rows == rows &&
        p.cols == cols && p.q8 == q8) {
      return &p;
    }
  }
  return nullptr;
}

// At encode time: the prepack an int8-input matmul of this shape will use
// (Q4, or Q8 with q8), reserved now. Where the device has no memory for it
// (or the copy would pass the GEMM's 2 GB operand limit) the command runs on
// the engine layout.
void reserve_prepack(int64_t h, int64_t qs_off, int64_t sc_off, int64_t rows, int64_t cols,
                     bool q8 = false) {
  if (find_prepack(h, qs_off, sc_off, rows, cols, q8) != nullptr) return;
  const int64_t bytes = q8 ? dnx_q8_i8pack_bytes(rows, cols) : dnx_q4_f6pack_bytes(rows, cols);
  void* dev = nullptr;
  if (bytes <= 0 || bytes >= (1ll << 31) || hipMalloc(&dev, (size_t)bytes) != hipSuccess) return;
  gPrepacks.push_back({h, qs_off, sc_off, rows, cols, dev, false, q8});
}

void stale_prepacks(int64_t h, int64_t offset, int64_t bytes) {
  for (Prepack& p : gPrepacks) {
    if (p.handle != h || !p.packed) continue;
    const int64_t qs_end = p.qs_off + p.rows * (p.q8 ? p.cols : p.cols / 2);
    const int64_t sc_end = p.sc_off + p.rows * (p.cols / 32) * (p.q8 ? 4 : 2);
    const int64_t end = offset + bytes;
    if ((offset < qs_end && p.qs_off < end) || (offset < sc_end && p.sc_off < end)) {
      p.packed = false;
    }
  }
}

void stale_panel(int64_t h, int64_t offset, int64_t bytes) {
  if (h == gPanel.handle && offset < gPanel.offset + gPanel.n * gPanel.cols * 4 &&
      gPanel.offset < offset + bytes) {
    gPanel = PanelKey{};
  }
}

void free_prepacks(int64_t h) {
  for (size_t i = 0; i < gPrepacks.size();) {
    if (gPrepacks[i].handle == h) {
      (void)hipFree(gPrepacks[i].dev);
      gPrepacks[i] = gPrepacks.back();
      gPrepacks.pop_back();
    } else {
      i++;
    }
  }
}

// The prepacked route: the prepack (made on first use), the activation
// panel from fp32 x, the GEMM: the chunk GEMM (one launch over the whole K)
// where matmul_uses_f6_chunk takes the shape, else the tiled GEMM (the same
// products as the engine-layout fp6 GEMM, bit for bit).
// The prepack of a matrix made if it is not (first use, or stale).
int ensure_packed(Prepack& pp, int64_t w, int64_t qsOff, int64_t scOff, int64_t rows,
                  int64_t cols) {
  if (pp.packed) return DNX_OK;
  const int rc = pp.q8 ? dnx_pack_q8_i8((const int8_t*)dev_at(w, qsOff),
                                        (const float*)dev_at(w, scOff), pp.dev, rows, cols,
                                        (dnx_stream_t)gStream)
                       : dnx_pack_q4_f6((const uint8_t*)dev_at(w, qsOff),
                                        (const uint16_t*)dev_at(w, scOff), pp.dev, rows, cols,
                                        (dnx_stream_t)gStream);
  if (rc != DNX_OK) return rc;
  after_dispatch(kKindQuantizeWeights);
  pp.packed = true;
  return DNX_OK;
}

// The activation panel of x in the workspace (the fp6 GEMMs', or with i8
// the int8 GEMM's), unless it is there already.
int ensure_panel(int64_t xh, int64_t xOff, int64_t n, int64_t cols, bool i8 = false) {
  if (gPanel.handle == xh && gPanel.offset == xOff && gPanel.n == n && gPanel.cols == cols &&
      gPanel.i8 == i8) {
    return DNX_OK;
  }
  gPanel = PanelKey{};
  const float* x = (const float*)dev_at(xh, xOff);
  const int rc = i8 ? dnx_quantize_q8_i8panel(x, gWs, n, cols, (dnx_stream_t)gStream)
                    : dnx_quantize_q8_f6panel(x, gWs, n, cols, (dnx_stream_t)gStream);
  if (rc != DNX_OK) return rc;
  after_dispatch(kKindQuantize);
  gPanel = PanelKey{xh, xOff, n, cols, i8};
  return DNX_OK;
}

int run_matmul_prepacked(Prepack& pp, int64_t w, int64_t qsOff, int64_t scOff, int64_t xh,
                         int64_t xOff, float* y, int64_t rows, int64_t cols, int64_t n) {
  auto s = (dnx_stream_t)gStream;
  int rc = ensure_packed(pp, w, qsOff, scOff, rows, cols);
  if (rc != DNX_OK) return rc;
  rc = ensure_panel(xh, xOff, n, cols, pp.q8);
  if (rc != DNX_OK) return rc;
  if (pp.q8) {
    rc = dnx_gemm_q8_i8p(pp.dev, gWs, y, rows, cols, n, s);
    if (rc == DNX_OK) after_dispatch(kKindGemmQ8I8);
    return rc;
  }
  rc = dnx::matmul_uses_f6_chunk(true, rows, cols, n)
           ? dnx_gemm_q4_f6s(pp.dev, gWs, y, rows, cols, n, s)
           : dnx_gemm_q4_f6p(pp.dev, gWs, y, rows, cols, n, s);
  if (rc == DNX_OK) after_dispatch(kKindGemmQ4I8);
  return rc;
}

// The matmul of one recorded command, on the product route of
// matmul_route.h (the same as dnx_matmul_q8 / _q4), with the fp6 GEMMs (Q4)
// or the int8 GEMM on prepacked operands (Q8) on a prepacked copy of the
// weights where one is reserved.
bool run_matmul(const Cmd& c, bool q4) {
  const int64_t w = c.a[0], qsOff = c.a[1], scOff = c.a[2], x = c.a[3], xOff = c.a[4];
  const int64_t y = c.a[5], yOff = c.a[6], rows = c.a[7], cols = c.a[8], n = c.a[9];
  use_as_weights(w);
  read_region(x, xOff, n * cols * 4);
  // The panel quantizer reads x 16 bytes at a time: an x at a 4-byte offset
  // that is not 16-byte aligned takes the route without the prepack.
  const bool x16 = ((uintptr_t)dev_at(x, xOff) & 15) == 0;
  Prepack* pp = nullptr;
  if (c.int8_inputs && x16) {
    if (q4 && (dnx::matmul_uses_f6(true, rows, cols, n) ||
               dnx::matmul_uses_f6_chunk(true, rows, cols, n))) {
      pp = find_prepack(w, qsOff, scOff, rows, cols);
    } else if (!q4 && dnx::matmul_uses_i8p(false, rows, cols, n)) {
      pp = find_prepack(w, qsOff, scOff, rows, cols, true);
    }
  }
  if (pp != nullptr) {
    const int rc = run_matmul_prepacked(*pp, w, qsOff, scOff, x, xOff, (float*)dev_at(y, yOff),
                                        rows, cols, n);
    wrote_region(y, yOff, n * rows * 4);
    if (rc != DNX_OK) {
      LOG("matmul %s %ldx%ld n=%ld (prepacked) failed (%d)\n", q4 ? "q4" : "q8", (long)rows,
          (long)cols, (long)n, rc);
    }
    return rc == DNX_OK;
  }
  gPanel = PanelKey{};  // the route may write the workspace
  const int rc = dnx::matmul_route(
      q4, dev_at(w, qsOff), dev_at(w, scOff), (const float*)dev_at(x, xOff),
      (float*)dev_at(y, yOff), rows, cols, n, c.int8_inputs, gWs, gWsBytes, gStream,
      [q4](dnx::MatmulStep step) {
        switch (step) {
          case dnx::MatmulStep::kGemvFloat: after_dispatch(q4 ? kKindGemvQ4 : kKindGemvQ8); break;
          case dnx::MatmulStep::kGemmFloat: after_dispatch(q4 ? kKindGemmQ4 : kKindGemmQ8); break;
          case dnx::MatmulStep::kGemv: after_dispatch(q4 ? kKindGemvQ4I8 : kKindGemvQ8I8); break;
          case dnx::MatmulStep::kQuantize:
          case dnx::MatmulStep::kQuantizeF6: after_dispatch(kKindQuantize); break;
          case dnx::MatmulStep::kGemm:
          case dnx::MatmulStep::kGemmF6: after_dispatch(q4 ? kKindGemmQ4I8 : kKindGemmQ8I8); break;
        }
      });
  wrote_region(y, yOff, n * rows * 4);
  if (rc != DNX_OK) {
    LOG("matmul %s %ldx%ld n=%ld (%s inputs) failed (%d)\n", q4 ? "q4" : "q8", (long)rows,
        (long)cols, (long)n, c.int8_inputs ? "int8" : "float", rc);
  }
  return rc == DNX_OK;
}

// Fusion of a gate/up pair and its glue: commands i, i+1 are matmuls of one
// format over the same input and shape into g and u (offset 0), and i+2 is
// lab_gpu_enc_swiglu(g, u, n * rows), as GpuForward encodes an MLP. One
// kernel computes both products and the glue; it also writes u, so the
// result is exactly what the three dispatches leave.
bool fusable_pair(const Cmd& a, const Cmd& b, const Cmd& c) {
  if (!(a.op == kOpMatmulQ8 || a.op == kOpMatmulQ4) || b.op != a.op || c.op != kOpSwiglu) {
    return false;
  }
  const int64_t n = a.a[9], rows = a.a[7];
  return a.int8_inputs && b.int8_inputs && n <= 4 && a.a[3] == b.a[3] && a.a[4] == b.a[4] && a.a[7] == b.a[7] &&
         a.a[8] == b.a[8] && a.a[9] == b.a[9] && a.a[6] == 0 && b.a[6] == 0 &&
         a.a[5] != b.a[5] && c.a[0] == a.a[5] && c.a[1] == b.a[5] && c.a[2] == n * rows;
}

// DNX_OK, or the launcher's code; DNX_EINVAL means the pair kernel refused
// the shape before launching anything (x too wide for its LDS at this n), and
// the caller then runs the three commands unfused.
int run_pair(const Cmd& a, const Cmd& b) {
  const bool q4 = a.op == kOpMatmulQ4;
  const int64_t x = a.a[3], xOff = a.a[4], rows = a.a[7], cols = a.a[8], n = a.a[9];
  use_as_weights(a.a[0]);
  use_as_weights(b.a[0]);
  read_region(x, xOff, n * cols * 4);
  const void* gq = dev_at(a.a[0], a.a[1]);
  const void* gs = dev_at(a.a[0], a.a[2]);
  const void* uq = dev_at(b.a[0], b.a[1]);
  const void* us = dev_at(b.a[0], b.a[2]);
  const float* xs = (const float*)dev_at(x, xOff);
  float* h = (float*)dev_at(a.a[5], 0);
  float* u = (float*)dev_at(b.a[5], 0);
  const int rc =
      q4 ? dnx_gate_up_q4((const uint8_t*)gq, (const uint16_t*)gs, (const uint8_t*)uq,
                          (const uint16_t*)us, xs, h, u, rows, cols, n, gStream)
         : dnx_gate_up_q8((const int8_t*)gq, (const float*)gs, (const int8_t*)uq,
                          (const float*)us, xs, h, u, rows, cols, n, gStream);
  if (rc == DNX_EINVAL) return rc;
  if (rc == DNX_OK) {
    after_dispatch(q4 ? kKindGemvQ4I8 : kKindGemvQ8I8);
    also_ran(q4 ? kKindGemvQ4I8 : kKindGemvQ8I8);
    also_ran(kKindSwiglu);
  }
  wrote_region(a.a[5], 0, n * rows * 4);
  wrote_region(b.a[5], 0, n * rows * 4);
  if (rc != DNX_OK) LOG("gate/up pair %ldx%ld n=%ld failed (%d)\n", (long)rows, (long)cols, (long)n, rc);
  return rc;
}

// Fusion of up to four decode matmuls over the same input: commands
// i .. i+L-1 (L >= 2) are one-token matmuls of one format, int8 inputs, the
// same x region and width (GpuForward.forward's q, k, v and gate
// projections, gpu.dart:1148-1156). Their outputs must be disjoint from each
// other and from x, so running them in one launch leaves what the L
// dispatches leave. Returns L, or 0.
bool overlaps(int64_t h0, int64_t o0, int64_t b0, int64_t h1, int64_t o1, int64_t b1) {
  return h0 == h1 && o0 < o1 + b1 && o1 < o0 + b0;
}

// The number of commands from i on that one segmented launch can run (1 when
// only cmds[i] qualifies, 0 when it does not).
size_t multi_len(const std::vector<Cmd>& cmds, size_t i) {
  const Cmd& a = cmds[i];
  if (!(a.op == kOpMatmulQ8 || a.op == kOpMatmulQ4) || !a.int8_inputs || a.a[9] != 1) return 0;
  const int64_t x = a.a[3], xOff = a.a[4], cols = a.a[8];
  size_t len = 0;
  for (size_t j = i; j < cmds.size() && len < 4; j++, len++) {
    const Cmd& b = cmds[j];
    if (b.op != a.op || !b.int8_inputs || b.a[9] != 1 || b.a[3] != x || b.a[4] != xOff ||
        b.a[8] != cols) {
      break;
    }
    if (overlaps(b.a[5], b.a[6], b.a[7] * 4, x, xOff, cols * 4)) break;
    bool clash = false;
    for (size_t k = i; k < j; k++) {
      clash = clash || overlaps(b.a[5], b.a[6], b.a[7] * 4, cmds[k].a[5], cmds[k].a[6],
                                cmds[k].a[7] * 4);
    }
    if (clash) break;
  }
  return len;
}

size_t fusable_multi(const std::vector<Cmd>& cmds, size_t i) {
  const size_t len = multi_len(cmds, i);
  return len >= 2 ? len : 0;
}

// DNX_OK, or the launcher's code; DNX_EINVAL means nothing was launched (the
// caller then runs the commands one by one).
int run_multi(const std::vector<Cmd>& cmds, size_t i, size_t len) {
  const Cmd& a = cmds[i];
  const bool q4 = a.op == kOpMatmulQ4;
  const int64_t x = a.a[3], xOff = a.a[4], cols = a.a[8];
  const void* qs[4];
  const void* sc[4];
  float* ys[4];
  int64_t rows[4];
  for (size_t k = 0; k < len; k++) {
    const Cmd& c = cmds[i + k];
    use_as_weights(c.a[0]);
    qs[k] = dev_at(c.a[0], c.a[1]);
    sc[k] = dev_at(c.a[0], c.a[2]);
    ys[k] = (float*)dev_at(c.a[5], c.a[6]);
    rows[k] = c.a[7];
  }
  read_region(x, xOff, cols * 4);
  const float* xs = (const float*)dev_at(x, xOff);
  const int rc =
      q4 ? dnx_gemv_multi_q4((const uint8_t* const*)qs, (const uint16_t* const*)sc, ys, rows,
                             (int)len, xs, cols, gStream)
         : dnx_gemv_multi_q8((const int8_t* const*)qs, (const float* const*)sc, ys, rows,
                             (int)len, xs, cols, gStream);
  if (rc == DNX_EINVAL) return rc;
  if (rc == DNX_OK) {
    after_dispatch(q4 ? kKindGemvQ4I8 : kKindGemvQ8I8);
    also_ran(q4 ? kKindGemvQ4I8 : kKindGemvQ8I8, (int)len - 1);
  }
  for (size_t k = 0; k < len; k++) wrote_region(cmds[i + k].a[5], cmds[i + k].a[6], rows[k] * 4);
  if (rc != DNX_OK) LOG("%zu fused matmuls of width %ld failed (%d)\n", len, (long)cols, rc);
  return rc;
}

// The prepack a recorded Q4 matmul runs on by the chunk route (int8
// inputs, a chunk shape, x 16-byte aligned, a prepack reserved), or null.
Prepack* chunk_prepack(const Cmd& c) {
  if (c.op != kOpMatmulQ4 || !c.int8_inputs) return nullptr;
  const int64_t rows = c.a[7], cols = c.a[8], n = c.a[9];
  if (!dnx::matmul_uses_f6_chunk(true, rows, cols, n)) return nullptr;
  if (((uintptr_t)dev_at(c.a[3], c.a[4]) & 15) != 0) return nullptr;
  return find_prepack(c.a[0], c.a[1], c.a[2], rows, cols);
}

// The command after the one the commit runs now (set by the commit loop for
// the commands that can hand the matmul after them its activation panel).
const Cmd* gNext = nullptr;

// Whether that next command is a prefill matmul on the chunk route reading
// [h + off, n x cols floats) as its input: the producer of that input then
// writes its panel too, and the matmul (or the group that starts with it)
// finds it made (gPanel).
bool next_reads_panel(int64_t h, int64_t off, int64_t n, int64_t cols) {
  if (gNext == nullptr || gWs == nullptr) return false;
  const Cmd& c = *gNext;
  return chunk_prepack(c) != nullptr && c.a[3] == h && c.a[4] == off && c.a[9] == n &&
         c.a[8] == cols;
}

// Consecutive prefill matmuls of one x on the chunk route (a chunk's q, k
// and v, or gate and up): how many (2..4) one launch runs, 0 for none. As in
// multi_len, no output may overlap x or another output, and none may land
// in a buffer that holds a group member's weights.
size_t chunk_multi_len(const std::vector<Cmd>& cmds, size_t i) {
  const Cmd& a = cmds[i];
  if (chunk_prepack(a) == nullptr) return 0;
  const int64_t x = a.a[3], xOff = a.a[4], cols = a.a[8], n = a.a[9];
  size_t len = 0;
  for (size_t j = i; j < cmds.size() && len < kMaxChunkSegs; j++, len++) {
    const Cmd& b = cmds[j];
    if (b.a[3] != x || b.a[4] != xOff || b.a[8] != cols || b.a[9] != n ||
        chunk_prepack(b) == nullptr) {
      break;
    }
    const int64_t yb = n * b.a[7] * 4;
    if (overlaps(b.a[5], b.a[6], yb, x, xOff, n * cols * 4)) break;
    bool clash = false;
    for (size_t k = i; k < j; k++) {
      clash = clash ||
              overlaps(b.a[5], b.a[6], yb, cmds[k].a[5], cmds[k].a[6], n * cmds[k].a[7] * 4) ||
              b.a[5] == cmds[k].a[0] || cmds[k].a[5] == b.a[0];
    }
    if (clash || b.a[5] == b.a[0]) break;
  }
  return len >= 2 ? len : 0;
}

// DNX_OK, or the launcher's code; DNX_EINVAL means the GEMM was not
// launched (the caller then runs the matmuls one by one, which reuse the
// prepacks and the panel made here).
int run_chunk_multi(const std::vector<Cmd>& cmds, size_t i, size_t len) {
  const Cmd& a = cmds[i];
  const int64_t x = a.a[3], xOff = a.a[4], cols = a.a[8], n = a.a[9];
  const void* packed[kMaxChunkSegs];
  float* ys[kMaxChunkSegs];
  int64_t rows[kMaxChunkSegs];
  int rc = DNX_OK;
  for (size_t k = 0; k < len && rc == DNX_OK; k++) {
    const Cmd& c = cmds[i + k];
    use_as_weights(c.a[0]);
    Prepack* pp = chunk_prepack(c);
    rc = ensure_packed(*pp, c.a[0], c.a[1], c.a[2], c.a[7], cols);
    packed[k] = pp->dev;
    ys[k] = (float*)dev_at(c.a[5], c.a[6]);
    rows[k] = c.a[7];
  }
  if (rc != DNX_OK) return rc;
  read_region(x, xOff, n * cols * 4);
  rc = ensure_panel(x, xOff, n, cols);
  if (rc != DNX_OK) return rc;
  rc = dnx_gemm_q4_f6s_multi(packed, ys, rows, (int)len, gWs, cols, n, (dnx_stream_t)gStream);
  if (rc == DNX_EINVAL) return rc;
  if (rc == DNX_OK) {
    after_dispatch(kKindGemmQ4I8);
    also_ran(kKindGemmQ4I8, (int)len - 1);
  }
  for (size_t k = 0; k < len; k++) {
    wrote_region(cmds[i + k].a[5], cmds[i + k].a[6], n * rows[k] * 4);
  }
  if (rc != DNX_OK) LOG("%zu prefill matmuls of width %ld failed (%d)\n", len, (long)cols, rc);
  return rc;
}

// Fusion of a one-token matmul and the residual add of its output into x
// (GpuForward adds each block's output into x, gpu.dart:1180-1187): the
// GEMV's epilogue also adds each output into its row of x (dnx_gemv_add_*),
// when the add reads exactly the matmul's output and x overlaps neither the
// matmul's input (which every workgroup reads first), its output nor its
// weights.
bool fusable_matmul_add(const Cmd& a, const Cmd& b) {
  if (!(a.op == kOpMatmulQ8 || a.op == kOpMatmulQ4) || !a.int8_inputs || a.a[9] != 1 ||
      b.op != kOpAdd) {
    return false;
  }
  const int64_t rows = a.a[7], cols = a.a[8];
  const int64_t m = b.a[0], mOff = b.a[1], x = b.a[2], xOff = b.a[3], count = b.a[4];
  if (m != a.a[5] || mOff != a.a[6] || count != rows) return false;
  return x != a.a[0] && !overlaps(x, xOff, rows * 4, a.a[3], a.a[4], cols * 4) &&
         !overlaps(x, xOff, rows * 4, m, mOff, rows * 4);
}

// DNX_OK, or the launcher's code; DNX_EINVAL means nothing was launched.
int run_matmul_add(const Cmd& a, const Cmd& b) {
  const bool q4 = a.op == kOpMatmulQ4;
  const int64_t w = a.a[0], x = a.a[3], xOff = a.a[4], y = a.a[5], yOff = a.a[6];
  const int64_t rows = a.a[7], cols = a.a[8], res = b.a[2], resOff = b.a[3];
  use_as_weights(w);
  read_region(x, xOff, cols * 4);
  read_region(res, resOff, rows * 4);
  const float* xs = (const float*)dev_at(x, xOff);
  float* ys = (float*)dev_at(y, yOff);
  float* rs = (float*)dev_at(res, resOff);
  const int rc =
      q4 ? dnx_gemv_add_q4((const uint8_t*)dev_at(w, a.a[1]), (const uint16_t*)dev_at(w, a.a[2]),
                           xs, ys, rs, rows, cols, gStream)
         : dnx_gemv_add_q8((const int8_t*)dev_at(w, a.a[1]), (const float*)dev_at(w, a.a[2]), xs,
                           ys, rs, rows, cols, gStream);
  if (rc == DNX_EINVAL) return rc;
  if (rc == DNX_OK) {
    after_dispatch(q4 ? kKindGemvQ4I8 : kKindGemvQ8I8);
    also_ran(kKindAdd);
  }
  wrote_region(y, yOff, rows * 4);
  wrote_region(res, resOff, rows * 4);
  if (rc != DNX_OK) LOG("matmul + add %ldx%ld failed (%d)\n", (long)rows, (long)cols, rc);
  return rc;
}

// Fusion of the RMSNorm of one row with the one-token matmuls that read its
// output (GpuForward norms x before each block, gpu.dart:1145-1156 and
// :1180-1185): the GEMV norms x in its prologue with the standalone kernel's
// values, quantizes the result and writes it to the norm's output
// (dnx_gate_up_norm_* for an MLP's gate/up pair and glue,
// dnx_gemv_multi_norm_* for one to four projections). The norm must not
// accumulate, its output must not overlap its input or weight and must be
// exactly the matmuls' input, and no matmul output may overlap the norm's
// input, weight or output (the prologue reads the first two in every
// workgroup; workgroup 0 writes the third at its end). Returns the number of
// commands after the norm that the launch covers (3 for a pair and its glue),
// or 0.
bool clear_of_norm(const Cmd& nrm, int64_t h, int64_t off, int64_t bytes) {
  const int64_t nb = nrm.a[7] * 4;
  return !overlaps(h, off, bytes, nrm.a[0], nrm.a[1], nb) &&
         !overlaps(h, off, bytes, nrm.a[2], nrm.a[3], nb) &&
         !overlaps(h, off, bytes, nrm.a[4], nrm.a[5], nb);
}

bool fusable_argmax(const Cmd& a, const Cmd& b);

size_t fusable_norm_matmul(const std::vector<Cmd>& cmds, size_t i, bool& pair) {
  const Cmd& nrm = cmds[i];
  if (nrm.op != kOpRmsNorm || nrm.a[9] != 0 || nrm.a[6] != 1 || i + 1 >= cmds.size()) return 0;
  const int64_t nb = nrm.a[7] * 4;
  if (overlaps(nrm.a[4], nrm.a[5], nb, nrm.a[0], nrm.a[1], nb) ||
      overlaps(nrm.a[4], nrm.a[5], nb, nrm.a[2], nrm.a[3], nb)) {
    return 0;
  }
  const Cmd& a = cmds[i + 1];
  if (a.a[3] != nrm.a[4] || a.a[4] != nrm.a[5] || a.a[8] != nrm.a[7]) return 0;
  if (i + 3 < cmds.size() && fusable_pair(a, cmds[i + 2], cmds[i + 3])) {
    const int64_t rb = a.a[7] * 4;
    if (a.a[9] != 1 || !clear_of_norm(nrm, a.a[5], 0, rb) ||
        !clear_of_norm(nrm, cmds[i + 2].a[5], 0, rb) || a.a[0] == nrm.a[4] ||
        cmds[i + 2].a[0] == nrm.a[4]) {
      return 0;
    }
    pair = true;
    return 3;
  }
  const size_t len = multi_len(cmds, i + 1);
  // A matmul whose output an argmax reads keeps its own fusion (the LM head
  // and the token, gpu.dart:1222-1236): the norm then runs alone.
  if (len == 1 && i + 2 < cmds.size() && fusable_argmax(a, cmds[i + 2])) return 0;
  for (size_t k = 0; k < len; k++) {
    const Cmd& c = cmds[i + 1 + k];
    // The weights are read while workgroup 0 writes the norm's output.
    if (!clear_of_norm(nrm, c.a[5], c.a[6], c.a[7] * 4) || c.a[0] == nrm.a[4]) return 0;
  }
  pair = false;
  return len;
}

// DNX_OK, or the launcher's code; DNX_EINVAL means nothing was launched (the
// caller then runs the norm alone and goes on with the commands after it).
int run_norm_matmul(const std::vector<Cmd>& cmds, size_t i, size_t len, bool pair) {
  const Cmd& nrm = cmds[i];
  const int64_t x = nrm.a[0], xOff = nrm.a[1], w = nrm.a[2], wOff = nrm.a[3];
  const int64_t out = nrm.a[4], outOff = nrm.a[5], cols = nrm.a[7];
  const float eps = (float)__builtin_bit_cast(double, nrm.a[8]);
  const Cmd& a = cmds[i + 1];
  const bool q4 = a.op == kOpMatmulQ4;
  read_region(x, xOff, cols * 4);
  read_region(w, wOff, cols * 4);
  const float* xs = (const float*)dev_at(x, xOff);
  const float* ws = (const float*)dev_at(w, wOff);
  float* os = (float*)dev_at(out, outOff);
  int rc;
  if (pair) {
    const Cmd& b = cmds[i + 2];
    const int64_t rows = a.a[7];
    use_as_weights(a.a[0]);
    use_as_weights(b.a[0]);
    const void* gq = dev_at(a.a[0], a.a[1]);
    const void* gs = dev_at(a.a[0], a.a[2]);
    const void* uq = dev_at(b.a[0], b.a[1]);
    const void* us = dev_at(b.a[0], b.a[2]);
    float* h = (float*)dev_at(a.a[5], 0);
    float* u = (float*)dev_at(b.a[5], 0);
    rc = q4 ? dnx_gate_up_norm_q4((const uint8_t*)gq, (const uint16_t*)gs, (const uint8_t*)uq,
                                  (const uint16_t*)us, xs, ws, os, eps, h, u, rows, cols, gStream)
            : dnx_gate_up_norm_q8((const int8_t*)gq, (const float*)gs, (const int8_t*)uq,
                                  (const float*)us, xs, ws, os, eps, h, u, rows, cols, gStream);
    if (rc == DNX_EINVAL) return rc;
    wrote_region(a.a[5], 0, rows * 4);
    wrote_region(b.a[5], 0, rows * 4);
  } else {
    const void* qs[4];
    const void* sc[4];
    float* ys[4];
    int64_t rows[4];
    for (size_t k = 0; k < len; k++) {
      const Cmd& c = cmds[i + 1 + k];
      use_as_weights(c.a[0]);
      qs[k] = dev_at(c.a[0], c.a[1]);
      sc[k] = dev_at(c.a[0], c.a[2]);
      ys[k] = (float*)dev_at(c.a[5], c.a[6]);
      rows[k] = c.a[7];
    }
    rc = q4 ? dnx_gemv_multi_norm_q4((const uint8_t* const*)qs, (const uint16_t* const*)sc, ys,
                                     rows, (int)len, xs, ws, os, eps, cols, gStream)
            : dnx_gemv_multi_norm_q8((const int8_t* const*)qs, (const float* const*)sc, ys, rows,
                                     (int)len, xs, ws, os, eps, cols, gStream);
    if (rc == DNX_EINVAL) return rc;
    for (size_t k = 0; k < len; k++) {
      wrote_region(cmds[i + 1 + k].a[5], cmds[i + 1 + k].a[6], rows[k] * 4);
    }
  }
  if (rc == DNX_OK) {
    after_dispatch(q4 ? kKindGemvQ4I8 : kKindGemvQ8I8);
    also_ran(kKindRmsNorm);
    if (pair) {
      also_ran(q4 ? kKindGemvQ4I8 : kKindGemvQ8I8);
      also_ran(kKindSwiglu);
    } else {
      also_ran(q4 ? kKindGemvQ4I8 : kKindGemvQ8I8, (int)len - 1);
    }
  }
  wrote_region(out, outOff, cols * 4);
  if (rc != DNX_OK) LOG("rms_norm + %zu matmuls of width %ld failed (%d)\n", len, (long)cols, rc);
  return rc;
}

// Fusion of a residual add and the RMSNorm of its result (GpuForward.forward
// adds the block's output into x, then norms x for the next block,
// gpu.dart:1180-1187): dnx_add_rms_norm, when the norm reads exactly the
// add's destination, does not accumulate, and m, x and out do not overlap.
bool fusable_add_norm(const Cmd& a, const Cmd& b) {
  if (a.op != kOpAdd || b.op != kOpRmsNorm || b.a[9] != 0) return false;
  const int64_t m = a.a[0], mOff = a.a[1], x = a.a[2], xOff = a.a[3], count = a.a[4];
  const int64_t out = b.a[4], outOff = b.a[5], rows = b.a[6], cols = b.a[7];
  if (b.a[0] != x || b.a[1] != xOff || rows * cols != count) return false;
  const int64_t bytes = count * 4;
  return !overlaps(m, mOff, bytes, x, xOff, bytes) && !overlaps(out, outOff, bytes, x, xOff, bytes) &&
         !overlaps(out, outOff, bytes, m, mOff, bytes);
}

int run_add_norm(const Cmd& a, const Cmd& b) {
  const int64_t m = a.a[0], mOff = a.a[1], x = a.a[2], xOff = a.a[3], count = a.a[4];
  const int64_t w = b.a[2], wOff = b.a[3], out = b.a[4], outOff = b.a[5], rows = b.a[6];
  const int64_t cols = b.a[7];
  const double eps = __builtin_bit_cast(double, b.a[8]);
  read_region(m, mOff, count * 4);
  read_region(x, xOff, count * 4);
  read_region(w, wOff, cols * 4);
  // With the panel of out when the next command is a prefill matmul of it.
  bool panel = next_reads_panel(out, outOff, rows, cols);
  int rc = DNX_EINVAL;
  if (panel) {
    gPanel = PanelKey{};
    rc = dnx_add_rms_norm_f6panel((const float*)dev_at(m, mOff), (float*)dev_at(x, xOff),
                                  (const float*)dev_at(w, wOff), (float*)dev_at(out, outOff), gWs,
                                  rows, cols, (float)eps, gStream);
  }
  if (rc == DNX_EINVAL) {
    panel = false;
    rc = dnx_add_rms_norm((const float*)dev_at(m, mOff), (float*)dev_at(x, xOff),
                          (const float*)dev_at(w, wOff), (float*)dev_at(out, outOff), rows, cols,
                          (float)eps, gStream);
  }
  if (rc == DNX_EINVAL) return rc;
  if (rc == DNX_OK) {
    after_dispatch(kKindRmsNorm);
    also_ran(kKindAdd);
    if (panel) also_ran(kKindQuantize);
  }
  wrote_region(x, xOff, count * 4);
  wrote_region(out, outOff, count * 4);
  if (panel && rc == DNX_OK) gPanel = PanelKey{out, outOff, rows, cols};
  if (rc != DNX_OK) LOG("add + rms_norm %ldx%ld failed (%d)\n", (long)rows, (long)cols, rc);
  return rc;
}

// Fusion of two head norm + RoPE steps over one rope table (a decode step's
// q and k, gpu.dart:1162-1163) whose operands do not overlap each other or
// the weights and table they read.
int64_t head_rope_bytes(const Cmd& c) { return ((c.a[10] - 1) * c.a[2] + c.a[8] * c.a[9]) * 4; }

bool fusable_rope_pair(const Cmd& a, const Cmd& b) {
  if (a.op != kOpHeadNormRope || b.op != kOpHeadNormRope) return false;
  for (int k = 5; k <= 11; k++) {
    if (k != 8 && a.a[k] != b.a[k]) return false;  // rope, stride, hd, n, eps; heads may differ
  }
  if (a.a[10] <= 0) return false;
  const int64_t ab = head_rope_bytes(a), bb = head_rope_bytes(b);
  const int64_t rb = ((a.a[10] - 1) * a.a[7] + a.a[9]) * 4, wb = a.a[9] * 4;
  return !overlaps(a.a[0], a.a[1], ab, b.a[0], b.a[1], bb) &&
         !overlaps(a.a[0], a.a[1], ab, a.a[5], a.a[6], rb) &&
         !overlaps(b.a[0], b.a[1], bb, a.a[5], a.a[6], rb) &&
         !overlaps(a.a[0], a.a[1], ab, b.a[3], b.a[4], wb) &&
         !overlaps(b.a[0], b.a[1], bb, a.a[3], a.a[4], wb);
}

int run_rope_pair(const Cmd& a, const Cmd& b) {
  const int64_t rope = a.a[5], ropeOff = a.a[6], ropeStride = a.a[7], hd = a.a[9], n = a.a[10];
  const double eps = __builtin_bit_cast(double, a.a[11]);
  const int64_t ab = head_rope_bytes(a), bb = head_rope_bytes(b);
  read_region(a.a[0], a.a[1], ab);
  read_region(b.a[0], b.a[1], bb);
  read_region(a.a[3], a.a[4], hd * 4);
  read_region(b.a[3], b.a[4], hd * 4);
  read_region(rope, ropeOff, ((n - 1) * ropeStride + hd) * 4);
  const int rc = dnx_head_norm_rope2(
      (float*)dev_at(a.a[0], a.a[1]), a.a[2], (const float*)dev_at(a.a[3], a.a[4]), a.a[8],
      (float*)dev_at(b.a[0], b.a[1]), b.a[2], (const float*)dev_at(b.a[3], b.a[4]), b.a[8],
      (const float*)dev_at(rope, ropeOff), ropeStride, hd, n, (float)eps, gStream);
  if (rc == DNX_EINVAL) return rc;
  if (rc == DNX_OK) {
    after_dispatch(kKindHeadNormRope);
    also_ran(kKindHeadNormRope);
  }
  wrote_region(a.a[0], a.a[1], ab);
  wrote_region(b.a[0], b.a[1], bb);
  if (rc != DNX_OK) LOG("head norm + rope pair failed (%d)\n", rc);
  return rc;
}

// Fusion of a decode token's q and k head norms + RoPE with its attention
// (gpu.dart:1157-1175): the norm of q (offset 0, the attention's q), the
// norm of the token's key row keys[position] with the same rope row, hd and
// eps, then the one-token attention over them. dnx_attention_rope norms
// both inside the split-key attention and leaves q, the key row and out as
// the three dispatches would. out and gate must not share a buffer with q
// or the keys, the norm weights and rope table must not lie in q's or the
// keys' buffers, and out shares no buffer with anything the launch reads.
bool fusable_rope_attention(const Cmd& a, const Cmd& b, const Cmd& c) {
  if (a.op != kOpHeadNormRope || b.op != kOpHeadNormRope || c.op != kOpAttention) return false;
  const int64_t q = c.a[0], keys = c.a[1], values = c.a[2], gate = c.a[3], out = c.a[4];
  const int64_t position = c.a[5], n = c.a[6], heads = c.a[7], kvHeads = c.a[8], hd = c.a[9];
  if (n != 1 || a.a[10] != 1 || b.a[10] != 1) return false;
  if (a.a[0] != q || a.a[1] != 0 || a.a[8] != heads || a.a[9] != hd) return false;
  if (b.a[0] != keys || b.a[1] != position * kvHeads * hd * 4 || b.a[8] != kvHeads ||
      b.a[9] != hd) {
    return false;
  }
  for (int k = 5; k <= 7; k++) {
    if (a.a[k] != b.a[k]) return false;  // rope table, offset, stride
  }
  if (a.a[11] != b.a[11] || q == keys || q == values || keys == values) return false;
  for (const int64_t h : {out, gate, a.a[3], b.a[3], a.a[5]}) {
    if (h == q || h == keys) return false;
  }
  // out is written while the norm weights, the rope table, the gate and the
  // values are read: no shared buffer.
  for (const int64_t h : {values, gate, a.a[3], b.a[3], a.a[5]}) {
    if (h == out) return false;
  }
  return true;
}

// DNX_OK, or the launcher's code; DNX_EINVAL means nothing was launched.
int run_rope_attention(const Cmd& a, const Cmd& b, const Cmd& c) {
  const int64_t q = c.a[0], keys = c.a[1], values = c.a[2], gate = c.a[3], out = c.a[4];
  const int64_t position = c.a[5], heads = c.a[7], kvHeads = c.a[8], hd = c.a[9];
  const int64_t window = c.a[10];
  const int64_t rope = a.a[5], ropeOff = a.a[6];
  const double eps = __builtin_bit_cast(double, a.a[11]);
  const int64_t kvBytes = (position + 1) * kvHeads * hd * 4;
  read_region(q, 0, heads * hd * 4);
  read_region(keys, 0, kvBytes);
  read_region(values, 0, kvBytes);
  if (gate >= 0) read_region(gate, 0, heads * 4);
  read_region(a.a[3], a.a[4], hd * 4);
  read_region(b.a[3], b.a[4], hd * 4);
  read_region(rope, ropeOff, hd * 4);
  const int rc = dnx_attention_rope(
      (float*)dev_at(q, 0), (float*)dev_at(keys, 0), (const float*)dev_at(values, 0),
      gate >= 0 ? (const float*)dev_at(gate, 0) : nullptr, (float*)dev_at(out, 0), position,
      heads, kvHeads, hd, window, (const float*)dev_at(a.a[3], a.a[4]),
      (const float*)dev_at(b.a[3], b.a[4]), (const float*)dev_at(rope, ropeOff), (float)eps,
      gStream);
  if (rc == DNX_EINVAL) return rc;
  if (rc == DNX_OK) {
    after_dispatch(kKindAttention);
    also_ran(kKindHeadNormRope, 2);
  }
  wrote_region(q, 0, heads * hd * 4);
  wrote_region(keys, b.a[1], kvHeads * hd * 4);
  wrote_region(out, 0, heads * hd * 4);
  if (rc != DNX_OK) LOG("head norms + attention failed (%d)\n", rc);
  return rc;
}

// Fusion of a decode matmul (n = 1) and the argmax of its whole output.
bool fusable_argmax(const Cmd& a, const Cmd& b) {
  return (a.op == kOpMatmulQ8 || a.op == kOpMatmulQ4) && a.int8_inputs && b.op == kOpArgmax &&
         a.a[9] == 1 &&
         b.a[0] == a.a[5] && b.a[1] == a.a[6] && b.a[2] == a.a[7];
}

bool run_matmul_argmax(const Cmd& a, const Cmd& b) {
  const bool q4 = a.op == kOpMatmulQ4;
  const int64_t w = a.a[0], x = a.a[3], xOff = a.a[4], y = a.a[5], yOff = a.a[6];
  const int64_t rows = a.a[7], cols = a.a[8];
  use_as_weights(w);
  read_region(x, xOff, cols * 4);
  const void* qs = dev_at(w, a.a[1]);
  const void* sc = dev_at(w, a.a[2]);
  const float* xs = (const float*)dev_at(x, xOff);
  float* ys = (float*)dev_at(y, yOff);
  int64_t* out = (int64_t*)dev_at(b.a[3], b.a[4]);
  const int rc =
      q4 ? dnx_gemv_q4_argmax((const uint8_t*)qs, (const uint16_t*)sc, xs, ys, rows, cols, out,
                              gGemvArgmaxWs, gStream)
         : dnx_gemv_q8_argmax((const int8_t*)qs, (const float*)sc, xs, ys, rows, cols, out,
                              gGemvArgmaxWs, gStream);
  if (rc == DNX_OK) {
    after_dispatch(q4 ? kKindGemvQ4I8 : kKindGemvQ8I8);
    also_ran(kKindArgmax);
  }
  wrote_region(y, yOff, rows * 4);
  wrote_region(b.a[3], b.a[4], 8);
  if (rc != DNX_OK) LOG("matmul+argmax %ldx%ld failed (%d)\n", (long)rows, (long)cols, rc);
  return rc == DNX_OK;
}

bool run(const Cmd& c) {
  switch (c.op) {
    case kOpMatmulQ8:
      return run_matmul(c, false);
    case kOpMatmulQ4:
      return run_matmul(c, true);
    case kOpSwiglu: {
      const int64_t g = c.a[0], u = c.a[1], count = c.a[2];
      read_region(g, 0, count * 4);
      read_region(u, 0, count * 4);
      // With the panel of g when the next command is a prefill matmul of it
      // (a chunk's down projection).
      const int64_t pn = gNext != nullptr ? gNext->a[9] : 0;
      const int64_t pc = gNext != nullptr ? gNext->a[8] : 0;
      bool panel = pn * pc == count && next_reads_panel(g, 0, pn, pc);
      int rc = DNX_EINVAL;
      if (panel) {
        gPanel = PanelKey{};
        rc = dnx_swiglu_f6panel((float*)dev_at(g, 0), (const float*)dev_at(u, 0), gWs, pn, pc,
                                gStream);
      }
      if (rc == DNX_EINVAL) {
        panel = false;
        rc = dnx_swiglu((float*)dev_at(g, 0), (const float*)dev_at(u, 0), count, gStream);
      }
      after_dispatch(kKindSwiglu);
      if (panel && rc == DNX_OK) also_ran(kKindQuantize);
      wrote_region(g, 0, count * 4);
      if (panel && rc == DNX_OK) gPanel = PanelKey{g, 0, pn, pc};
      return rc == DNX_OK;
    }
    case kOpQuantize:
    case kOpQuantizeBf16: {
      const bool bf16 = c.op == kOpQuantizeBf16;
      const int64_t src = c.a[0], srcOff = c.a[1], qs = c.a[2], qsOff = c.a[3];
      const int64_t sc = c.a[4], scOff = c.a[5], rows = c.a[6], cols = c.a[7], pad = c.a[8];
      read_region(src, srcOff, rows * cols * (bf16 ? 2 : 4));
      const int rc =
          bf16 ? dnx_quantize_q8_bf16((const uint16_t*)dev_at(src, srcOff),
                                      (int8_t*)dev_at(qs, qsOff), (float*)dev_at(sc, scOff), rows,
                                      cols, pad, gStream)
               : dnx_quantize_q8((const float*)dev_at(src, srcOff), (int8_t*)dev_at(qs, qsOff),
                                 (float*)dev_at(sc, scOff), rows, cols, pad, gStream);
      after_dispatch(kKindQuantizeWeights);
      wrote_region(qs, qsOff, rows * pad);
      wrote_region(sc, scOff, rows * (pad / 32) * 4);
      return rc == DNX_OK;
    }
    case kOpQuantizeQ4:
    case kOpQuantizeQ4Bf16: {
      const bool bf16 = c.op == kOpQuantizeQ4Bf16;
      const int64_t src = c.a[0], srcOff = c.a[1], qs = c.a[2], qsOff = c.a[3];
      const int64_t sc = c.a[4], scOff = c.a[5], rows = c.a[6], cols = c.a[7];
      read_region(src, srcOff, rows * cols * (bf16 ? 2 : 4));
      const int rc =
          bf16 ? dnx_quantize_q4_bf16((const uint16_t*)dev_at(src, srcOff),
                                      (uint8_t*)dev_at(qs, qsOff), (uint16_t*)dev_at(sc, scOff),
                                      rows, cols, gStream)
               : dnx_quantize_q4((const float*)dev_at(src, srcOff), (uint8_t*)dev_at(qs, qsOff),
                                 (uint16_t*)dev_at(sc, scOff), rows, cols, gStream);
      after_dispatch(kKindQuantizeWeights);
      wrote_region(qs, qsOff, rows * (cols / 2));
      wrote_region(sc, scOff, rows * (cols / 32) * 2);
      return rc == DNX_OK;
    }
    case kOpQ6kToQ8: {
      const int64_t src = c.a[0], srcOff = c.a[1], qs = c.a[2], qsOff = c.a[3];
      const int64_t sc = c.a[4], scOff = c.a[5], rows = c.a[6], cols = c.a[7];
      read_region(src, srcOff, rows * (cols / 256) * 210);
      const int rc = dnx_q6k_to_q8(dev_at(src, srcOff), (int8_t*)dev_at(qs, qsOff),
                                   (float*)dev_at(sc, scOff), rows, cols, gStream);
      after_dispatch(kKindQuantizeWeights);
      wrote_region(qs, qsOff, rows * cols);
      wrote_region(sc, scOff, rows * (cols / 32) * 4);
      return rc == DNX_OK;
    }
    case kOpSplitQ8:
    case kOpSplitQ4: {
      const bool q4 = c.op == kOpSplitQ4;
      const int64_t src = c.a[0], srcOff = c.a[1], qs = c.a[2], qsOff = c.a[3];
      const int64_t sc = c.a[4], scOff = c.a[5], rows = c.a[6], cols = c.a[7];
      const int64_t count = rows * (cols / 32);
      read_region(src, srcOff, count * (q4 ? 18 : 34));
      const int rc = q4 ? dnx_split_q4_0(dev_at(src, srcOff), (uint8_t*)dev_at(qs, qsOff),
                                         (uint16_t*)dev_at(sc, scOff), count, gStream)
                        : dnx_split_q8_0(dev_at(src, srcOff), (int8_t*)dev_at(qs, qsOff),
                                         (float*)dev_at(sc, scOff), count, gStream);
      after_dispatch(kKindQuantizeWeights);
      wrote_region(qs, qsOff, count * (q4 ? 16 : 32));
      wrote_region(sc, scOff, count * (q4 ? 2 : 4));
      return rc == DNX_OK;
    }
    case kOpRmsNorm: {
      const int64_t x = c.a[0], xOff = c.a[1], w = c.a[2], wOff = c.a[3], out = c.a[4];
      const int64_t outOff = c.a[5], rows = c.a[6], cols = c.a[7], acc = c.a[9];
      const double eps = __builtin_bit_cast(double, c.a[8]);
      read_region(x, xOff, rows * cols * 4);
      read_region(w, wOff, cols * 4);
      if (acc) read_region(out, outOff, rows * cols * 4);
      // With the panel of out when the next command is a prefill matmul of
      // it (and the norm does not accumulate).
      bool panel = acc == 0 && next_reads_panel(out, outOff, rows, cols);
      int rc = DNX_EINVAL;
      if (panel) {
        gPanel = PanelKey{};
        rc = dnx_rms_norm_f6panel((const float*)dev_at(x, xOff), (const float*)dev_at(w, wOff),
                                  (float*)dev_at(out, outOff), gWs, rows, cols, (float)eps,
                                  gStream);
      }
      if (rc == DNX_EINVAL) {
        panel = false;
        rc = dnx_rms_norm((const float*)dev_at(x, xOff), (const float*)dev_at(w, wOff),
                          (float*)dev_at(out, outOff), rows, cols, (float)eps, acc != 0, gStream);
      }
      after_dispatch(kKindRmsNorm);
      if (panel && rc == DNX_OK) also_ran(kKindQuantize);
      wrote_region(out, outOff, rows * cols * 4);
      if (panel && rc == DNX_OK) gPanel = PanelKey{out, outOff, rows, cols};
      return rc == DNX_OK;
    }
    case kOpHeadNormRope: {
      const int64_t x = c.a[0], xOff = c.a[1], xStride = c.a[2], w = c.a[3], wOff = c.a[4];
      const int64_t rope = c.a[5], ropeOff = c.a[6], ropeStride = c.a[7], heads = c.a[8];
      const int64_t hd = c.a[9], n = c.a[10];
      const double eps = __builtin_bit_cast(double, c.a[11]);
      const int64_t xBytes = ((n - 1) * xStride + heads * hd) * 4;
      read_region(x, xOff, xBytes);
      read_region(w, wOff, hd * 4);
      read_region(rope, ropeOff, ((n - 1) * ropeStride + hd) * 4);
      const int rc = dnx_head_norm_rope((float*)dev_at(x, xOff), xStride,
                                        (const float*)dev_at(w, wOff),
                                        (const float*)dev_at(rope, ropeOff), ropeStride, heads,
                                        hd, n, (float)eps, gStream);
      after_dispatch(kKindHeadNormRope);
      wrote_region(x, xOff, xBytes);
      return rc == DNX_OK;
    }
    case kOpConv: {
      const int64_t bcx = c.a[0], weight = c.a[1], wOff = c.a[2], history = c.a[3], y = c.a[4];
      const int64_t width = c.a[5], k = c.a[6], n = c.a[7];
      read_region(bcx, 0, n * 3 * width * 4);
      read_region(weight, wOff, width * k * 4);
      read_region(history, 0, (k - 1) * width * 4);
      const int rc = dnx_short_conv((const float*)dev_at(bcx, 0),
                                    (const float*)dev_at(weight, wOff),
                                    (float*)dev_at(history, 0), (float*)dev_at(y, 0), width, k,
                                    n, gStream);
      after_dispatch(kKindConv);
      wrote_region(history, 0, (k - 1) * width * 4);
      wrote_region(y, 0, n * width * 4);
      return rc == DNX_OK;
    }
    case kOpAttention: {
      const int64_t q = c.a[0], keys = c.a[1], values = c.a[2], gate = c.a[3], out = c.a[4];
      const int64_t position = c.a[5], n = c.a[6], heads = c.a[7], kvHeads = c.a[8];
      const int64_t hd = c.a[9], window = c.a[10];
      const int64_t kvBytes = (position + n) * kvHeads * hd * 4;
      read_region(q, 0, n * heads * hd * 4);
      read_region(keys, 0, kvBytes);
      read_region(values, 0, kvBytes);
      if (gate >= 0) read_region(gate, 0, n * heads * 4);
      const float* gp = gate >= 0 ? (const float*)dev_at(gate, 0) : nullptr;
      // With the panel of out when the next command is a prefill matmul of
      // it (a chunk's o projection) and the attention's row combine runs.
      bool panel = next_reads_panel(out, 0, n, heads * hd);
      int rc = DNX_EINVAL;
      if (panel) {
        gPanel = PanelKey{};
        rc = dnx_attention_f6panel((const float*)dev_at(q, 0), (const float*)dev_at(keys, 0),
                                   (const float*)dev_at(values, 0), gp, (float*)dev_at(out, 0),
                                   gWs, position, n, heads, kvHeads, hd, window, gStream);
      }
      if (rc == DNX_EINVAL) {
        panel = false;
        rc = dnx_attention((const float*)dev_at(q, 0), (const float*)dev_at(keys, 0),
                           (const float*)dev_at(values, 0), gp, (float*)dev_at(out, 0), position,
                           n, heads, kvHeads, hd, window, gStream);
      }
      after_dispatch(kKindAttention);
      if (panel && rc == DNX_OK) also_ran(kKindQuantize);
      wrote_region(out, 0, n * heads * hd * 4);
      if (panel && rc == DNX_OK) gPanel = PanelKey{out, 0, n, heads * hd};
      return rc == DNX_OK;
    }
    case kOpCopy:
    case kOpAdd: {
      const int64_t src = c.a[0], srcOff = c.a[1], dst = c.a[2], dstOff = c.a[3], count = c.a[4];
      read_region(src, srcOff, count * 4);
      if (c.op == kOpAdd) read_region(dst, dstOff, count * 4);
      const int rc = c.op == kOpAdd
                         ? dnx_add((const float*)dev_at(src, srcOff),
                                   (float*)dev_at(dst, dstOff), count, gStream)
                         : dnx_copy((const float*)dev_at(src, srcOff),
                                    (float*)dev_at(dst, dstOff), count, gStream);
      after_dispatch(c.op == kOpAdd ? kKindAdd : kKindCopy);
      wrote_region(dst, dstOff, count * 4);
      return rc == DNX_OK;
    }
    case kOpSteer: {
      const int64_t x = c.a[0], xOff = c.a[1], v = c.a[2], vOff = c.a[3], rows = c.a[4];
      const int64_t cols = c.a[5], mode = c.a[6];
      const double scale = __builtin_bit_cast(double, c.a[7]);
      read_region(x, xOff, rows * cols * 4);
      read_region(v, vOff, cols * 4);
      const int rc = dnx_steer((float*)dev_at(x, xOff), (const float*)dev_at(v, vOff), rows, cols,
                               mode, (float)scale, gStream);
      after_dispatch(kKindSteer);
      wrote_region(x, xOff, rows * cols * 4);
      return rc == DNX_OK;
    }
    case kOpArgmax: {
      const int64_t x = c.a[0], xOff = c.a[1], n = c.a[2], out = c.a[3], outOff = c.a[4];
      read_region(x, xOff, n * 4);
      const int rc = dnx_argmax((const float*)dev_at(x, xOff), n, (int64_t*)dev_at(out, outOff),
                                gArgmaxWs, gStream);
      after_dispatch(kKindArgmax);
      wrote_region(out, outOff, 8);
      return rc == DNX_OK;
    }
    case kOpGelu: {
      const int64_t x = c.a[0], xOff = c.a[1], count = c.a[2];
      read_region(x, xOff, count * 4);
      const int rc = dnx_gelu((float*)dev_at(x, xOff), count, gStream);
      after_dispatch(kKindGelu);
      wrote_region(x, xOff, count * 4);
      return rc == DNX_OK;
    }
  }
  return false;
}

// Host (pageable, e.g. a mapped cache file) -> HBM for lab_gpu_wrap. Large
// regions go in kWrapChunk pieces through kWrapBuffers pinned staging
// buffers: kWrapThreads host threads copy a piece (and take its page faults)
// while the DMA engine moves the pieces before it, on a stream of its own
// (default priority). Small regions, or no staging memory, take one
// hipMemcpy. Returns when the data is in HBM.
constexpr size_t kWrapChunk = (size_t)8 << 20;
constexpr int kWrapBuffers = 4;
constexpr int kWrapThreads = 8;
void* gWrapStage[kWrapBuffers] = {};
hipEvent_t gWrapDone[kWrapBuffers];
hipStream_t gWrapStream;
bool gWrapReady = false, gWrapFailed = false;

void parallel_copy(void* dst, const void* src, size_t bytes) {
  const size_t part = ((bytes + kWrapThreads - 1) / kWrapThreads + 4095) & ~(size_t)4095;
  std::thread pool[kWrapThreads - 1];
  int started = 0;
  for (int t = 1; t < kWrapThreads; t++) {
    const size_t off = (size_t)t * part;
    if (off >= bytes) break;
    const size_t n = std::min(part, bytes - off);
    pool[started++] = std::thread([=] { memcpy((char*)dst + off, (const char*)src + off, n); });
  }
  memcpy(dst, src, std::min(part, bytes));
  for (int t = 0; t < started; t++) pool[t].join();
}

bool wrap_copy(void* dev, const void* src, size_t bytes) {
  if (bytes >= 2 * kWrapChunk && !gWrapReady && !gWrapFailed) {
    bool ok = hipStreamCreateWithFlags(&gWrapStream, hipStreamNonBlocking) == hipSuccess;
    for (int b = 0; ok && b < kWrapBuffers; b++) {
      ok = hipHostMalloc(&gWrapStage[b], kWrapChunk, hipHostMallocDefault) == hipSuccess &&
           hipEventCreate(&gWrapDone[b]) == hipSuccess;
    }
    gWrapReady = ok;
    gWrapFailed = !ok;
  }
  if (bytes < 2 * kWrapChunk || !gWrapReady) {
    return hipMemcpy(dev, src, bytes, hipMemcpyHostToDevice) == hipSuccess;
  }
  bool ok = true;
  size_t i = 0;
  for (size_t off = 0; ok && off < bytes; off += kWrapChunk, i++) {
    const int b = (int)(i % kWrapBuffers);
    if (i >= kWrapBuffers) ok = hipEventSynchronize(gWrapDone[b]) == hipSuccess;
    const size_t n = std::min(kWrapChunk, bytes - off);
    if (ok) parallel_copy(gWrapStage[b], (const char*)src + off, n);
    ok = ok && hipMemcpyAsync((char*)dev + off, gWrapStage[b], n, hipMemcpyHostToDevice,
                              gWrapStream) == hipSuccess &&
         hipEventRecord(gWrapDone[b], gWrapStream) == hipSuccess;
  }
  return hipStreamSynchronize(gWrapStream) == hipSuccess && ok;
}

}  // namespace

extern "C" {

int64_t lab_gpu_init(void) {
  if (gReady) return 1;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count < 1) {
    LOG("no HIP device\n");
    return 0;
  }
  if (hipSetDevice(0) != hipSuccess) {
    LOG("hipSetDevice(0) failed\n");
    return 0;
  }
  // Default priority: streams of other priorities are not used here.
  if (hipStreamCreateWithFlags(&gStream, hipStreamNonBlocking) != hipSuccess ||
      hipEventCreate(&gStart) != hipSuccess || hipEventCreate(&gStop) != hipSuccess) {
    LOG("stream or event creation failed\n");
    return 0;
  }
  for (int i = 0; i < kMaxProfiled; i++) {
    if (hipEventCreate(&gProfEvents[i]) != hipSuccess) {
      LOG("event creation failed\n");
      return 0;
    }
  }
  if (hipMalloc(&gArgmaxWs, (size_t)dnx_argmax_workspace_bytes(0)) != hipSuccess ||
      hipMalloc(&gGemvArgmaxWs, (size_t)dnx_gemv_argmax_workspace_bytes()) != hipSuccess ||
      hipMemset(gGemvArgmaxWs, 0, (size_t)dnx_gemv_argmax_workspace_bytes()) != hipSuccess) {
    LOG("scratch allocation failed\n");
    return 0;
  }
  const char* mode = getenv("DIANOIA_GPU_INT8_INPUTS");
  if (mode != nullptr && strcmp(mode, "0") == 0) gInt8Inputs = false;
  const long page = sysconf(_SC_PAGESIZE);
  if (page > 0) gPage = page;
  const char* track = getenv("DIANOIA_GPU_TRACK_WRITES");
  if (track == nullptr || strcmp(track, "0") != 0) {
    struct sigaction sa;
    memset(&sa, 0, sizeof(sa));
    sa.sa_sigaction = on_segv;
    sa.sa_flags = SA_SIGINFO | SA_ONSTACK | SA_RESTART;
    sigemptyset(&sa.sa_mask);
    gTrack = sigaction(SIGSEGV, &sa, &gPrevSegv) == 0;
  }
  gReady = true;
  return 1;
}

int64_t lab_gpu_buffer(int64_t bytes) {
  const int64_t h = create(bytes, true);
  if (h < 0) return -1;
  memset(gBuffers[h].host, 0, (size_t)(shadow_pages(bytes) * gPage));
  if (hipMemset(gBuffers[h].dev, 0, (size_t)bytes) != hipSuccess) {
    lab_gpu_release(h);
    return -1;
  }
  track(h);  // host and HBM both zero: every page clean
  return h;
}

int64_t lab_gpu_readback_buffer(int64_t bytes) { return lab_gpu_buffer(bytes); }

int64_t lab_gpu_wrap(void* address, int64_t bytes) {
  if (address == nullptr) return -1;
  const int64_t h = create(bytes, false);
  if (h < 0) return -1;
  if (!wrap_copy(gBuffers[h].dev, address, (size_t)bytes)) {
    lab_gpu_release(h);
    return -1;
  }
  gBuffers[h].weights = true;
  return h;
}

int64_t lab_gpu_wrap_copies(void) { return 1; }

void* lab_gpu_contents(int64_t handle) {
  if (!valid(handle)) return nullptr;
  // A caller takes views here before writing through them: a SIGSEGV
  // handler installed since the last check turns tracking off now, before
  // those writes (a write to a protected page would go to that handler).
  check_handler();
  Buffer& b = gBuffers[handle];
  if (b.host == nullptr) {
    // A wrapped buffer: its host view is made on request from HBM.
    if (!wait_pending()) return nullptr;
    if (hipHostMalloc(&b.host, (size_t)b.size, hipHostMallocDefault) != hipSuccess) {
      b.host = nullptr;
      return nullptr;
    }
    if (hipMemcpy(b.host, b.dev, (size_t)b.size, hipMemcpyDeviceToHost) != hipSuccess) {
      return nullptr;
    }
  }
  return b.host;
}

double lab_gpu_last_ms(void) { return gLastMs; }

void lab_gpu_transfer_bytes(int64_t* up, int64_t* down) {
  if (up != nullptr) *up = gUpBytes;
  if (down != nullptr) *down = gDownBytes;
}

int64_t lab_gpu_tracking_writes(void) { return gTrack ? 1 : 0; }

void lab_gpu_release(int64_t handle) {
  if (!valid(handle)) return;
  wait_pending();
  untrack(handle);
  free_prepacks(handle);
  Buffer& b = gBuffers[handle];
  (void)hipFree(b.dev);
  if (b.host) (void)hipHostFree(b.host);
  b = Buffer();
  gFree[gFreeCount++] = handle;
  gLive--;
}

int64_t lab_gpu_live_buffers(void) { return gLive; }

void lab_gpu_begin(void) {
  wait_pending();
  check_handler();  // as in lab_gpu_contents: before the host fills inputs
  gCmds.clear();
  gFailed = false;
}

int64_t lab_gpu_commit(int64_t wait) {
  if (!gReady) return 0;
  check_handler();
  gWritten.clear();
  gPanel = PanelKey{};
  gProfiled = 0;
  bool ok = !gFailed;
  (void)hipEventRecord(gStart, gStream);
  for (size_t i = 0; i < gCmds.size(); i++) {
    bool pair = false;
    if (i + 2 < gCmds.size() && fusable_pair(gCmds[i], gCmds[i + 1], gCmds[i + 2])) {
      const int rc = run_pair(gCmds[i], gCmds[i + 1]);
      if (rc == DNX_EINVAL) {  // not launched: the two matmuls and the glue as recorded
        ok = run(gCmds[i]) && ok;
        ok = run(gCmds[i + 1]) && ok;
        ok = run(gCmds[i + 2]) && ok;
      } else {
        ok = rc == DNX_OK && ok;
      }
      i += 2;
    } else if (i + 1 < gCmds.size() && fusable_argmax(gCmds[i], gCmds[i + 1])) {
      ok = run_matmul_argmax(gCmds[i], gCmds[i + 1]) && ok;
      i += 1;
    } else if (size_t len = fusable_norm_matmul(gCmds, i, pair)) {
      const int rc = run_norm_matmul(gCmds, i, len, pair);
      if (rc == DNX_EINVAL) {  // not launched: the norm alone, then what follows it
        ok = run(gCmds[i]) && ok;
      } else {
        ok = rc == DNX_OK && ok;
        i += len;
      }
    } else if (i + 1 < gCmds.size() && fusable_matmul_add(gCmds[i], gCmds[i + 1])) {
      const int rc = run_matmul_add(gCmds[i], gCmds[i + 1]);
      if (rc == DNX_EINVAL) {  // not launched: the matmul alone, then the add
        ok = run(gCmds[i]) && ok;
      } else {
        ok = rc == DNX_OK && ok;
        i += 1;
      }
    } else if (i + 1 < gCmds.size() && fusable_add_norm(gCmds[i], gCmds[i + 1])) {
      gNext = i + 2 < gCmds.size() ? &gCmds[i + 2] : nullptr;
      const int rc = run_add_norm(gCmds[i], gCmds[i + 1]);
      if (rc == DNX_EINVAL) {
        ok = run(gCmds[i]) && ok;
        ok = run(gCmds[i + 1]) && ok;
      } else {
        ok = rc == DNX_OK && ok;
      }
      i += 1;
    } else if (i + 2 < gCmds.size() &&
               fusable_rope_attention(gCmds[i], gCmds[i + 1], gCmds[i + 2])) {
      const int rc = run_rope_attention(gCmds[i], gCmds[i + 1], gCmds[i + 2]);
      if (rc == DNX_EINVAL) {  // not launched: the norms here, the attention next
        const int rp = fusable_rope_pair(gCmds[i], gCmds[i + 1])
                           ? run_rope_pair(gCmds[i], gCmds[i + 1])
                           : DNX_EINVAL;
        if (rp == DNX_EINVAL) {
          ok = run(gCmds[i]) && ok;
          ok = run(gCmds[i + 1]) && ok;
        } else {
          ok = rp == DNX_OK && ok;
        }
      } else {
        ok = rc == DNX_OK && ok;
        i += 1;
      }
      i += 1;
    } else if (i + 1 < gCmds.size() && fusable_rope_pair(gCmds[i], gCmds[i + 1])) {
      const int rc = run_rope_pair(gCmds[i], gCmds[i + 1]);
      if (rc == DNX_EINVAL) {
        ok = run(gCmds[i]) && ok;
        ok = run(gCmds[i + 1]) && ok;
      } else {
        ok = rc == DNX_OK && ok;
      }
      i += 1;
    } else if (const size_t len = fusable_multi(gCmds, i)) {
      const int rc = run_multi(gCmds, i, len);
      if (rc == DNX_EINVAL) {  // not launched: the matmuls as recorded
        for (size_t k = 0; k < len; k++) ok = run(gCmds[i + k]) && ok;
      } else {
        ok = rc == DNX_OK && ok;
      }
      i += len - 1;
    } else if (const size_t len = chunk_multi_len(gCmds, i)) {
      const int rc = run_chunk_multi(gCmds, i, len);
      if (rc == DNX_EINVAL) {  // not launched: the matmuls as recorded
        for (size_t k = 0; k < len; k++) ok = run(gCmds[i + k]) && ok;
      } else {
        ok = rc == DNX_OK && ok;
      }
      i += len - 1;
    } else {
      gNext = i + 1 < gCmds.size() ? &gCmds[i + 1] : nullptr;
      ok = run(gCmds[i]) && ok;
    }
    gNext = nullptr;
  }
  // Results back to the host views, each written byte once (regions of a
  // buffer merged where they overlap or touch). A dirty page a copy covers
  // whole is made clean (and protected) before the copy is queued.
  std::sort(gWritten.begin(), gWritten.end(), [](const Region& a, const Region& b) {
    return a.handle != b.handle ? a.handle < b.handle : a.offset < b.offset;
  });
  std::vector<Region> merged;
  for (const Region& r : gWritten) {
    if (r.bytes <= 0) continue;
    if (!merged.empty() && merged.back().handle == r.handle &&
        r.offset <= merged.back().offset + merged.back().bytes) {
      Region& m = merged.back();
      m.bytes = std::max(m.offset + m.bytes, r.offset + r.bytes) - m.offset;
    } else {
      merged.push_back(r);
    }
  }
  // The copies themselves run as one kernel per DNX_COPY_MAX regions, which
  // writes the pinned views directly (one launch per region cost about
  // 1.7 us each, some 70 per decode step).
  const void* csrc[DNX_COPY_MAX];
  void* cdst[DNX_COPY_MAX];
  int64_t cbytes[DNX_COPY_MAX];
  int pending = 0;
  auto flush = [&]() {
    if (pending == 0) return;
    if (dnx_copy_regions(csrc, cdst, cbytes, pending, gStream) != DNX_OK) {
      for (int k = 0; k < pending; k++) {  // the launch failed: copy one by one
        (void)hipMemcpyAsync(cdst[k], csrc[k], (size_t)cbytes[k], hipMemcpyDeviceToHost, gStream);
      }
    }
    pending = 0;
  };
  for (const Region& r : merged) {
    Buffer& b = gBuffers[r.handle];
    if (b.host != nullptr && r.bytes > 0) {
      if (b.tracked) {
        const int64_t end = r.offset + r.bytes;
        const int64_t p1 = end == b.size ? shadow_pages(b.size) : end / gPage;
        for (int64_t p = (r.offset + gPage - 1) / gPage; p < p1; p++) {
          if (!page_clean(r.handle, p)) make_clean(r.handle, p, p + 1);
        }
      }
      csrc[pending] = dev_at(r.handle, r.offset);
      cdst[pending] = (char*)b.host + r.offset;
      cbytes[pending] = r.bytes;
      if (++pending == DNX_COPY_MAX) flush();
      gDownBytes += r.bytes;
    }
  }
  flush();
  if (hipEventRecord(gStop, gStream) != hipSuccess) ok = false;
  gCmds.clear();
  gFailed = false;
  gPending = true;
  if (!wait) return ok ? 1 : 0;
  if (!wait_pending()) {
    LOG("waiting for the GPU failed\n");
    return 0;
  }
  return ok ? 1 : 0;
}

int64_t lab_gpu_wait(void) {
  if (!wait_pending()) {
    LOG("waiting for the GPU failed\n");
    return 0;
  }
  return 1;
}

static void enc_matmul(Op op, int64_t w, int64_t qsOffset, int64_t scalesOffset, int64_t x,
                       int64_t xOffset, int64_t y, int64_t yOffset, int64_t rows, int64_t cols,
                       int64_t n) {
  const bool q4 = op == kOpMatmulQ4;
  const int64_t blocks = cols / 32;
  const bool ok = rows > 0 && cols > 0 && n > 0 && cols % 32 == 0 &&
                  in_bounds(w, qsOffset, q4 ? rows * cols / 2 : rows * cols) &&
                  in_bounds(w, scalesOffset, rows * blocks * (q4 ? 2 : 4)) &&
                  in_bounds(x, xOffset, n * cols * 4) && in_bounds(y, yOffset, n * rows * 4) &&
                  ((uintptr_t)dev_at(w, qsOffset) % 16) == 0 &&
                  ((uintptr_t)dev_at(w, scalesOffset) % (q4 ? 2 : 4)) == 0 &&
                  (xOffset % 4) == 0 && (yOffset % 4) == 0 && grow_scratch(cols, n);
  if (!ok) {
    LOG("enc_matmul_%s: invalid arguments (rows=%ld cols=%ld n=%ld)\n", q4 ? "q4" : "q8",
        (long)rows, (long)cols, (long)n);
    gFailed = true;
    return;
  }
  if (q4 && gInt8Inputs &&
      (dnx::matmul_uses_f6(true, rows, cols, n) ||
       dnx::matmul_uses_f6_chunk(true, rows, cols, n))) {
    reserve_prepack(w, qsOffset, scalesOffset, rows, cols);
  }
  if (!q4 && gInt8Inputs && dnx::matmul_uses_i8p(false, rows, cols, n)) {
    reserve_prepack(w, qsOffset, scalesOffset, rows, cols, true);
  }
  record(op, {w, qsOffset, scalesOffset, x, xOffset, y, yOffset, rows, cols, n});
}

void lab_gpu_enc_matmul_q8(int64_t w, int64_t qsOffset, int64_t scalesOffset, int64_t x,
                           int64_t xOffset, int64_t y, int64_t yOffset, int64_t rows,
                           int64_t cols, int64_t n) {
  enc_matmul(kOpMatmulQ8, w, qsOffset, scalesOffset, x, xOffset, y, yOffset, rows, cols, n);
}

void lab_gpu_enc_matmul_q4(int64_t w, int64_t qsOffset, int64_t scalesOffset, int64_t x,
                           int64_t xOffset, int64_t y, int64_t yOffset, int64_t rows,
                           int64_t cols, int64_t n) {
  enc_matmul(kOpMatmulQ4, w, qsOffset, scalesOffset, x, xOffset, y, yOffset, rows, cols, n);
}

void lab_gpu_enc_swiglu(int64_t g, int64_t u, int64_t count) {
  if (count < 0 || !in_bounds(g, 0, count * 4) || !in_bounds(u, 0, count * 4)) {
    LOG("enc_swiglu: invalid arguments\n");
    gFailed = true;
    return;
  }
  record(kOpSwiglu, {g, u, count});
}

static void enc_quantize(Op op, int64_t src, int64_t srcOffset, int64_t qs, int64_t qsOffset,
                         int64_t scales, int64_t scalesOffset, int64_t rows, int64_t cols,
                         int64_t colsPad) {
  const int64_t esize = op == kOpQuantizeBf16 ? 2 : 4;
  const bool ok = rows >= 0 && cols > 0 && colsPad >= cols && colsPad % 32 == 0 &&
                  in_bounds(src, srcOffset, rows * cols * esize) &&
                  in_bounds(qs, qsOffset, rows * colsPad) &&
                  in_bounds(scales, scalesOffset, rows * (colsPad / 32) * 4) &&
                  srcOffset % esize == 0 && qsOffset % 4 == 0 && scalesOffset % 4 == 0;
  if (!ok) {
    LOG("enc_quantize: invalid arguments\n");
    gFailed = true;
    return;
  }
  record(op, {src, srcOffset, qs, qsOffset, scales, scalesOffset, rows, cols, colsPad});
}

void lab_gpu_enc_quantize_q8(int64_t src, int64_t srcOffset, int64_t qs, int64_t qsOffset,
                             int64_t scales, int64_t scalesOffset, int64_t rows, int64_t cols,
                             int64_t colsPad) {
  enc_quantize(kOpQuantize, src, srcOffset, qs, qsOffset, scales, scalesOffset, rows, cols,
               colsPad);
}

void lab_gpu_enc_quantize_q8_bf16(int64_t src, int64_t srcOffset, int64_t qs, int64_t qsOffset,
                                  int64_t scales, int64_t scalesOffset, int64_t rows,
                                  int64_t cols, int64_t colsPad) {
  enc_quantize(kOpQuantizeBf16, src, srcOffset, qs, qsOffset, scales, scalesOffset, rows, cols,
               colsPad);
}

static void enc_quantize_q4(Op op, int64_t src, int64_t srcOffset, int64_t qs, int64_t qsOffset,
                            int64_t scales, int64_t scalesOffset, int64_t rows, int64_t cols) {
  const int64_t esize = op == kOpQuantizeQ4Bf16 ? 2 : 4;
  const bool ok = rows >= 0 && cols > 0 && cols % 32 == 0 &&
                  in_bounds(src, srcOffset, rows * cols * esize) &&
                  in_bounds(qs, qsOffset, rows * (cols / 2)) &&
                  in_bounds(scales, scalesOffset, rows * (cols / 32) * 2) &&
                  srcOffset % esize == 0 && qsOffset % 4 == 0 && scalesOffset % 2 == 0;
  if (!ok) {
    LOG("enc_quantize_q4: invalid arguments\n");
    gFailed = true;
    return;
  }
  record(op, {src, srcOffset, qs, qsOffset, scales, scalesOffset, rows, cols});
}

void lab_gpu_enc_quantize_q4(int64_t src, int64_t srcOffset, int64_t qs, int64_t qsOffset,
                             int64_t scales, int64_t scalesOffset, int64_t rows, int64_t cols) {
  enc_quantize_q4(kOpQuantizeQ4, src, srcOffset, qs, qsOffset, scales, scalesOffset, rows, cols);
}

void lab_gpu_enc_quantize_q4_bf16(int64_t src, int64_t srcOffset, int64_t qs, int64_t qsOffset,
                                  int64_t scales, int64_t scalesOffset, int64_t rows,
                                  int64_t cols) {
  enc_quantize_q4(kOpQuantizeQ4Bf16, src, srcOffset, qs, qsOffset, scales, scalesOffset, rows,
                  cols);
}

void lab_gpu_enc_q6k_to_q8(int64_t src, int64_t srcOffset, int64_t qs, int64_t qsOffset,
                           int64_t scales, int64_t scalesOffset, int64_t rows, int64_t cols) {
  const bool ok = rows >= 0 && cols > 0 && cols % 256 == 0 &&
                  in_bounds(src, srcOffset, rows * (cols / 256) * 210) &&
                  in_bounds(qs, qsOffset, rows * cols) &&
                  in_bounds(scales, scalesOffset, rows * (cols / 32) * 4) &&
                  qsOffset % 4 == 0 && scalesOffset % 4 == 0;
  if (!ok) {
    LOG("enc_q6k_to_q8: invalid arguments\n");
    gFailed = true;
    return;
  }
  record(kOpQ6kToQ8, {src, srcOffset, qs, qsOffset, scales, scalesOffset, rows, cols});
}

static void enc_split(bool q4, int64_t src, int64_t srcOffset, int64_t qs, int64_t qsOffset,
                      int64_t scales, int64_t scalesOffset, int64_t rows, int64_t cols) {
  const int64_t count = rows >= 0 && cols > 0 ? rows * (cols / 32) : 0;
  const bool ok = rows >= 0 && cols > 0 && cols % 32 == 0 &&
                  in_bounds(src, srcOffset, count * (q4 ? 18 : 34)) &&
                  in_bounds(qs, qsOffset, count * (q4 ? 16 : 32)) &&
                  in_bounds(scales, scalesOffset, count * (q4 ? 2 : 4)) &&
                  srcOffset % 4 == 0 && qsOffset % 16 == 0 && scalesOffset % (q4 ? 2 : 4) == 0;
  if (!ok) {
    LOG("enc_split_%s: invalid arguments\n", q4 ? "q4_0" : "q8_0");
    gFailed = true;
    return;
  }
  record(q4 ? kOpSplitQ4 : kOpSplitQ8, {src, srcOffset, qs, qsOffset, scales, scalesOffset,
                                        rows, cols});
}

void lab_gpu_enc_split_q8_0(int64_t src, int64_t srcOffset, int64_t qs, int64_t qsOffset,
                            int64_t scales, int64_t scalesOffset, int64_t rows, int64_t cols) {
  enc_split(false, src, srcOffset, qs, qsOffset, scales, scalesOffset, rows, cols);
}

void lab_gpu_enc_split_q4_0(int64_t src, int64_t srcOffset, int64_t qs, int64_t qsOffset,
                            int64_t scales, int64_t scalesOffset, int64_t rows, int64_t cols) {
  enc_split(true, src, srcOffset, qs, qsOffset, scales, scalesOffset, rows, cols);
}

// The layer steps: arguments are checked here (the reference's kernels
// would read out of bounds); an invalid one fails the command buffer.
static bool fail_enc(const char* what) {
  LOG("%s: invalid arguments\n", what);
  gFailed = true;
  return false;
}

void lab_gpu_enc_rms_norm(int64_t x, int64_t xOffset, int64_t w, int64_t wOffset, int64_t out,
                          int64_t outOffset, int64_t rows, int64_t cols, double eps,
                          int64_t accumulate) {
  if (rows < 0 || cols <= 0 || !in_bounds(x, xOffset, rows * cols * 4) ||
      !in_bounds(w, wOffset, cols * 4) || !in_bounds(out, outOffset, rows * cols * 4) ||
      xOffset % 4 || wOffset % 4 || outOffset % 4) {
    fail_enc("enc_rms_norm");
    return;
  }
  record(kOpRmsNorm, {x, xOffset, w, wOffset, out, outOffset, rows, cols,
                      __builtin_bit_cast(int64_t, eps), accumulate});
}

void lab_gpu_enc_head_norm_rope(int64_t x, int64_t xOffset, int64_t xStride, int64_t w,
                                int64_t wOffset, int64_t rope, int64_t ropeOffset,
                                int64_t ropeStride, int64_t heads, int64_t hd, int64_t n,
                                double eps) {
  if (n <= 0 || heads <= 0 || hd <= 0 || hd % 2 || hd > 512 || xStride < heads * hd ||
      ropeStride < hd || !in_bounds(x, xOffset, ((n - 1) * xStride + heads * hd) * 4) ||
      !in_bounds(w, wOffset, hd * 4) ||
      !in_bounds(rope, ropeOffset, ((n - 1) * ropeStride + hd) * 4) || xOffset % 4 ||
      wOffset % 4 || ropeOffset % 4) {
    fail_enc("enc_head_norm_rope");
    return;
  }
  record(kOpHeadNormRope, {x, xOffset, xStride, w, wOffset, rope, ropeOffset, ropeStride, heads,
                           hd, n, __builtin_bit_cast(int64_t, eps)});
}

void lab_gpu_enc_conv(int64_t bcx, int64_t weight, int64_t weightOffset, int64_t history,
                      int64_t y, int64_t width, int64_t k, int64_t n) {
  if (n <= 0 || width <= 0 || k < 2 || k > 16 || !in_bounds(bcx, 0, n * 3 * width * 4) ||
      !in_bounds(weight, weightOffset, width * k * 4) ||
      !in_bounds(history, 0, (k - 1) * width * 4) || !in_bounds(y, 0, n * width * 4) ||
      weightOffset % 4) {
    fail_enc("enc_conv");
    return;
  }
  record(kOpConv, {bcx, weight, weightOffset, history, y, width, k, n});
}

void lab_gpu_enc_attention(int64_t q, int64_t keys, int64_t values, int64_t gate, int64_t out,
                           int64_t position, int64_t n, int64_t heads, int64_t kvHeads,
                           int64_t hd, int64_t window) {
  const int64_t kvBytes = (position + n) * kvHeads * hd * 4;
  if (n <= 0 || position < 0 || heads <= 0 || kvHeads <= 0 || heads % kvHeads || hd <= 0 ||
      hd % 4 || 256 % hd || window < 0 || !in_bounds(q, 0, n * heads * hd * 4) ||
      !in_bounds(keys, 0, kvBytes) || !in_bounds(values, 0, kvBytes) ||
      (gate >= 0 && !in_bounds(gate, 0, n * heads * 4)) ||
      !in_bounds(out, 0, n * heads * hd * 4)) {
    fail_enc("enc_attention");
    return;
  }
  record(kOpAttention, {q, keys, values, gate, out, position, n, heads, kvHeads, hd, window});
}

void lab_gpu_enc_copy(int64_t src, int64_t srcOffset, int64_t dst, int64_t dstOffset,
                      int64_t count) {
  if (count < 0 || !in_bounds(src, srcOffset, count * 4) ||
      !in_bounds(dst, dstOffset, count * 4) || srcOffset % 4 || dstOffset % 4) {
    fail_enc("enc_copy");
    return;
  }
  record(kOpCopy, {src, srcOffset, dst, dstOffset, count});
}

void lab_gpu_enc_add(int64_t src, int64_t srcOffset, int64_t dst, int64_t dstOffset,
                     int64_t count) {
  if (count < 0 || !in_bounds(src, srcOffset, count * 4) ||
      !in_bounds(dst, dstOffset, count * 4) || srcOffset % 4 || dstOffset % 4) {
    fail_enc("enc_add");
    return;
  }
  record(kOpAdd, {src, srcOffset, dst, dstOffset, count});
}

void lab_gpu_enc_steer(int64_t x, int64_t xOffset, int64_t v, int64_t vOffset, int64_t rows,
                       int64_t cols, int64_t mode, double scale) {
  if (rows < 0 || cols <= 0 || (mode != 0 && mode != 1) ||
      !in_bounds(x, xOffset, rows * cols * 4) || !in_bounds(v, vOffset, cols * 4) ||
      xOffset % 4 || vOffset % 4) {
    fail_enc("enc_steer");
    return;
  }
  record(kOpSteer, {x, xOffset, v, vOffset, rows, cols, mode, __builtin_bit_cast(int64_t, scale)});
}

void lab_gpu_enc_argmax(int64_t x, int64_t xOffset, int64_t n, int64_t out, int64_t outOffset) {
  if (n <= 0 || !in_bounds(x, xOffset, n * 4) || !in_bounds(out, outOffset, 8) ||
      xOffset % 4 != 0 || outOffset % 8 != 0) {
    LOG("enc_argmax: invalid arguments\n");
    gFailed = true;
    return;
  }
  record(kOpArgmax, {x, xOffset, n, out, outOffset});
}

void lab_gpu_enc_gelu(int64_t x, int64_t xOffset, int64_t count) {
  if (count < 0 || !in_bounds(x, xOffset, count * 4) || xOffset % 4 != 0) {
    LOG("enc_gelu: invalid arguments\n");
    gFailed = true;
    return;
  }
  record(kOpGelu, {x, xOffset, count});
}

void lab_gpu_set_profiling(int64_t on) { gProfiling = on != 0; }

int64_t lab_gpu_set_int8_inputs(int64_t on) {
  const int64_t was = gInt8Inputs ? 1 : 0;
  gInt8Inputs = on != 0;
  return was;
}

int64_t lab_gpu_profile(double* ms, int64_t* counts, int64_t kinds) {
  for (int64_t k = 0; k < kinds && k < kKinds; k++) {
    ms[k] = gKindMs[k];
    counts[k] = gKindCount[k];
    gKindMs[k] = 0;
    gKindCount[k] = 0;
  }
  return kKinds;
}

void lab_gpu_set_decode_rows(int64_t rows) { (void)rows; }
int64_t lab_gpu_set_q8_group(int64_t invocations) {
  (void)invocations;
  return 0;
}
int64_t lab_gpu_set_q8_vector(int64_t on) {
  (void)on;
  return 0;
}
int64_t lab_gpu_register_q8_head(int64_t w, int64_t qs, int64_t rows, int64_t cols,
                                 int64_t q4Body) {
  (void)w; (void)qs; (void)rows; (void)cols; (void)q4Body;
  return 0;
}

void lab_gpu_device_name(char* out, int64_t capacity) {
  if (out == nullptr || capacity <= 0) return;
  hipDeviceProp_t prop;
  if (gReady && hipGetDeviceProperties(&prop, 0) == hipSuccess) {
    snprintf(out, (size_t)capacity, "%s (%s)", prop.name, prop.gcnArchName);
  } else {
    snprintf(out, (size_t)capacity, "%s", "");
  }
}

int64_t lab_gpu_max_buffer_length(void) {
  size_t free_b = 0, total = 0;
  if (!gReady || hipMemGetInfo(&free_b, &total) != hipSuccess) return 0;
  return (int64_t)total;
}

// The LDS a workgroup may use.
int64_t lab_gpu_max_shared_memory(void) { return 160 * 1024; }

int64_t lab_gpu_recommended_working_set(void) { return lab_gpu_max_buffer_length(); }

int64_t lab_gpu_thermal_state(void) { return -1; }

int64_t lab_gpu_physical_memory(void) {
  return (int64_t)sysconf(_SC_PHYS_PAGES) * (int64_t)sysconf(_SC_PAGESIZE);
}

}  // extern "C"
