// wl_api.hip - the C ABI (include/windlass_hip.h): contexts, weight upload, operator dispatch.
//
// Host-side only; the kernels live in wl_gemv.hip, wl_dequant.hip, wl_gemm.hip and wl_moe.hip.
// Every entry point validates shapes on the host before anything is launched, so a kernel
// never sees an operand that does not match its grid.
#include <algorithm>
#include <atomic>
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/windlass_hip.h"
#include "wl_dequant.h"
#include "wl_fmma.h"
#include "wl_gemm.h"
#include "wl_gemv.h"
#include "wl_intdot.h"
#include "wl_layer.h"
#include "wl_moe.h"
#include "wl_probe.h"

// Bytes of padding after every weight buffer: the GEMV reads the aligned dwords around
// 2-byte-aligned fields and may touch up to 16 bytes past the last block.
static constexpr size_t kWeightPad = 256;

struct wl_weight {
  int type;
  int64_t rows;  // per expert
  int64_t cols;
  int64_t row_bytes;
  int32_t experts;
  uint8_t *dev;
  size_t bytes;  // rows * experts * row_bytes
  bool owned;    // false for a view into a stage (wl_stage_weight): the stage owns the memory
};

// One LayerStream stage slot in HBM (src/LayerStream.cs:36-59, 62-124): its tensors at their
// 64-byte aligned offsets. `copied` marks the end of the copies queued into it, `released` the
// last compute that reads it (the next copy into the slot waits for that).
struct wl_stage {
  uint8_t *dev;
  size_t bytes;
  hipEvent_t copied, released;
  bool has_release;
};

// S_PART holds the K-chunk partials of split GEMV rows, S_XB the bf16 copy of x for the GEMM,
// S_QA the 8-bit activations of the integer path, S_MSYNC the one-launch MoE's counters
// (allocated and zeroed once; every launch leaves them zero).
// S_L* are wl_layer_dev's activations (S_LO: wl_matmul_add_dev's product when the add is not
// the GEMV's own store; S_LR the router's logits and the shared expert's gate, S_LM the MoE
// FFN's output, S_LS the shared expert's).
enum { S_X = 0, S_Y, S_H, S_MOE, S_OUT, S_AUX, S_PART, S_XB, S_QA, S_ATT,
       S_LXN, S_LQ, S_LK, S_LV, S_LATT, S_LO, S_LG, S_LU, S_LR, S_LM, S_LS, S_ROWS, S_ARG, S_MSYNC, S_COUNT };

struct wl_ctx {
  int device;
  int num_cu;
  hipStream_t stream;
  hipStream_t copy;  // stage uploads (default priority), created on first use
  int int_dot;  // Transformer.IntDot (src/Transformer.cs:23)
  int float_mma;  // wl_set_float_mma: Q4_K / Q6_K decode GEMVs of 1-8 tokens on the matrix cores
  int moe_chain;  // wl_set_moe_one_launch(0): the MoE entries always run the launch chain
  bool capturing = false;  // between wl_capture_begin and wl_capture_end
  unsigned moe_launches;  // one-launch MoE launches so far (their counter sets alternate)
  bool moe_unchecked;     // one-launch MoE launches since the err word was last read
  int moe_spin = wl::MOE_SPIN;  // polls of the one-launch MoE's bounded waits
  // growable scratch (device)
  void *buf[S_COUNT];
  size_t cap[S_COUNT];
  // pinned staging of batch-step rows (positions, slots): a ring whose entries are reused only
  // after their copy has run, so the host may queue ahead
  static constexpr int kRowRing = 4;
  int32_t *rows_host = nullptr;
  size_t rows_ints = 0;  // ints per ring entry
  hipEvent_t rows_ev[kRowRing] = {};
  bool rows_used[kRowRing] = {};
  int rows_next = 0;
  // RopeTable's cache (src/Transformer.cs:396-414): cos/sin of the rotated pairs by position for
  // one RoPE setting, filled on first use of a position and reused by every layer after it; a
  // setting change refills it
  struct {
    float4 *dev = nullptr;  // [cap][wl::kRopePairs]
    int64_t cap = 0;        // positions
    std::vector<uint8_t> have;
    int n = 0;
    double base = 0.0, fs = 0.0;
    const float *freqs = nullptr;
  } rope;
};

static thread_local std::string g_err;

static int fail(int code, const char *fmt, ...) {
  char msg[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(msg, sizeof msg, fmt, ap);
  va_end(ap);
  g_err = msg;
  return code;
}

static int hip_fail(hipError_t e, const char *what) {
  return fail(WL_E_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

#define WL_HIP(call, what)                                 \
  do {                                                     \
    hipError_t e_ = (call);                                \
    if (e_ != hipSuccess) return hip_fail(e_, what);       \
  } while (0)

static const char *type_name(int t) {
  switch (t) {
    case WL_TYPE_F32: return "f32";
    case WL_TYPE_F16: return "f16";
    case WL_TYPE_BF16: return "bf16";
    case WL_TYPE_Q4_0: return "q4_0";
    case WL_TYPE_Q4_1: return "q4_1";
    case WL_TYPE_Q5_0: return "q5_0";
    case WL_TYPE_Q5_1: return "q5_1";
    case WL_TYPE_Q8_0: return "q8_0";
    case WL_TYPE_Q2_K: return "q2_K";
    case WL_TYPE_Q3_K: return "q3_K";
    case WL_TYPE_Q4_K: return "q4_K";
    case WL_TYPE_Q5_K: return "q5_K";
    case WL_TYPE_Q6_K: return "q6_K";
    case WL_TYPE_IQ2_XXS: return "iq2_xxs";
    case WL_TYPE_IQ4_NL: return "iq4_nl";
    case WL_TYPE_IQ3_S: return "iq3_s";
    case WL_TYPE_IQ2_S: return "iq2_s";
    case WL_TYPE_IQ4_XS: return "iq4_xs";
  }
  return "type";
}

extern "C" int wl_type_layout(int t, int *be, int *bb) {
  int e = 0, b = 0;
  switch (t) {
    case WL_TYPE_F32: e = 1; b = 4; break;
    case WL_TYPE_F16: case WL_TYPE_BF16: e = 1; b = 2; break;
    case WL_TYPE_Q4_0: e = 32; b = 18; break;
    case WL_TYPE_Q4_1: e = 32; b = 20; break;
    case WL_TYPE_Q5_0: e = 32; b = 22; break;
    case WL_TYPE_Q5_1: e = 32; b = 24; break;
    case WL_TYPE_Q8_0: e = 32; b = 34; break;
    case WL_TYPE_Q2_K: e = 256; b = 84; break;
    case WL_TYPE_Q3_K: e = 256; b = 110; break;
    case WL_TYPE_Q4_K: e = 256; b = 144; break;
    case WL_TYPE_Q5_K: e = 256; b = 176; break;
    case WL_TYPE_Q6_K: e = 256; b = 210; break;
    case WL_TYPE_IQ2_XXS: e = 256; b = 66; break;
    case WL_TYPE_IQ4_NL: e = 32; b = 18; break;
    case WL_TYPE_IQ3_S: e = 256; b = 110; break;
    case WL_TYPE_IQ2_S: e = 256; b = 82; break;
    case WL_TYPE_IQ4_XS: e = 256; b = 136; break;
    // known to the file format but not multiplied here (activation formats, integer and f64
    // tensors, the I-quants whose grids have no source provenance): a reader can still lay out
    // their tensors; wl_upload refuses them
    case WL_TYPE_Q8_1: e = 32; b = 36; break;
    case WL_TYPE_Q8_K: e = 256; b = 292; break;
    case WL_TYPE_IQ2_XS: e = 256; b = 74; break;
    case WL_TYPE_IQ3_XXS: e = 256; b = 98; break;
    case WL_TYPE_IQ1_S: e = 256; b = 50; break;
    case WL_TYPE_IQ1_M: e = 256; b = 56; break;
    case WL_TYPE_I8: e = 1; b = 1; break;
    case WL_TYPE_I16: e = 1; b = 2; break;
    case WL_TYPE_I32: e = 1; b = 4; break;
    case WL_TYPE_I64: case WL_TYPE_F64: e = 1; b = 8; break;
  }
  if (be) *be = e;
  if (bb) *bb = b;
  return e != 0;
}

extern "C" int wl_version(void) { return 100; }

extern "C" const char *wl_last_error(void) { return g_err.c_str(); }

extern "C" int wl_can_decode(int t) { return wl::dequant_supports(t) ? 1 : 0; }

extern "C" int wl_can_matmul(int t) { return wl::gemv_supports(t) ? 1 : 0; }

extern "C" int wl_can_int_dot(int t) { return wl::intdot_supports(t) ? 1 : 0; }

// Fault injection for the error paths: when armed with n > 0, the n-th device allocation from
// then on (weights, stages, context scratch) reports failure without allocating, once.
static std::atomic<int> g_fail_alloc{0};

static hipError_t dev_alloc(void **p, size_t bytes) {
  int n = g_fail_alloc.load();
  while (n > 0 && !g_fail_alloc.compare_exchange_weak(n, n - 1)) {
  }
  if (n == 1) {
    *p = nullptr;
    return hipErrorOutOfMemory;
  }
  return hipMalloc(p, bytes);
}

extern "C" int wl_debug_fail_alloc(int n) {
  if (n < 0) return fail(WL_E_ARG, "wl_debug_fail_alloc: n must be >= 0");
  g_fail_alloc.store(n);
  return WL_OK;
}

static int ensure(wl_ctx *c, int slot, size_t bytes) {
  if (c->cap[slot] >= bytes) return WL_OK;
  if (c->capturing)
    return fail(WL_E_ARG, "a captured call needs %zu bytes of scratch slot %d, which holds %zu: run the same calls "
                "once before the capture", bytes, slot, c->cap[slot]);
  if (c->buf[slot]) {
    hipStreamSynchronize(c->stream);
    hipFree(c->buf[slot]);
    c->buf[slot] = nullptr;
    c->cap[slot] = 0;
  }
  size_t want = bytes < 4096 ? 4096 : bytes;
  if (dev_alloc(&c->buf[slot], want) != hipSuccess) {
    c->buf[slot] = nullptr;
    return fail(WL_E_NOMEM, "cannot allocate %zu bytes of device scratch", want);
  }
  c->cap[slot] = want;
  return WL_OK;
}

// ---- The allocation-free entry point's scratch ----
// One file-scope device array per GPU, held until the process ends. In host code `scratch` only
// names the symbol: its device address on each GPU comes from hipGetSymbolAddress with that GPU
// current (wl_create, once per device), and only that address is handed to kernels.
static constexpr size_t kStaticScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];
static constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch_ptr[kMaxDevices];

// Resolves this device's copy of `scratch` (the device must be current).
static int resolve_scratch(int device) {
  if (device < 0 || device >= kMaxDevices) return fail(WL_E_ARG, "device %d is beyond the library's %d", device,
                                                       kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[device]) return WL_OK;
  void *p = nullptr;
  WL_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
  if (!p) return fail(WL_E_DEVICE, "hipGetSymbolAddress(scratch) returned no address");
  g_scratch_ptr[device] = p;
  return WL_OK;
}

static void *static_scratch(int device) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  return device >= 0 && device < kMaxDevices ? g_scratch_ptr[device] : nullptr;
}

// The scratch of one call: the context's growable slot, or (fixed non-null) the static array,
// whose size bounds what the call may need.
static int scratch_for(wl_ctx *c, int slot, size_t bytes, void *fixed, void **out) {
  if (fixed) {
    if (bytes > kStaticScratchBytes)
      return fail(WL_E_SHAPE, "this call needs %zu bytes of scratch; the allocation-free entry point has %zu",
                  bytes, kStaticScratchBytes);
    *out = fixed;
    return WL_OK;
  }
  if (int rc = ensure(c, slot, bytes)) return rc;
  *out = c->buf[slot];
  return WL_OK;
}

extern "C" int wl_create(int device, wl_ctx **out) {
  if (!out) return fail(WL_E_ARG, "wl_create: out is null");
  *out = nullptr;
  int n = 0;
  WL_HIP(hipGetDeviceCount(&n), "hipGetDeviceCount");
  if (device < 0 || device >= n) return fail(WL_E_ARG, "device %d is outside 0..%d", device, n - 1);
  WL_HIP(hipSetDevice(device), "hipSetDevice");
  wl_ctx *c = new wl_ctx();
  c->device = device;
  hipDeviceProp_t prop;
  c->num_cu = hipGetDeviceProperties(&prop, device) == hipSuccess && prop.multiProcessorCount > 0
                  ? prop.multiProcessorCount : 256;
  if (int rc = resolve_scratch(device)) {
    delete c;
    return rc;
  }
  hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete c;
    return hip_fail(e, "hipStreamCreate");
  }
  *out = c;
  return WL_OK;
}

extern "C" void wl_destroy(wl_ctx *c) {
  if (!c) return;
  hipSetDevice(c->device);
  hipStreamSynchronize(c->stream);
  for (void *&b : c->buf)
    if (b) hipFree(b);
  if (c->rows_host) hipHostFree(c->rows_host);
  if (c->rope.dev) hipFree(c->rope.dev);
  for (hipEvent_t &e : c->rows_ev)
    if (e) hipEventDestroy(e);
  hipStreamDestroy(c->stream);
  if (c->copy) {
    hipStreamSynchronize(c->copy);
    hipStreamDestroy(c->copy);
  }
  delete c;
}

extern "C" void *wl_stream(wl_ctx *c) { return c ? (void *)c->stream : nullptr; }

// After the stream has drained: the one-launch MoE's sticky err word, set when one of its
// bounded waits ran out (that launch's output is then wrong). Read once per run of such launches
// and cleared, so each failure is reported once, by the first synchronizing call after it.
static int moe_status(wl_ctx *c) {
  if (!c->moe_unchecked || !c->buf[S_MSYNC]) return WL_OK;
  c->moe_unchecked = false;
  unsigned err = 0;
  wl::MoeSync *sy = (wl::MoeSync *)c->buf[S_MSYNC];
  WL_HIP(hipMemcpyAsync(&err, &sy->err[0], sizeof(err), hipMemcpyDeviceToHost, c->stream), "copy moe status");
  WL_HIP(hipStreamSynchronize(c->stream), "moe status");
  if (!err) return WL_OK;
  static const unsigned zero = 0;
  WL_HIP(hipMemcpyAsync(&sy->err[0], &zero, sizeof(zero), hipMemcpyHostToDevice, c->stream), "clear moe status");
  WL_HIP(hipStreamSynchronize(c->stream), "clear moe status");
  return fail(WL_E_DEVICE, "moe: a workgroup of the one-launch MoE gave up waiting for its inputs; that call's "
                           "output is wrong");
}

extern "C" int wl_sync(wl_ctx *c) {
  if (!c) return fail(WL_E_ARG, "context is null");
  WL_HIP(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  return moe_status(c);
}

// F32, F16 and BF16 rows have one-value blocks in GGUF, but the GPU kernels read them in runs
// of 32 values: other lengths are refused rather than cut short.
static int float_rows_ok(int type, int64_t cols, const char *who) {
  if ((type == 0 || type == 1 || type == 30) && cols % 32)
    return fail(WL_E_UNSUPPORTED, "%s: %s rows of %lld values are not whole runs of 32 for the GPU kernels", who,
                type_name(type), (long long)cols);
  return WL_OK;
}

extern "C" int wl_upload(wl_ctx *c, int type, const void *blocks, int64_t rows, int64_t cols, int64_t row_bytes,
                         int32_t experts, wl_weight **out) {
  if (!c || !out || !blocks) return fail(WL_E_ARG, "wl_upload: null argument");
  *out = nullptr;
  int be, bb;
  if (!wl_type_layout(type, &be, &bb) || !wl::dequant_supports(type))
    return fail(WL_E_UNSUPPORTED, "Windlass cannot decode %s weights on the GPU.", type_name(type));
  if (rows <= 0 || cols <= 0 || experts <= 0) return fail(WL_E_SHAPE, "wl_upload: empty shape");
  if (cols % be) return fail(WL_E_SHAPE, "%s rows of %lld values are not whole blocks of %d", type_name(type),
                             (long long)cols, be);
  if (row_bytes != cols / be * bb)
    return fail(WL_E_SHAPE, "row_bytes %lld does not match %lld %s values (%lld)", (long long)row_bytes,
                (long long)cols, type_name(type), (long long)(cols / be * bb));
  if (cols > (1 << 30) || rows > (1 << 30)) return fail(WL_E_SHAPE, "wl_upload: dimension too large");
  if (int rc = float_rows_ok(type, cols, "wl_upload")) return rc;
  WL_HIP(hipSetDevice(c->device), "hipSetDevice");
  wl_weight *w = new wl_weight();
  w->type = type;
  w->rows = rows;
  w->cols = cols;
  w->row_bytes = row_bytes;
  w->experts = experts;
  w->bytes = (size_t)rows * (size_t)experts * (size_t)row_bytes;
  w->owned = true;
  if (dev_alloc((void **)&w->dev, w->bytes + kWeightPad) != hipSuccess) {
    delete w;
    return fail(WL_E_NOMEM, "cannot allocate %zu bytes for a %s weight", (size_t)(rows * experts * row_bytes),
                type_name(type));
  }
  hipError_t e = hipMemcpyAsync(w->dev, blocks, w->bytes, hipMemcpyHostToDevice, c->stream);
  if (e == hipSuccess) e = hipMemsetAsync(w->dev + w->bytes, 0, kWeightPad, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) {
    hipFree(w->dev);
    delete w;
    return hip_fail(e, "weight upload");
  }
  *out = w;
  return WL_OK;
}

extern "C" int wl_weight_free(wl_ctx *c, wl_weight *w) {
  if (!w) return WL_OK;
  if (c) hipStreamSynchronize(c->stream);
  if (w->owned) hipFree(w->dev);
  delete w;
  return WL_OK;
}

// ------------------------------------------------------------------------------ stages

extern "C" int wl_host_alloc(int64_t bytes, void **out) {
  if (!out || bytes <= 0) return fail(WL_E_ARG, "wl_host_alloc: bad argument");
  *out = nullptr;
  if (hipHostMalloc(out, (size_t)bytes, hipHostMallocDefault) != hipSuccess) {
    *out = nullptr;
    return fail(WL_E_NOMEM, "cannot allocate %lld bytes of pinned host memory", (long long)bytes);
  }
  return WL_OK;
}

extern "C" int wl_host_free(void *p) {
  if (p) WL_HIP(hipHostFree(p), "hipHostFree");
  return WL_OK;
}

extern "C" int wl_stage_create(wl_ctx *c, int64_t bytes, wl_stage **out) {
  if (!c || !out) return fail(WL_E_ARG, "wl_stage_create: null argument");
  *out = nullptr;
  if (bytes <= 0) return fail(WL_E_SHAPE, "wl_stage_create: empty stage");
  WL_HIP(hipSetDevice(c->device), "hipSetDevice");
  if (!c->copy) WL_HIP(hipStreamCreateWithFlags(&c->copy, hipStreamNonBlocking), "copy stream");
  wl_stage *s = new wl_stage();
  s->bytes = (size_t)bytes;
  if (dev_alloc((void **)&s->dev, s->bytes + kWeightPad) != hipSuccess) {
    delete s;
    return fail(WL_E_NOMEM, "cannot allocate a stage of %lld bytes", (long long)bytes);
  }
  hipError_t e = hipEventCreateWithFlags(&s->copied, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&s->released, hipEventDisableTiming);
  // the padding after the slot is read by the kernels' aligned windows: keep it defined
  if (e == hipSuccess) e = hipMemsetAsync(s->dev + s->bytes, 0, kWeightPad, c->copy);
  if (e == hipSuccess) e = hipEventRecord(s->copied, c->copy);
  if (e != hipSuccess) {
    hipFree(s->dev);
    delete s;
    return hip_fail(e, "stage setup");
  }
  *out = s;
  return WL_OK;
}

extern "C" int wl_stage_free(wl_ctx *c, wl_stage *s) {
  if (!s) return WL_OK;
  if (c) {
    hipStreamSynchronize(c->stream);
    if (c->copy) hipStreamSynchronize(c->copy);
  }
  hipEventDestroy(s->copied);
  hipEventDestroy(s->released);
  hipFree(s->dev);
  delete s;
  return WL_OK;
}

extern "C" int wl_stage_upload_async(wl_ctx *c, wl_stage *s, const void *host, int64_t offset, int64_t bytes) {
  if (!c || !s || !host) return fail(WL_E_ARG, "wl_stage_upload_async: null argument");
  if (offset < 0 || bytes < 0 || (size_t)(offset + bytes) > s->bytes)
    return fail(WL_E_ARG, "stage upload of %lld bytes at %lld is outside the %zu-byte slot", (long long)bytes,
                (long long)offset, s->bytes);
  if (bytes == 0) return WL_OK;
  // the slot is overwritten only after the compute that read it last (LayerStream.WaitSlot)
  if (s->has_release) WL_HIP(hipStreamWaitEvent(c->copy, s->released, 0), "wait for the slot's release");
  WL_HIP(hipMemcpyAsync(s->dev + offset, host, (size_t)bytes, hipMemcpyHostToDevice, c->copy), "stage copy");
  WL_HIP(hipEventRecord(s->copied, c->copy), "stage copy event");
  return WL_OK;
}

extern "C" int wl_stage_ready(wl_ctx *c, wl_stage *s) {
  if (!c || !s) return fail(WL_E_ARG, "wl_stage_ready: null argument");
  WL_HIP(hipStreamWaitEvent(c->stream, s->copied, 0), "wait for the stage's copies");
  return WL_OK;
}

extern "C" int wl_stage_release(wl_ctx *c, wl_stage *s) {
  if (!c || !s) return fail(WL_E_ARG, "wl_stage_release: null argument");
  WL_HIP(hipEventRecord(s->released, c->stream), "stage release event");
  s->has_release = true;
  return WL_OK;
}

extern "C" int wl_stage_sync(wl_ctx *c, wl_stage *s) {
  if (!c || !s) return fail(WL_E_ARG, "wl_stage_sync: null argument");
  WL_HIP(hipEventSynchronize(s->copied), "stage copies");
  return WL_OK;
}

extern "C" int wl_stage_weight(wl_ctx *c, wl_stage *s, int64_t offset, int type, int64_t rows, int64_t cols,
                               int64_t row_bytes, int32_t experts, wl_weight **out) {
  if (!c || !s || !out) return fail(WL_E_ARG, "wl_stage_weight: null argument");
  *out = nullptr;
  int be, bb;
  if (!wl_type_layout(type, &be, &bb) || !wl::dequant_supports(type))
    return fail(WL_E_UNSUPPORTED, "Windlass cannot decode %s weights on the GPU.", type_name(type));
  if (rows <= 0 || cols <= 0 || experts <= 0) return fail(WL_E_SHAPE, "wl_stage_weight: empty shape");
  if (cols % be) return fail(WL_E_SHAPE, "%s rows of %lld values are not whole blocks of %d", type_name(type),
                             (long long)cols, be);
  if (row_bytes != cols / be * bb)
    return fail(WL_E_SHAPE, "row_bytes %lld does not match %lld %s values (%lld)", (long long)row_bytes,
                (long long)cols, type_name(type), (long long)(cols / be * bb));
  if (cols > (1 << 30) || rows > (1 << 30)) return fail(WL_E_SHAPE, "wl_stage_weight: dimension too large");
  if (int rc = float_rows_ok(type, cols, "wl_stage_weight")) return rc;
  const size_t bytes = (size_t)rows * (size_t)experts * (size_t)row_bytes;
  // LayerStream lays tensors out at 64-byte aligned offsets (src/LayerStream.cs:64,195-201)
  if (offset < 0 || offset % 64 || (size_t)offset + bytes > s->bytes)
    return fail(WL_E_ARG, "a %zu-byte tensor at offset %lld does not fit the %zu-byte stage at 64-byte alignment",
                bytes, (long long)offset, s->bytes);
  wl_weight *w = new wl_weight();
  w->type = type;
  w->rows = rows;
  w->cols = cols;
  w->row_bytes = row_bytes;
  w->experts = experts;
  w->dev = s->dev + offset;
  w->bytes = bytes;
  w->owned = false;
  *out = w;
  return WL_OK;
}

// ------------------------------------------------------------------------------ matmul

static int check_expert(const wl_weight *w, int32_t expert) {
  if (expert < -1 || expert >= w->experts)
    return fail(WL_E_ARG, "Expert %d is outside 0..%d.", expert, w->experts - 1);
  return WL_OK;
}

// rows and base pointer of the operand WeightView (whole tensor or one expert's slice)
static void operand(const wl_weight *w, int32_t expert, const uint8_t **base, int64_t *rows) {
  if (expert < 0) {
    *base = w->dev;
    *rows = w->rows * w->experts;
  } else {
    *base = w->dev + (int64_t)expert * w->rows * w->row_bytes;
    *rows = w->rows;
  }
}

// One GEMV launch (plus its combine when rows are split along K) on the context's stream.
// With float_mma on, the Q4_K / Q6_K matrices take the matrix-core GEMV (a matrix set it does
// not take as a whole runs one matrix at a time, each on the path its format takes), so a
// matrix's arithmetic depends only on its format and the switch, never on T.
static int gemv(wl_ctx *c, const wl::GemvMat *mats, int nmat, int nm, const float *d_x, int cols, int T,
                void *fixed = nullptr) {
  if (c->float_mma) {
    if (wl::fmma_applies(mats, nmat, nm, cols)) {
      const int64_t nf = wl::fmma_scratch_floats(mats, nmat, nm, cols, T);
      void *part = nullptr;
      if (int rc = scratch_for(c, S_PART, (size_t)nf * sizeof(float), fixed, &part)) return rc;
      WL_HIP(wl::fmma_run(mats, nmat, nm, d_x, cols, cols, T, (float *)part, c->num_cu, c->stream), "gemv launch");
      return WL_OK;
    }
    bool any = false;
    for (int i = 0; i < nmat; i++) any = any || wl::fmma_applies(&mats[i], 1, nm, cols);
    if (any && nmat > 1) {
      for (int i = 0; i < nmat; i++)
        if (int rc = gemv(c, &mats[i], 1, nm, d_x, cols, T, fixed)) return rc;
      return WL_OK;
    }
  }
  const int64_t nf = wl::gemv_scratch_floats(mats, nmat, nm, cols, T);
  void *part = nullptr;
  if (nf > 0)
    if (int rc = scratch_for(c, S_PART, (size_t)nf * sizeof(float), fixed, &part)) return rc;
  WL_HIP(wl::gemv_run(mats, nmat, nm, d_x, cols, cols, T, (float *)part, c->num_cu, c->stream), "gemv launch");
  return WL_OK;
}

// The integer path runs when it is switched on and the weight has an integer kernel whose
// activation blocks fit the row (src/Transformer.cs:493).
static bool int_path(const wl_ctx *c, const wl_weight *w) {
  return c->int_dot && wl::intdot_supports(w->type) && wl::intdot_fits(w->type, (int)w->cols);
}

// FastMath.Quantize of x [T][cols] into S_QA (Q8_K when k, else Q8_0).
static int int_quantize(wl_ctx *c, const float *d_x, int T, int cols, int k, wl::QActsDev *qa,
                        void *fixed = nullptr) {
  void *buf = nullptr;
  if (int rc = scratch_for(c, S_QA, (size_t)wl::qacts_bytes(T, cols, k), fixed, &buf)) return rc;
  *qa = wl::qacts_at(buf, T, cols, k);
  WL_HIP(wl::quantize_launch(d_x, T, cols, k, *qa, c->stream), "quantize launch");
  return WL_OK;
}

// The activations of tokens t0.. within qa.
static wl::QActsDev int_tokens(const wl::QActsDev &qa, int t0, int cols, int k) {
  const int ab = k ? 256 : 32;
  // the matrix-core operand copy holds every token from 0 (it exists for one pass of at most 8)
  return wl::QActsDev{qa.q + (int64_t)t0 * cols, qa.d + (int64_t)t0 * (cols / ab),
                      qa.bsums ? qa.bsums + (int64_t)t0 * (cols / 16) : nullptr, t0 ? nullptr : qa.qf,
                      t0 ? nullptr : qa.df};
}

// Activations quantized for the integer kernels, made at most once per call and kind.
struct IntActs {
  wl::QActsDev qa[2];  // [k]: Q8_0, Q8_K
  bool made[2] = {false, false};
};

// Transformer.MatMul's integer branch (src/Transformer.cs:504-524): every (row, token) is
// FastMath.IntDot, in passes of as many tokens as a launch takes, on the activations of x
// (quantized once per call and kind). With up (same type and shape), y = silu(gate) * up per
// (row, token) instead (SwiGlu).
static int int_run(wl_ctx *c, const wl_weight *w, const uint8_t *base, const uint8_t *up_base, int64_t rows,
                   const float *d_x, IntActs &acts, int T, float *d_y, void *fixed = nullptr) {
  const int cols = (int)w->cols, k = wl::intdot_needs_k(w->type) ? 1 : 0;
  const int tp = wl::intdot_max_tokens(w->type, cols, up_base ? 2 : 1);
  if (tp < 1) return fail(WL_E_UNSUPPORTED, "integer dot: rows of %d values are too wide", cols);
  int rc;
  if (!acts.made[k]) {
    if ((rc = int_quantize(c, d_x, T, cols, k, &acts.qa[k], fixed))) return rc;
    acts.made[k] = true;
  }
  for (int t0 = 0; t0 < T; t0 += tp) {
    const int n = T - t0 < tp ? T - t0 : tp;
    const wl::QActsDev at = int_tokens(acts.qa[k], t0, cols, k);
    float *y = d_y + (int64_t)t0 * rows;
    if (up_base)
      WL_HIP(wl::intdot_swiglu_launch(w->type, base, up_base, w->row_bytes, (int)rows, cols, at, n, y, (int)rows,
                                      c->num_cu, c->stream),
             "int dot launch");
    else
      WL_HIP(wl::intdot_launch(w->type, base, w->row_bytes, (int)rows, cols, at, n, y, (int)rows, c->num_cu,
                               c->stream),
             "int dot launch");
  }
  return WL_OK;
}

static int intdot_matmul(wl_ctx *c, const wl_weight *w, const uint8_t *base, int64_t rows, const float *d_x, int T,
                         float *d_y, void *fixed = nullptr) {
  IntActs acts;
  return int_run(c, w, base, nullptr, rows, d_x, acts, T, d_y, fixed);
}

// fixed: the static scratch (the allocation-free entry point), or null for the context's slots.
static int matmul_dev(wl_ctx *c, const wl_weight *w, int32_t expert, const float *d_x, int32_t T, float *d_y,
                      void *fixed = nullptr) {
  if (!c || !w || !d_x || !d_y) return fail(WL_E_ARG, "matmul: null argument");
  int rc = check_expert(w, expert);
  if (rc) return rc;
  if (T <= 0) return fail(WL_E_SHAPE, "MatMul shape mismatch: T = %d", T);
  if (!wl::gemv_supports(w->type) && !wl::gemm_supports(w->type))
    return fail(WL_E_UNSUPPORTED, "No GPU matmul for %s.", type_name(w->type));
  const uint8_t *base;
  int64_t rows;
  operand(w, expert, &base, &rows);
  if (int_path(c, w)) return intdot_matmul(c, w, base, rows, d_x, T, d_y, fixed);
  if (T > 8 && wl::gemm_supports(w->type)) {
    void *xb = nullptr;
    if ((rc = scratch_for(c, S_XB, (size_t)wl::gemm_scratch_bytes(w->type, (int)rows, (int)w->cols, T, c->num_cu), fixed,
                          &xb)))
      return rc;
    WL_HIP(wl::gemm_launch(w->type, base, w->row_bytes, (int)rows, (int)w->cols, d_x, T, d_y, (int)rows, xb,
                           c->num_cu, c->stream),
           "gemm launch");
    return WL_OK;
  }
  // decode GEMV in passes of up to 8 tokens (a token's result does not depend on its pass)
  for (int t0 = 0; t0 < T; t0 += 8) {
    const wl::GemvMat m{base, nullptr, w->row_bytes, (int)rows, w->type, d_y + (int64_t)t0 * rows, (int)rows};
    const int Tp = T - t0 < 8 ? T - t0 : 8;
    if ((rc = gemv(c, &m, 1, 1, d_x + (int64_t)t0 * w->cols, (int)w->cols, Tp, fixed))) return rc;
  }
  return WL_OK;
}

extern "C" int wl_matmul_dev(wl_ctx *c, const wl_weight *w, int32_t expert, const float *d_x, int32_t T,
                             float *d_y) {
  return matmul_dev(c, w, expert, d_x, T, d_y);
}

// wl_matmul_dev without any allocation: every kernel's scratch (K-chunk and wave-column
// partials, the GEMM's bf16 copy of x and its chunk partials, the integer path's quantized
// activations) is this device's static array, resolved by wl_create. A call needing more
// than the array holds is refused before anything is launched. The scratch is fully written
// before it is read, so nothing is cleared; calls that overlap on one GPU share it and race.
extern "C" int wl_matmul_dev_noalloc(wl_ctx *c, const wl_weight *w, int32_t expert, const float *d_x, int32_t T,
                                     float *d_y) {
  if (!c) return fail(WL_E_ARG, "wl_matmul_dev_noalloc: context is null");
  void *fixed = static_scratch(c->device);
  if (!fixed) return fail(WL_E_DEVICE, "device %d has no resolved static scratch", c->device);
  return matmul_dev(c, w, expert, d_x, T, d_y, fixed);
}

// d_y += (W x) * rs. Up to 8 tokens on the GEMV kernels the add is their final store; otherwise
// the product goes to scratch and the residual kernel adds it. Either way o = W x is rounded to
// float first, then x + o * rs as two roundings (src/Transformer.cs:224,231).
extern "C" int wl_matmul_add_dev(wl_ctx *c, const wl_weight *w, int32_t expert, const float *d_x, int32_t T,
                                 float *d_y, float rs) {
  if (!c || !w || !d_x || !d_y) return fail(WL_E_ARG, "wl_matmul_add_dev: null argument");
  int rc = check_expert(w, expert);
  if (rc) return rc;
  if (T <= 0) return fail(WL_E_SHAPE, "MatMul shape mismatch: T = %d", T);
  const uint8_t *base;
  int64_t rows;
  operand(w, expert, &base, &rows);
  if (T <= 8 && wl::gemv_supports(w->type) && !int_path(c, w)) {
    wl::GemvMat m{base, nullptr, w->row_bytes, (int)rows, w->type, d_y, (int)rows};
    m.add = 1;
    m.rs = rs;
    return gemv(c, &m, 1, 1, d_x, (int)w->cols, T);
  }
  if ((rc = ensure(c, S_LO, (size_t)T * rows * sizeof(float)))) return rc;
  float *o = (float *)c->buf[S_LO];
  if ((rc = matmul_dev(c, w, expert, d_x, T, o))) return rc;
  WL_HIP(wl::residual_launch(d_y, o, (int64_t)T * rows, rs, c->stream), "residual");
  return WL_OK;
}

extern "C" int wl_matmul(wl_ctx *c, const wl_weight *w, int32_t expert, const float *x, int32_t T, float *y) {
  if (!c || !w || !x || !y) return fail(WL_E_ARG, "wl_matmul: null argument");
  int rc = check_expert(w, expert);
  if (rc) return rc;
  if (T <= 0) return fail(WL_E_SHAPE, "MatMul shape mismatch: T = %d", T);
  const uint8_t *base;
  int64_t rows;
  operand(w, expert, &base, &rows);
  const size_t xb = (size_t)T * w->cols * 4, yb = (size_t)T * rows * 4;
  if ((rc = ensure(c, S_X, xb)) || (rc = ensure(c, S_Y, yb))) return rc;
  WL_HIP(hipMemcpyAsync(c->buf[S_X], x, xb, hipMemcpyHostToDevice, c->stream), "copy x");
  if ((rc = matmul_dev(c, w, expert, (const float *)c->buf[S_X], T, (float *)c->buf[S_Y]))) return rc;
  WL_HIP(hipMemcpyAsync(y, c->buf[S_Y], yb, hipMemcpyDeviceToHost, c->stream), "copy y");
  WL_HIP(hipStreamSynchronize(c->stream), "matmul");
  return WL_OK;
}

extern "C" int wl_matmul_multi_dev(wl_ctx *c, int32_t n, const wl_weight *const *ws, const float *d_x, int32_t T,
                                   float *const *d_ys) {
  if (!c || !ws || !d_x || !d_ys) return fail(WL_E_ARG, "wl_matmul_multi_dev: null argument");
  if (n <= 0 || n > wl::GEMV_MAX_MATS) return fail(WL_E_ARG, "wl_matmul_multi_dev: n = %d outside 1..%d", n,
                                                   wl::GEMV_MAX_MATS);
  if (T <= 0 || T > 8) return fail(WL_E_SHAPE, "wl_matmul_multi_dev: T = %d outside 1..8", T);
  bool same = true, mixed_ok = true;
  for (int i = 0; i < n; i++) {
    if (!ws[i] || !d_ys[i]) return fail(WL_E_ARG, "wl_matmul_multi_dev: null weight or output %d", i);
    if (ws[i]->cols != ws[0]->cols) return fail(WL_E_SHAPE, "MatMul shape mismatch: fused matrices read different x");
    if (!wl::gemv_supports(ws[i]->type)) return fail(WL_E_UNSUPPORTED, "No GPU matmul for %s.", type_name(ws[i]->type));
    same = same && ws[i]->type == ws[0]->type;
    mixed_ok = mixed_ok && wl::gemv_mixed_supports(ws[i]->type);
  }
  bool any_int = false, all_int = true;
  int types[wl::GEMV_MAX_MATS];
  for (int i = 0; i < n; i++) {
    any_int = any_int || int_path(c, ws[i]);
    all_int = all_int && int_path(c, ws[i]);
    types[i] = ws[i]->type;
  }
  const int cols = (int)ws[0]->cols;
  if (all_int && n > 1 && wl::intmma_multi_supports(types, n, cols, T)) {
    // every matrix on the int8 matrix cores in one launch, on activations quantized once
    wl::QActsDev qa;
    if (int rc = int_quantize(c, d_x, T, cols, 1, &qa)) return rc;
    wl::MmaMat mats[3];
    for (int i = 0; i < n; i++) {
      const int rows = (int)(ws[i]->rows * ws[i]->experts);
      mats[i] = wl::MmaMat{ws[i]->dev, ws[i]->row_bytes, rows, ws[i]->type, d_ys[i], rows};
    }
    WL_HIP(wl::intmma_multi_launch(mats, n, cols, qa, T, c->stream), "int dot launch");
    return WL_OK;
  }
  if (any_int) {
    // the integer matrices share the activations; the others take the float path one by one
    IntActs acts;
    for (int i = 0; i < n; i++) {
      int rc = int_path(c, ws[i]) ? int_run(c, ws[i], ws[i]->dev, nullptr, ws[i]->rows * ws[i]->experts, d_x, acts,
                                            T, d_ys[i])
                                  : matmul_dev(c, ws[i], -1, d_x, T, d_ys[i]);
      if (rc) return rc;
    }
    return WL_OK;
  }
  if (!same && !mixed_ok) {
    for (int i = 0; i < n; i++) {
      int rc = matmul_dev(c, ws[i], -1, d_x, T, d_ys[i]);
      if (rc) return rc;
    }
    return WL_OK;
  }
  wl::GemvMat mats[wl::GEMV_MAX_MATS];
  for (int i = 0; i < n; i++) {
    const wl_weight *w = ws[i];
    const int rows = (int)(w->rows * w->experts);
    mats[i] = wl::GemvMat{w->dev, nullptr, w->row_bytes, rows, w->type, d_ys[i], rows};
  }
  return gemv(c, mats, n, 1, d_x, (int)ws[0]->cols, T);
}

extern "C" int wl_gate_up_dev(wl_ctx *c, const wl_weight *gate, const wl_weight *up, int32_t expert,
                              const float *d_x, int32_t T, float *d_h) {
  if (!c || !gate || !up || !d_x || !d_h) return fail(WL_E_ARG, "wl_gate_up_dev: null argument");
  int rc = check_expert(gate, expert);
  if (!rc) rc = check_expert(up, expert);
  if (rc) return rc;
  if (gate->type != up->type) return fail(WL_E_UNSUPPORTED, "gate and up must share a type for the fused launch");
  if (gate->rows != up->rows || gate->cols != up->cols || gate->experts != up->experts)
    return fail(WL_E_SHAPE, "MatMul shape mismatch: gate and up differ in shape");
  if (!wl::gemv_supports(gate->type)) return fail(WL_E_UNSUPPORTED, "No GPU matmul for %s.", type_name(gate->type));
  if (T <= 0) return fail(WL_E_SHAPE, "MatMul shape mismatch: T = %d", T);
  const uint8_t *gb, *ub;
  int64_t rows;
  operand(gate, expert, &gb, &rows);
  operand(up, expert, &ub, &rows);
  if (int_path(c, gate)) {
    // SwiGlu on the integer kernels: g = gate x, u = up x on the same activations, then
    // g / (1 + exp(-g)) * u once each row's terms are added
    IntActs acts;
    return int_run(c, gate, gb, ub, rows, d_x, acts, T, d_h);
  }
  for (int t0 = 0; t0 < T; t0 += 8) {
    const wl::GemvMat m{gb, ub, gate->row_bytes, (int)rows, gate->type, d_h + (int64_t)t0 * rows, (int)rows};
    const int Tp = T - t0 < 8 ? T - t0 : 8;
    if ((rc = gemv(c, &m, 1, 2, d_x + (int64_t)t0 * gate->cols, (int)gate->cols, Tp))) return rc;
  }
  return WL_OK;
}

extern "C" int wl_swiglu(wl_ctx *c, const wl_weight *gate, const wl_weight *up, const wl_weight *down,
                         int32_t expert, const float *x, int32_t T, float *out) {
  if (!c || !gate || !up || !down || !x || !out) return fail(WL_E_ARG, "wl_swiglu: null argument");
  if (T <= 0) return fail(WL_E_SHAPE, "MatMul shape mismatch: T = %d", T);
  if (down->cols != gate->rows) return fail(WL_E_SHAPE, "MatMul shape mismatch for the down projection");
  int rc = check_expert(down, expert);
  if (rc) return rc;
  const int64_t ff = gate->rows * (expert < 0 ? gate->experts : 1);
  const int64_t embd = down->rows * (expert < 0 ? down->experts : 1);
  const size_t xb = (size_t)T * gate->cols * 4, hb = (size_t)T * ff * 4, ob = (size_t)T * embd * 4;
  if ((rc = ensure(c, S_X, xb)) || (rc = ensure(c, S_H, hb)) || (rc = ensure(c, S_OUT, ob))) return rc;
  WL_HIP(hipMemcpyAsync(c->buf[S_X], x, xb, hipMemcpyHostToDevice, c->stream), "copy x");
  if (gate->type == up->type) {
    rc = wl_gate_up_dev(c, gate, up, expert, (const float *)c->buf[S_X], T, (float *)c->buf[S_H]);
  } else {
    rc = fail(WL_E_UNSUPPORTED, "gate and up of different types are not fused");
  }
  if (rc) return rc;
  if ((rc = matmul_dev(c, down, expert, (const float *)c->buf[S_H], T, (float *)c->buf[S_OUT]))) return rc;
  WL_HIP(hipMemcpyAsync(out, c->buf[S_OUT], ob, hipMemcpyDeviceToHost, c->stream), "copy out");
  WL_HIP(hipStreamSynchronize(c->stream), "swiglu");
  return WL_OK;
}

// ----------------------------------------------------------------------------- dequant

extern "C" int wl_dequant_dev(wl_ctx *c, const wl_weight *w, int64_t row0, int64_t nrows, float *d_dst) {
  if (!c || !w || !d_dst) return fail(WL_E_ARG, "wl_dequant_dev: null argument");
  const int64_t total = w->rows * w->experts;
  if (row0 < 0 || nrows < 0 || row0 + nrows > total)
    return fail(WL_E_ARG, "rows %lld..%lld are outside the tensor's %lld rows", (long long)row0,
                (long long)(row0 + nrows), (long long)total);
  WL_HIP(wl::dequant_launch(w->type, w->dev, w->row_bytes, row0, nrows, w->cols, d_dst, c->stream), "dequant launch");
  return WL_OK;
}

extern "C" int wl_dequant_f32(wl_ctx *c, const wl_weight *w, int64_t row0, int64_t nrows, float *dst) {
  if (!c || !w || !dst) return fail(WL_E_ARG, "wl_dequant_f32: null argument");
  const size_t bytes = (size_t)nrows * w->cols * 4;
  int rc = ensure(c, S_Y, bytes ? bytes : 4);
  if (rc) return rc;
  if ((rc = wl_dequant_dev(c, w, row0, nrows, (float *)c->buf[S_Y]))) return rc;
  WL_HIP(hipMemcpyAsync(dst, c->buf[S_Y], bytes, hipMemcpyDeviceToHost, c->stream), "copy dst");
  WL_HIP(hipStreamSynchronize(c->stream), "dequant");
  return WL_OK;
}

// --------------------------------------------------------------------------------- MoE

// scratch layout in S_MOE: sel | wts | prob | plan | h | yd | qx | qh (the last two: IntDot's
// quantized activations of x and h, sized for Q8_K, the larger layout)
struct MoeScratch {
  size_t sel, wts, prob, plan, h, yd, qx, qh, total;
};

static MoeScratch moe_layout(int T, int k, int ne, int ff, int embd) {
  auto al = [](size_t v) { return (v + 255) & ~size_t(255); };
  MoeScratch s{};
  size_t o = 0;
  s.sel = o; o = al(o + (size_t)T * k * 4);
  s.wts = o; o = al(o + (size_t)T * k * 4);
  s.prob = o; o = al(o + (size_t)T * ne * 4);
  s.plan = o; o = al(o + sizeof(wl::MoePlan));
  s.h = o; o = al(o + (size_t)T * k * ff * 4);
  s.yd = o; o = al(o + (size_t)T * k * embd * 4);
  const int64_t qx = wl::qacts_bytes(T, embd, 1) > wl::qacts_bytes(T, embd, 0) ? wl::qacts_bytes(T, embd, 1)
                                                                                 : wl::qacts_bytes(T, embd, 0);
  const int64_t qh = wl::qacts_bytes(T * k, ff, 1) > wl::qacts_bytes(T * k, ff, 0) ? wl::qacts_bytes(T * k, ff, 1)
                                                                                     : wl::qacts_bytes(T * k, ff, 0);
  s.qx = o; o = al(o + (size_t)qx);
  s.qh = o; o = al(o + (size_t)qh);
  s.total = o;
  return s;
}

extern "C" int wl_route(wl_ctx *c, const float *logits, int32_t T, int32_t n, int32_t k, int32_t renorm,
                        int32_t *sel, float *wts) {
  if (!c || !logits || !sel || !wts) return fail(WL_E_ARG, "wl_route: null argument");
  if (T <= 0 || n <= 0 || k <= 0 || k > n) return fail(WL_E_ARG, "wl_route: bad sizes T=%d n=%d k=%d", T, n, k);
  const size_t lb = (size_t)T * n * 4, kb = (size_t)T * k * 4;
  int rc;
  if ((rc = ensure(c, S_AUX, 2 * lb + 2 * kb + 1024))) return rc;
  uint8_t *base = (uint8_t *)c->buf[S_AUX];
  float *d_l = (float *)base;
  float *d_p = (float *)(base + lb);
  int *d_sel = (int *)(base + 2 * lb);
  float *d_w = (float *)(base + 2 * lb + kb);
  WL_HIP(hipMemcpyAsync(d_l, logits, lb, hipMemcpyHostToDevice, c->stream), "copy logits");
  WL_HIP(wl::route_launch(d_l, T, n, k, renorm, d_sel, d_w, d_p, c->stream), "route launch");
  WL_HIP(hipMemcpyAsync(sel, d_sel, kb, hipMemcpyDeviceToHost, c->stream), "copy sel");
  WL_HIP(hipMemcpyAsync(wts, d_w, kb, hipMemcpyDeviceToHost, c->stream), "copy wts");
  WL_HIP(hipStreamSynchronize(c->stream), "route");
  return WL_OK;
}

static int moe_check(const wl_weight *g, const wl_weight *u, const wl_weight *d, int32_t k) {
  if (!g || !u || !d) return fail(WL_E_ARG, "moe: null expert tensor");
  if (g->type != u->type) return fail(WL_E_UNSUPPORTED, "moe: gate and up must share a type");
  if (!wl::moe_supports(g->type) || !wl::moe_supports(d->type))
    return fail(WL_E_UNSUPPORTED, "No GPU expert matmul for %s / %s.", type_name(g->type), type_name(d->type));
  if (g->experts != u->experts || g->experts != d->experts || g->rows != u->rows || g->cols != u->cols ||
      d->cols != g->rows || d->rows != g->cols)
    return fail(WL_E_SHAPE, "MatMul shape mismatch between the expert tensors");
  if (k <= 0 || k > wl::MOE_MAX_K || k > g->experts) return fail(WL_E_ARG, "moe: k = %d outside 1..%d", k,
                                                                  g->experts < wl::MOE_MAX_K ? g->experts : wl::MOE_MAX_K);
  return WL_OK;
}

static int moe_dev(wl_ctx *c, const float *d_logits, int32_t k, int32_t renorm, const wl_weight *g,
                   const wl_weight *u, const wl_weight *d, const float *d_x, int32_t T, float *d_out) {
  int rc = moe_check(g, u, d, k);
  if (rc) return rc;
  const int ne = g->experts, ff = (int)g->rows, embd = (int)g->cols;
  if (!c->buf[S_MSYNC]) {
    if ((rc = ensure(c, S_MSYNC, sizeof(wl::MoeSync)))) return rc;
    WL_HIP(wl::moe_sync_init((wl::MoeSync *)c->buf[S_MSYNC], c->stream), "moe counters");
  }
  for (int t0 = 0; t0 < T; t0 += wl::MOE_MAX_T) {
    const int Tc = T - t0 < wl::MOE_MAX_T ? T - t0 : wl::MOE_MAX_T;
    MoeScratch s = moe_layout(Tc, k, ne, ff, embd);
    if ((rc = ensure(c, S_MOE, s.total))) return rc;
    uint8_t *b = (uint8_t *)c->buf[S_MOE];
    wl::MoeLaunch m{};
    m.logits = d_logits + (int64_t)t0 * ne;
    m.T = Tc; m.ne = ne; m.k = k; m.renorm = renorm;
    m.gu_type = g->type; m.d_type = d->type;
    m.gate = g->dev; m.up = u->dev; m.down = d->dev;
    m.gu_row_bytes = g->row_bytes; m.d_row_bytes = d->row_bytes;
    m.ff = ff; m.embd = embd;
    m.x = d_x + (int64_t)t0 * embd;
    m.out = d_out + (int64_t)t0 * embd;
    m.sel = (int *)(b + s.sel); m.wts = (float *)(b + s.wts); m.prob = (float *)(b + s.prob);
    m.plan = (wl::MoePlan *)(b + s.plan); m.h = (float *)(b + s.h); m.yd = (float *)(b + s.yd);
    // Transformer.IntDot: each product of the experts' SwiGlu whose type and width allow it
    // takes MatMul's integer branch (src/Transformer.cs:288,241-251,488-524)
    m.gu_int = c->int_dot && wl::intdot_supports(g->type) && wl::intdot_fits(g->type, embd);
    m.d_int = c->int_dot && wl::intdot_supports(d->type) && wl::intdot_fits(d->type, ff);
    m.qx = wl::qacts_at(b + s.qx, Tc, embd, wl::intdot_needs_k(g->type) ? 1 : 0);
    m.qh = wl::qacts_at(b + s.qh, Tc * k, ff, wl::intdot_needs_k(d->type) ? 1 : 0);
    // a captured graph replays fixed arguments, and the one launch's counter sets alternate
    // from call to call: captures take the launch chain (the same bits)
    m.sync = c->moe_chain || c->capturing ? nullptr : (wl::MoeSync *)c->buf[S_MSYNC];
    m.parity = (int)(c->moe_launches & 1);
    m.spin = c->moe_spin;
    // only a one-launch launch uses a counter set (and clears the other for the next one), so
    // only it moves the parity; a chain launch in between leaves the sets as they are
    const bool one = wl::moe_uses_one_launch(m);
    WL_HIP(wl::moe_launch(m, c->num_cu, c->stream), "moe launch");
    if (one) {
      c->moe_launches++;
      c->moe_unchecked = true;
    }
  }
  return WL_OK;
}

extern "C" int wl_moe_ffn_dev(wl_ctx *c, const float *d_logits, int32_t k, int32_t renorm, const wl_weight *g,
                              const wl_weight *u, const wl_weight *d, const float *d_x, int32_t T, float *d_out) {
  if (!c || !d_logits || !d_x || !d_out) return fail(WL_E_ARG, "wl_moe_ffn_dev: null argument");
  if (T <= 0) return fail(WL_E_SHAPE, "MatMul shape mismatch: T = %d", T);
  return moe_dev(c, d_logits, k, renorm, g, u, d, d_x, T, d_out);
}

extern "C" int wl_moe_ffn(wl_ctx *c, const float *logits, int32_t k, int32_t renorm, const wl_weight *g,
                          const wl_weight *u, const wl_weight *d, const float *x, int32_t T, float *out,
                          int32_t *expert_runs) {
  if (!c || !logits || !x || !out) return fail(WL_E_ARG, "wl_moe_ffn: null argument");
  if (T <= 0) return fail(WL_E_SHAPE, "MatMul shape mismatch: T = %d", T);
  int rc = moe_check(g, u, d, k);
  if (rc) return rc;
  const int ne = g->experts, embd = (int)g->cols;
  const size_t lb = (size_t)T * ne * 4, xb = (size_t)T * embd * 4;
  if ((rc = ensure(c, S_AUX, lb)) || (rc = ensure(c, S_X, xb)) || (rc = ensure(c, S_OUT, xb))) return rc;
  WL_HIP(hipMemcpyAsync(c->buf[S_AUX], logits, lb, hipMemcpyHostToDevice, c->stream), "copy logits");
  WL_HIP(hipMemcpyAsync(c->buf[S_X], x, xb, hipMemcpyHostToDevice, c->stream), "copy x");
  int runs = 0;
  for (int t0 = 0; t0 < T; t0 += wl::MOE_MAX_T) {
    const int Tc = T - t0 < wl::MOE_MAX_T ? T - t0 : wl::MOE_MAX_T;
    if ((rc = moe_dev(c, (const float *)c->buf[S_AUX] + (int64_t)t0 * ne, k, renorm, g, u, d,
                      (const float *)c->buf[S_X] + (int64_t)t0 * embd, Tc, (float *)c->buf[S_OUT] + (int64_t)t0 * embd)))
      return rc;
    if (expert_runs) {
      MoeScratch s = moe_layout(Tc, k, ne, (int)g->rows, embd);
      int ns = 0;
      WL_HIP(hipMemcpyAsync(&ns, (uint8_t *)c->buf[S_MOE] + s.plan + offsetof(wl::MoePlan, nslots), sizeof(int),
                            hipMemcpyDeviceToHost, c->stream), "copy runs");
      WL_HIP(hipStreamSynchronize(c->stream), "moe");
      runs += ns;
    }
  }
  WL_HIP(hipMemcpyAsync(out, c->buf[S_OUT], xb, hipMemcpyDeviceToHost, c->stream), "copy out");
  WL_HIP(hipStreamSynchronize(c->stream), "moe");
  if ((rc = moe_status(c))) return rc;
  if (expert_runs) *expert_runs = runs;
  return WL_OK;
}

extern "C" int wl_debug_moe_patience(wl_ctx *c, int32_t polls) {
  if (!c) return fail(WL_E_ARG, "wl_debug_moe_patience: null context");
  c->moe_spin = polls < 0 ? wl::MOE_SPIN : polls;
  return WL_OK;
}

// ----------------------------------------------------------------------------- integer path

extern "C" int wl_set_moe_one_launch(wl_ctx *c, int on) {
  if (!c) return fail(WL_E_ARG, "wl_set_moe_one_launch: null context");
  c->moe_chain = on ? 0 : 1;
  return WL_OK;
}

extern "C" int wl_set_float_mma(wl_ctx *c, int on) {
  if (!c) return fail(WL_E_ARG, "wl_set_float_mma: null context");
  c->float_mma = on ? 1 : 0;
  return WL_OK;
}

extern "C" int wl_set_int_dot(wl_ctx *c, int on) {
  if (!c) return fail(WL_E_ARG, "wl_set_int_dot: null context");
  c->int_dot = on ? 1 : 0;
  return WL_OK;
}

extern "C" int wl_quantize_dev(wl_ctx *c, const float *d_x, int32_t T, int32_t cols, int32_t k, int8_t *d_q,
                               float *d_d, int16_t *d_bsums) {
  if (!c || !d_x || !d_q || !d_d || (k && !d_bsums)) return fail(WL_E_ARG, "wl_quantize_dev: null argument");
  if (T < 0 || cols <= 0 || cols % (k ? 256 : 32))
    return fail(WL_E_SHAPE, "Quantize: %d columns are not whole %d-value blocks", cols, k ? 256 : 32);
  WL_HIP(wl::quantize_launch(d_x, T, cols, k ? 1 : 0, wl::QActsDev{d_q, d_d, d_bsums}, c->stream), "quantize launch");
  return WL_OK;
}

extern "C" int wl_quantize(wl_ctx *c, const float *x, int32_t T, int32_t cols, int32_t k, int8_t *q, float *d,
                           int16_t *bsums) {
  if (!c || !x || !q || !d || (k && !bsums)) return fail(WL_E_ARG, "wl_quantize: null argument");
  if (T < 0 || cols <= 0 || cols % (k ? 256 : 32))
    return fail(WL_E_SHAPE, "Quantize: %d columns are not whole %d-value blocks", cols, k ? 256 : 32);
  if (T == 0) return WL_OK;
  const int kk = k ? 1 : 0, bs = kk ? 256 : 32;
  const size_t xb = (size_t)T * cols * 4;
  int rc;
  if ((rc = ensure(c, S_X, xb)) || (rc = ensure(c, S_QA, (size_t)wl::qacts_bytes(T, cols, kk)))) return rc;
  const wl::QActsDev qa = wl::qacts_at(c->buf[S_QA], T, cols, kk);
  WL_HIP(hipMemcpyAsync(c->buf[S_X], x, xb, hipMemcpyHostToDevice, c->stream), "copy x");
  WL_HIP(wl::quantize_launch((const float *)c->buf[S_X], T, cols, kk, qa, c->stream), "quantize launch");
  WL_HIP(hipMemcpyAsync(q, qa.q, (size_t)T * cols, hipMemcpyDeviceToHost, c->stream), "copy q");
  WL_HIP(hipMemcpyAsync(d, qa.d, (size_t)T * (cols / bs) * 4, hipMemcpyDeviceToHost, c->stream), "copy d");
  if (kk)
    WL_HIP(hipMemcpyAsync(bsums, qa.bsums, (size_t)T * (cols / 16) * 2, hipMemcpyDeviceToHost, c->stream),
           "copy bsums");
  WL_HIP(hipStreamSynchronize(c->stream), "quantize");
  return WL_OK;
}

// ----------------------------------------------------------------- the rest of a layer

extern "C" int wl_rms_norm_dev(wl_ctx *c, const float *d_x, int64_t rows, int64_t dim, const float *d_w, float eps,
                               float *d_y) {
  if (!c || !d_x || !d_w || !d_y) return fail(WL_E_ARG, "wl_rms_norm_dev: null argument");
  if (rows < 0 || dim <= 0) return fail(WL_E_SHAPE, "wl_rms_norm_dev: %lld rows of %lld", (long long)rows,
                                        (long long)dim);
  WL_HIP(wl::rms_norm_launch(d_x, rows, dim, d_w, eps, d_y, c->stream), "rms norm");
  return WL_OK;
}

extern "C" int wl_rope_dev(wl_ctx *c, float *d_x, int32_t T, int32_t heads, int32_t head_dim, int32_t rope_dims,
                           int32_t neox, int32_t pos0, const int32_t *d_pos, double base, double freq_scale,
                           const float *d_freqs) {
  if (!c || !d_x) return fail(WL_E_ARG, "wl_rope_dev: null argument");
  if (T < 0 || heads <= 0 || head_dim <= 0 || rope_dims <= 0 || rope_dims > head_dim || rope_dims % 2)
    return fail(WL_E_SHAPE, "wl_rope_dev: %d rotated of %d per head", rope_dims, head_dim);
  WL_HIP(wl::rope_launch(d_x, (int64_t)heads * head_dim, T, heads, head_dim, rope_dims, neox, d_pos, pos0, base,
                         freq_scale, d_freqs, c->stream),
         "rope");
  return WL_OK;
}

extern "C" int wl_kv_store_dev(wl_ctx *c, const float *d_k, const float *d_v, int32_t T, int32_t kv_dim,
                               uint16_t *d_K, uint16_t *d_V, int32_t pos0) {
  if (!c || !d_k || !d_v || !d_K || !d_V) return fail(WL_E_ARG, "wl_kv_store_dev: null argument");
  if (T < 0 || kv_dim <= 0 || pos0 < 0) return fail(WL_E_SHAPE, "wl_kv_store_dev: bad shape");
  const int64_t off = (int64_t)pos0 * kv_dim;
  WL_HIP(wl::kv_store_launch(d_k, d_v, (int64_t)T * kv_dim, d_K + off, d_V + off, c->stream), "kv store");
  return WL_OK;
}

extern "C" int wl_attention_dev(wl_ctx *c, const float *d_q, int32_t T, int32_t heads, int32_t kv_heads,
                                int32_t head_dim, const uint16_t *d_K, const uint16_t *d_V, int32_t pos0, float scale,
                                float *d_out) {
  if (!c || !d_q || !d_K || !d_V || !d_out) return fail(WL_E_ARG, "wl_attention_dev: null argument");
  if (T < 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads || head_dim <= 0 || pos0 < 0)
    return fail(WL_E_SHAPE, "wl_attention_dev: %d heads over %d KV heads", heads, kv_heads);
  const int kv_dim = kv_heads * head_dim;
  int rc = ensure(c, S_ATT,
                  (size_t)wl::attention_scratch_floats(T, heads, head_dim, kv_dim, pos0 + T, d_K, d_V) * sizeof(float));
  if (rc) return rc;
  const int64_t qd = (int64_t)heads * head_dim;
  WL_HIP(wl::attention_launch(d_q, qd, T, d_K, d_V, kv_heads * head_dim, heads, kv_heads, head_dim, pos0, scale,
                              (float *)c->buf[S_ATT], d_out, qd, wl::RowMap{}, pos0 + T, c->stream),
         "attention");
  return WL_OK;
}

extern "C" int wl_scale_dev(wl_ctx *c, float *d_x, int64_t n, float s) {
  if (!c || !d_x) return fail(WL_E_ARG, "wl_scale_dev: null argument");
  if (n < 0) return fail(WL_E_SHAPE, "wl_scale_dev: n = %lld", (long long)n);
  WL_HIP(wl::scale_launch(d_x, n, s, c->stream), "scale");
  return WL_OK;
}

extern "C" int wl_residual_dev(wl_ctx *c, float *d_x, const float *d_o, int64_t n, float rs) {
  if (!c || !d_x || !d_o) return fail(WL_E_ARG, "wl_residual_dev: null argument");
  WL_HIP(wl::residual_launch(d_x, d_o, n, rs, c->stream), "residual");
  return WL_OK;
}

extern "C" int wl_argmax_dev(wl_ctx *c, const float *d_logits, int32_t rows, int64_t n, int32_t *d_out) {
  if (!c || !d_logits || !d_out) return fail(WL_E_ARG, "wl_argmax_dev: null argument");
  if (rows < 0 || n <= 0) return fail(WL_E_SHAPE, "wl_argmax_dev: bad shape");
  int rc = ensure(c, S_ARG, (size_t)2 * (rows > 0 ? rows : 1) * wl::argmax_parts(n) * sizeof(float));
  if (rc) return rc;
  WL_HIP(wl::argmax_launch(d_logits, rows, n, d_out, (float *)c->buf[S_ARG], c->stream), "argmax");
  return WL_OK;
}

// Two host int32 arrays of n values each (the second may be null) copied to S_ROWS on the
// context's stream through the pinned ring: the host may reuse its arrays on return and queue
// ahead; a ring entry is rewritten only after its copy has run.
static int stage_rows(wl_ctx *c, const int32_t *a, const int32_t *b, int n, int32_t **d_rows) {
  const int words = b ? 2 * n : n;
  int rc;
  if ((rc = ensure(c, S_ROWS, (size_t)words * sizeof(int32_t)))) return rc;
  int32_t *rows = (int32_t *)c->buf[S_ROWS];
  if ((size_t)words > c->rows_ints) {  // grow the pinned ring (after every queued copy from it)
    WL_HIP(hipStreamSynchronize(c->stream), "row staging");
    if (c->rows_host) hipHostFree(c->rows_host);
    c->rows_host = nullptr;
    c->rows_ints = 0;
    const size_t ints = (size_t)words < 1024 ? 1024 : (size_t)words;
    WL_HIP(hipHostMalloc((void **)&c->rows_host, ints * wl_ctx::kRowRing * sizeof(int32_t), hipHostMallocDefault),
           "row staging");
    c->rows_ints = ints;
    for (bool &u : c->rows_used) u = false;
  }
  const int e = c->rows_next;
  c->rows_next = (e + 1) % wl_ctx::kRowRing;
  if (!c->rows_ev[e]) WL_HIP(hipEventCreateWithFlags(&c->rows_ev[e], hipEventDisableTiming), "row staging");
  if (c->rows_used[e]) WL_HIP(hipEventSynchronize(c->rows_ev[e]), "row staging");
  int32_t *stage = c->rows_host + (size_t)e * c->rows_ints;
  memcpy(stage, a, (size_t)n * sizeof(int32_t));
  if (b) memcpy(stage + n, b, (size_t)n * sizeof(int32_t));
  WL_HIP(hipMemcpyAsync(rows, stage, (size_t)words * sizeof(int32_t), hipMemcpyHostToDevice, c->stream), "row copy");
  WL_HIP(hipEventRecord(c->rows_ev[e], c->stream), "row staging");
  c->rows_used[e] = true;
  *d_rows = rows;
  return WL_OK;
}

extern "C" int wl_embed_dev(wl_ctx *c, const wl_weight *embd, const int32_t *tokens, int32_t T, float *d_x) {
  if (!c || !embd || !tokens || !d_x) return fail(WL_E_ARG, "wl_embed_dev: null argument");
  if (T < 0) return fail(WL_E_SHAPE, "wl_embed_dev: T = %d", T);
  for (int t = 0; t < T; t++)
    if (tokens[t] < 0 || tokens[t] >= embd->rows * embd->experts)
      return fail(WL_E_ARG, "Token id %d is outside the vocabulary.", tokens[t]);
  if (T == 0) return WL_OK;
  int32_t *d_ids;  // the checked ids, staged to the device: every row in one launch
  int rc = stage_rows(c, tokens, nullptr, T, &d_ids);
  if (rc) return rc;
  return wl_embed_dev_ids(c, embd, d_ids, T, d_x);
}

extern "C" int wl_embed_dev_ids(wl_ctx *c, const wl_weight *embd, const int32_t *d_tokens, int32_t T, float *d_x) {
  if (!c || !embd || !d_tokens || !d_x) return fail(WL_E_ARG, "wl_embed_dev_ids: null argument");
  if (T < 0) return fail(WL_E_SHAPE, "wl_embed_dev_ids: T = %d", T);
  WL_HIP(wl::dequant_rows_launch(embd->type, embd->dev, embd->row_bytes, d_tokens, T, embd->rows * embd->experts,
                                 embd->cols, d_x, c->stream),
         "embedding rows");
  return WL_OK;
}

// Transformer.Layer (src/Transformer.cs:177-232) with every activation in HBM. rm/max_n: the
// rows' positions and cache slots (a batch step) and the most positions a row attends to;
// each: every product in GEMV passes of at most 8 rows, so a row's bits do not depend on the
// batch (ForwardBatch's EachToken, src/Transformer.cs:127-170).
// The rows' RoPE angles in the context's table: positions hpos[0..T-1] (host values), or pos0 ..
// pos0 + T - 1 when hpos is null. Missing positions are filled by one launch over their range,
// queued before the caller's launches that read them.
static int rope_angles(wl_ctx *c, const int32_t *hpos, int T, int pos0, int n, double base, double fs,
                       const float *freqs, const float4 **tab) {
  auto &R = c->rope;
  if (R.n != n || R.base != base || R.fs != fs || R.freqs != freqs) {
    std::fill(R.have.begin(), R.have.end(), (uint8_t)0);
    R.n = n;
    R.base = base;
    R.fs = fs;
    R.freqs = freqs;
  }
  int top = 0, lo = -1, hi = -1;
  for (int i = 0; i < T; i++) {
    const int p = hpos ? hpos[i] : pos0 + i;
    if (p + 1 > top) top = p + 1;
  }
  if (top > R.cap) {
    if (c->capturing)
      return fail(WL_E_ARG, "a captured call needs RoPE angles of %d positions, the table holds %lld: run the same "
                  "calls once before the capture", top, (long long)R.cap);
    const int64_t cap = ((int64_t)top + 4095) / 4096 * 4096;
    if (R.dev) {
      hipStreamSynchronize(c->stream);
      hipFree(R.dev);
      R.dev = nullptr;
      R.cap = 0;
    }
    void *d = nullptr;
    if (dev_alloc(&d, (size_t)cap * wl::kRopePairs * sizeof(float4)) != hipSuccess)
      return fail(WL_E_NOMEM, "cannot allocate the RoPE table of %lld positions", (long long)cap);
    R.dev = (float4 *)d;
    R.cap = cap;
    R.have.assign((size_t)cap, 0);
  }
  for (int i = 0; i < T; i++) {
    const int p = hpos ? hpos[i] : pos0 + i;
    if (!R.have[p]) {
      lo = lo < 0 || p < lo ? p : lo;
      hi = p > hi ? p : hi;
    }
  }
  if (hi >= 0) {
    WL_HIP(wl::rope_table_launch(R.dev, lo, hi - lo + 1, n, base, fs, freqs, c->stream), "rope table");
    for (int p = lo; p <= hi; p++) R.have[p] = 1;
  }
  *tab = R.dev;
  return WL_OK;
}

static int layer_run(wl_ctx *c, const wl_layer_desc *L, float *d_x, int32_t T, int32_t pos0, uint16_t *d_K,
                     uint16_t *d_V, const wl::RowMap &rm, const int32_t *hpos, int max_n, bool each) {
  if (!c || !L || !d_x || !d_K || !d_V) return fail(WL_E_ARG, "wl_layer_dev: null argument");
  // OLMo 2 (src/Transformer.cs:182,224-230): post-norms instead of pre-norms
  const bool post = L->d_post_attention_norm || L->d_post_ffw_norm;
  if (!L->attn_q || !L->attn_k || !L->attn_v || !L->attn_output || !L->ffn_gate || !L->ffn_up || !L->ffn_down ||
      (post ? !(L->d_post_attention_norm && L->d_post_ffw_norm) : !(L->d_attn_norm && L->d_ffn_norm)))
    return fail(WL_E_ARG, "wl_layer_dev: a required tensor is missing");
  const int E = L->embd, H = L->heads, KH = L->kv_heads, HD = L->head_dim;
  if (T <= 0 || pos0 < 0 || E <= 0 || H <= 0 || KH <= 0 || H % KH || HD <= 0)
    return fail(WL_E_SHAPE, "wl_layer_dev: bad shape");
  const int QD = H * HD, KD = KH * HD;
  const bool moe = L->ffn_gate_inp != nullptr;
  const bool shared = moe && L->ffn_gate_shexp;
  int64_t FF = L->ffn_gate->rows;
  if (L->attn_q->cols != E || L->attn_q->rows != QD || L->attn_k->rows != KD || L->attn_v->rows != KD ||
      L->attn_output->cols != QD || L->attn_output->rows != E || L->ffn_gate->cols != E || L->ffn_up->rows != FF ||
      L->ffn_down->cols != FF || L->ffn_down->rows != E)
    return fail(WL_E_SHAPE, "wl_layer_dev: tensor shapes do not match the layer");
  if (moe) {
    // the router's shape here; moe_dev checks the experts and expert_used
    if (L->ffn_gate_inp->cols != E || L->ffn_gate_inp->rows != L->ffn_gate->experts || L->ffn_gate_inp->experts != 1)
      return fail(WL_E_SHAPE, "wl_layer_dev: ffn_gate_inp must be %d x %d", (int)L->ffn_gate->experts, E);
    if (shared) {
      const wl_weight *sg = L->ffn_gate_shexp, *su = L->ffn_up_shexp, *sd = L->ffn_down_shexp, *si = L->ffn_gate_inp_shexp;
      if (!su || !sd) return fail(WL_E_ARG, "wl_layer_dev: the shared expert needs gate, up and down");
      if (sg->cols != E || su->cols != E || su->rows != sg->rows || sd->rows != E || sd->cols != sg->rows ||
          (si && (si->cols != E || si->rows != 1)))
        return fail(WL_E_SHAPE, "wl_layer_dev: shared expert tensors have inconsistent shapes");
      if (sg->rows > FF) FF = sg->rows;  // S_LG / S_LU hold either FFN's rows
    }
  }
  const int rd = L->rope_dims > 0 ? L->rope_dims : HD;
  if (rd > HD || rd % 2) return fail(WL_E_SHAPE, "wl_layer_dev: %d rotated of %d per head", rd, HD);
  int rc;
  if ((rc = ensure(c, S_LXN, (size_t)T * E * 4)) || (rc = ensure(c, S_LQ, (size_t)T * QD * 4)) ||
      (rc = ensure(c, S_LK, (size_t)T * KD * 4)) || (rc = ensure(c, S_LV, (size_t)T * KD * 4)) ||
      (rc = ensure(c, S_LATT, (size_t)T * QD * 4)) ||
      (rc = ensure(c, S_LG, (size_t)T * FF * 4)) || (rc = ensure(c, S_LU, (size_t)T * FF * 4)) ||
      (rc = ensure(c, S_ATT, (size_t)wl::attention_scratch_floats(T, H, HD, KD, max_n, d_K, d_V) * 4)))
    return rc;
  float *xn = (float *)c->buf[S_LXN], *q = (float *)c->buf[S_LQ], *k = (float *)c->buf[S_LK],
        *v = (float *)c->buf[S_LV], *att = (float *)c->buf[S_LATT],
        *g = (float *)c->buf[S_LG], *u = (float *)c->buf[S_LU];
  const float rs = L->residual_scale != 0.f ? L->residual_scale : 1.f;
  // y = W x over the T rows: past 8 rows the GEMM, or with each GEMV passes of 8
  auto mm = [&](const wl_weight *w, const float *x, float *y, bool add) -> int {
    const int step = each ? 8 : T;
    for (int t0 = 0; t0 < T; t0 += step) {
      const int n = T - t0 < step ? T - t0 : step;
      const float *xs = x + (int64_t)t0 * w->cols;
      float *ys = y + (int64_t)t0 * w->rows;
      const int r = add ? wl_matmul_add_dev(c, w, -1, xs, n, ys, rs) : matmul_dev(c, w, -1, xs, n, ys);
      if (r) return r;
    }
    return WL_OK;
  };
  // attention block (x itself is the input under post-norms: OLMo 2 has no pre-norm)
  const float *ain = post ? d_x : xn;
  if (!post && (rc = wl_rms_norm_dev(c, d_x, T, E, L->d_attn_norm, L->eps, xn))) return rc;
  if (T <= 8 || each) {
    for (int t0 = 0; t0 < T; t0 += 8) {  // q, k, v in one launch per 8 rows
      const int n = T - t0 < 8 ? T - t0 : 8;
      const wl_weight *ws[3] = {L->attn_q, L->attn_k, L->attn_v};
      float *ys[3] = {q + (int64_t)t0 * QD, k + (int64_t)t0 * KD, v + (int64_t)t0 * KD};
      if ((rc = wl_matmul_multi_dev(c, 3, ws, ain + (int64_t)t0 * E, n, ys))) return rc;
    }
  } else if ((rc = mm(L->attn_q, ain, q, false)) || (rc = mm(L->attn_k, ain, k, false)) ||
             (rc = mm(L->attn_v, ain, v, false))) {
    return rc;
  }
  if (L->d_q_bias) WL_HIP(wl::bias_launch(q, L->d_q_bias, T, QD, c->stream), "q bias");
  if (L->d_k_bias) WL_HIP(wl::bias_launch(k, L->d_k_bias, T, KD, c->stream), "k bias");
  if (L->d_v_bias) WL_HIP(wl::bias_launch(v, L->d_v_bias, T, KD, c->stream), "v bias");
  // q/k norms per head (qwen3) or over the whole rows (QkNormFull, OLMo 2: src/Transformer.cs:192-201)
  const bool full = L->qk_norm_full != 0;
  if (L->d_q_norm && (rc = wl_rms_norm_dev(c, q, full ? T : (int64_t)T * H, full ? QD : HD, L->d_q_norm, L->eps, q)))
    return rc;
  if (L->d_k_norm && (rc = wl_rms_norm_dev(c, k, full ? T : (int64_t)T * KH, full ? KD : HD, L->d_k_norm, L->eps, k)))
    return rc;
  // RoPE, the fp16 KV store and attention (one launch for a token or batch rows on their own slots,
  // with the positions' angles from the context's table)
  const double fs = L->rope_freq_scale != 0.0 ? L->rope_freq_scale : 1.0;
  const float scale = L->attention_scale != 0.f ? L->attention_scale : 1.0f / (float)sqrt((double)HD);
  const float4 *tab = nullptr;
  if (wl::rope_attention_fused(T, rm, HD, KH, rd, d_K, d_V) &&
      (rc = rope_angles(c, hpos, T, pos0, rd, L->rope_base, fs, L->d_rope_freqs, &tab)))
    return rc;
  WL_HIP(wl::rope_attention_launch(q, k, v, T, H, KH, HD, rd, L->neox, pos0, L->rope_base, fs, L->d_rope_freqs, tab,
                                   d_K, d_V, rm, scale, (float *)c->buf[S_ATT], att, max_n, c->stream),
         "rope, kv store and attention");
  if (post) {
    // o = RmsNorm(W_o att), then x += o * rs (src/Transformer.cs:223-225)
    if ((rc = ensure(c, S_LM, (size_t)T * E * 4))) return rc;
    float *o = (float *)c->buf[S_LM];
    if ((rc = mm(L->attn_output, att, o, false)) ||
        (rc = wl_rms_norm_dev(c, o, T, E, L->d_post_attention_norm, L->eps, o)))
      return rc;
    WL_HIP(wl::residual_launch(d_x, o, (int64_t)T * E, rs, c->stream), "residual");
  } else if ((rc = mm(L->attn_output, att, d_x, true))) {
    return rc;
  }
  // feed-forward block
  const float *fin = post ? d_x : xn;
  if (!post && (rc = wl_rms_norm_dev(c, d_x, T, E, L->d_ffn_norm, L->eps, xn))) return rc;
  // SwiGlu (src/Transformer.cs:241-251) into y (added into y with add): up to 8 rows (or every
  // row with each) gate and up in one GEMV launch with the SiLU epilogue; a prompt: the two
  // GEMMs, then the SiLU pass
  auto swiglu = [&](const wl_weight *wg, const wl_weight *wu, const wl_weight *wd, float *y, bool add) -> int {
    const bool fused = wg->type == wu->type && (T <= 8 || each || int_path(c, wg) || !wl::gemm_supports(wg->type));
    int r;
    if (fused) {
      if ((r = wl_gate_up_dev(c, wg, wu, -1, fin, T, g))) return r;
    } else {
      if ((r = mm(wg, fin, g, false)) || (r = mm(wu, fin, u, false))) return r;
      WL_HIP(wl::silu_mul_launch(g, u, (int64_t)T * wg->rows, c->stream), "silu");
    }
    return mm(wd, g, y, add);
  };
  if (!moe && !post) return swiglu(L->ffn_gate, L->ffn_up, L->ffn_down, d_x, true);
  if (!moe) {
    // the FFN's output RMS-normed before the residual add (src/Transformer.cs:229-231)
    if ((rc = ensure(c, S_LM, (size_t)T * E * 4))) return rc;
    float *o = (float *)c->buf[S_LM];
    if ((rc = swiglu(L->ffn_gate, L->ffn_up, L->ffn_down, o, false)) ||
        (rc = wl_rms_norm_dev(c, o, T, E, L->d_post_ffw_norm, L->eps, o)))
      return rc;
    WL_HIP(wl::residual_launch(d_x, o, (int64_t)T * E, rs, c->stream), "residual");
    return WL_OK;
  }
  // MoeFfn (src/Transformer.cs:259-311): router logits, routed experts, the shared expert, then
  // the residual add (:231)
  const int ne = (int)L->ffn_gate->experts;
  if ((rc = ensure(c, S_LR, (size_t)T * (ne > 1 ? ne : 1) * 4)) || (rc = ensure(c, S_LM, (size_t)T * E * 4)) ||
      (shared && (rc = ensure(c, S_LS, (size_t)T * E * 4))))
    return rc;
  float *lg = (float *)c->buf[S_LR], *o = (float *)c->buf[S_LM], *sh = (float *)c->buf[S_LS];
  if ((rc = mm(L->ffn_gate_inp, fin, lg, false))) return rc;
  if ((rc = moe_dev(c, lg, L->expert_used, L->expert_weights_norm, L->ffn_gate, L->ffn_up, L->ffn_down, fin, T, o)))
    return rc;
  if (shared) {
    if ((rc = swiglu(L->ffn_gate_shexp, L->ffn_up_shexp, L->ffn_down_shexp, sh, false))) return rc;
    // the router's logits are used: its buffer takes the shared expert's gate
    if (L->ffn_gate_inp_shexp && (rc = mm(L->ffn_gate_inp_shexp, fin, lg, false))) return rc;
    WL_HIP(wl::shared_expert_launch(o, sh, L->ffn_gate_inp_shexp ? lg : nullptr, T, E, c->stream), "shared expert");
  }
  if (post && (rc = wl_rms_norm_dev(c, o, T, E, L->d_post_ffw_norm, L->eps, o))) return rc;
  WL_HIP(wl::residual_launch(d_x, o, (int64_t)T * E, rs, c->stream), "residual");
  return WL_OK;
}

extern "C" int wl_layer_dev(wl_ctx *c, const wl_layer_desc *L, float *d_x, int32_t T, int32_t pos0, uint16_t *d_K,
                            uint16_t *d_V) {
  return layer_run(c, L, d_x, T, pos0, d_K, d_V, wl::RowMap{}, nullptr, pos0 + T, false);
}

// Transformer.ForwardBatch's layer (src/Transformer.cs:127-170): N rows, each the next token of
// its own sequence, at position pos[i] of cache slot slot[i].
extern "C" int wl_layer_batch_dev(wl_ctx *c, const wl_layer_desc *L, float *d_x, int32_t N, const int32_t *pos,
                                  const int32_t *slot, int32_t slots, int32_t slot_positions, uint16_t *d_K,
                                  uint16_t *d_V) {
  if (!c || !pos || !slot) return fail(WL_E_ARG, "wl_layer_batch_dev: null argument");
  if (N <= 0 || slots <= 0 || slot_positions <= 0) return fail(WL_E_SHAPE, "wl_layer_batch_dev: bad shape");
  int max_n = 0;
  for (int i = 0; i < N; i++) {
    if (slot[i] < 0 || slot[i] >= slots)
      return fail(WL_E_ARG, "Row %d's slot %d is outside 0..%d.", i, slot[i], slots - 1);
    if (pos[i] < 0 || pos[i] >= slot_positions)
      return fail(WL_E_ARG, "The prompt and reply need %d positions; the context is %d.", pos[i] + 1, slot_positions);
    for (int j = 0; j < i; j++)
      if (slot[j] == slot[i]) return fail(WL_E_ARG, "A sequence can take one token per batch step.");
    if (pos[i] + 1 > max_n) max_n = pos[i] + 1;
  }
  int rc;
  int32_t *rows;
  if ((rc = stage_rows(c, pos, slot, N, &rows))) return rc;
  wl::RowMap rm;
  rm.pos = rows;
  rm.slot = rows + N;
  rm.cap = slot_positions;
  return layer_run(c, L, d_x, N, 0, d_K, d_V, rm, pos, max_n, true);
}

extern "C" int wl_read_peak_dev(wl_ctx *c, const void *d_src, int64_t bytes, int32_t workgroups, uint32_t *d_out) {
  if (!c || !d_src || !d_out) return fail(WL_E_ARG, "wl_read_peak_dev: null argument");
  if (bytes < 16 || bytes % 16) return fail(WL_E_SHAPE, "wl_read_peak_dev: %lld bytes are not whole 16-byte words",
                                            (long long)bytes);
  const int wgs = workgroups > 0 ? workgroups : 8 * c->num_cu;
  WL_HIP(hipSetDevice(c->device), "hipSetDevice");
  WL_HIP(wl::read_peak_launch(d_src, bytes, wgs, d_out, c->stream), "read_peak_kernel");
  return WL_OK;
}

// ------------------------------------------------------------------------------ graphs
// A run of _dev calls captured once from the context's stream and replayed as one graph launch:
// the host enqueues one command instead of one per kernel.
struct wl_graph {
  hipGraphExec_t exec;
};

extern "C" int wl_capture_begin(wl_ctx *c) {
  if (!c) return fail(WL_E_ARG, "wl_capture_begin: null context");
  if (c->capturing) return fail(WL_E_ARG, "wl_capture_begin: the context is already capturing");
  WL_HIP(hipSetDevice(c->device), "hipSetDevice");
  WL_HIP(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
  c->capturing = true;
  return WL_OK;
}

extern "C" int wl_capture_end(wl_ctx *c, wl_graph **out) {
  if (!c || !out) return fail(WL_E_ARG, "wl_capture_end: null argument");
  *out = nullptr;
  if (!c->capturing) return fail(WL_E_ARG, "wl_capture_end: the context is not capturing");
  c->capturing = false;
  hipGraph_t g = nullptr;
  WL_HIP(hipStreamEndCapture(c->stream, &g), "hipStreamEndCapture (a call during the capture failed or synchronised)");
  hipGraphExec_t exec = nullptr;
  const hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  hipGraphDestroy(g);
  if (e != hipSuccess) return fail(WL_E_DEVICE, "hipGraphInstantiate: %s", hipGetErrorString(e));
  *out = new wl_graph{exec};
  return WL_OK;
}

extern "C" int wl_graph_launch(wl_ctx *c, const wl_graph *g) {
  if (!c || !g) return fail(WL_E_ARG, "wl_graph_launch: null argument");
  if (c->capturing) return fail(WL_E_ARG, "wl_graph_launch: the context is capturing");
  WL_HIP(hipGraphLaunch(g->exec, c->stream), "hipGraphLaunch");
  return WL_OK;
}

extern "C" int wl_graph_free(wl_graph *g) {
  if (!g) return WL_OK;
  const hipError_t e = hipGraphExecDestroy(g->exec);
  delete g;
  return e == hipSuccess ? WL_OK : fail(WL_E_DEVICE, "hipGraphExecDestroy: %s", hipGetErrorString(e));
}
