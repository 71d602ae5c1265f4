// nx_api.hip — the extern "C" boundary of libnexus_hip.so (include/nexus_hip.h).
//
// Validation mirrors the reference where the reference validates
// (src/engine/mod.rs:975-991, src/gguf/mod.rs:962-1030); every device launch
// is preceded by host-side checks that the shapes match what the kernels and
// their grids assume.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "nx_device.hpp"
#include "nx_internal.hpp"

// one token on the GEMV path: the gate/up kernel routes it itself
#ifndef NX_ROUTE_IN_GEMV_MAX_E
#define NX_ROUTE_IN_GEMV_MAX_E kFusedRouteMaxE
#endif
#ifndef NX_ROUTE_IN_GEMV
#define NX_ROUTE_IN_GEMV 1
#endif

namespace nx {

static thread_local std::string g_err;

int fail(int code, const std::string &msg) {
  g_err = msg;
  return code;
}
void clear_error() { g_err.clear(); }

bool format_info(int fmt, FormatInfo *fi) {
  switch (fmt) {
  case NX_FMT_Q4_K: *fi = {fmt, 256, 144, 128, 16}; return true;
  case NX_FMT_Q8_0: *fi = {fmt, 32, 34, 32, 2}; return true;
  case NX_FMT_Q4_0: *fi = {fmt, 32, 18, 16, 2}; return true;
  // resident Q2_K: 2-bit codes (16 bytes per 64-element segment), 8
  // scale-plane bytes per segment
  case NX_FMT_Q2_K: *fi = {fmt, 256, 84, 64, 32}; return true;
  case NX_FMT_F32: *fi = {fmt, 4, 16, 16, 0}; return true;
  // 16-bit floats: 16 values per 32-byte segment, no scale plane
  case NX_FMT_F16:
  case NX_FMT_BF16: *fi = {fmt, 1, 2, 2, 0}; return true;
  }
  return false;
}

static const char *fmt_name(int fmt) {
  switch (fmt) {
  case NX_FMT_Q4_K: return "Q4_K";
  case NX_FMT_Q8_0: return "Q8_0";
  case NX_FMT_Q4_0: return "Q4_0";
  case NX_FMT_Q2_K: return "Q2_K";
  case NX_FMT_F32: return "F32";
  case NX_FMT_F16: return "F16";
  case NX_FMT_BF16: return "BF16";
  }
  return "?";
}

static size_t gguf_bytes(int fmt, size_t n) {
  switch (fmt) {
  case NX_FMT_Q4_K: return (n + 255) / 256 * 144;
  case NX_FMT_Q8_0: return (n + 31) / 32 * 34;
  case NX_FMT_Q4_0: return (n + 31) / 32 * 18;
  case NX_FMT_Q2_K: return (n + 255) / 256 * 84;
  case NX_FMT_F32: return n * 4;
  case NX_FMT_F16:
  case NX_FMT_BF16: return n * 2;
  }
  return 0;
}

// Scratch of nx_moe_forward_noalloc: one static array per device, resident
// until the process ends.  Host code never passes `scratch` itself to a
// kernel (in host code the name is a host-side stand-in, not a device
// address); it uses the address hipGetSymbolAddress returns for the device.
constexpr size_t kScratchBytes = size_t(64) << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

static std::mutex g_scratch_mu;
static std::vector<uint8_t *> g_scratch_ptr;  // per device; null until looked up

// The scratch array's address on `device` (which must be current), looked up
// once per device.
static int scratch_address(int device, uint8_t **out) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if ((int)g_scratch_ptr.size() <= device) g_scratch_ptr.resize(device + 1, nullptr);
  if (!g_scratch_ptr[device]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      (void)hipGetLastError();
      return fail(NX_ERR_DEVICE, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    }
    g_scratch_ptr[device] = static_cast<uint8_t *>(p);
  }
  *out = g_scratch_ptr[device];
  return NX_OK;
}

int ws_get(nx_ctx *c, int slot, size_t bytes, void **out) {
  if (bytes == 0) bytes = 256;
  // any other use of the route slots ends what nx_moe_last_routes can read
  if (slot == WS_ROUTE_EXPERT || slot == WS_ROUTE_WEIGHT || slot == WS_ROUTE_COUNT)
    c->last_exp = nullptr;
  if (c->scratch_mode) {
    DevBuf &s = c->scratch_slot[slot];
    if (s.ptr && s.cap >= bytes) {
      *out = s.ptr;
      return NX_OK;
    }
    const size_t cap = (bytes + 255) / 256 * 256;
    if (cap > kScratchBytes - c->scratch_used)
      return fail(NX_ERR_UNSUPPORTED,
                  "nx_moe_forward_noalloc: this call needs more than the " +
                      std::to_string(kScratchBytes) + "-byte scratch array (" +
                      std::to_string(c->scratch_used + cap) + " bytes so far)");
    s.ptr = c->scratch + c->scratch_used;
    s.cap = cap;
    c->scratch_used += cap;
    *out = s.ptr;
    return NX_OK;
  }
  DevBuf &b = c->ws[slot];
  if (b.cap < bytes) {
    if (b.ptr) {
      NX_HIP(hipStreamSynchronize(c->stream));
      NX_HIP(hipFree(b.ptr));
      b.ptr = nullptr;
      b.cap = 0;
    }
    size_t cap = bytes + bytes / 4;
    cap = (cap + 255) / 256 * 256;
    if (hipMalloc(&b.ptr, cap) != hipSuccess) {
      (void)hipGetLastError();
      b.ptr = nullptr;
      return fail(NX_ERR_OOM, "device allocation of " + std::to_string(cap) + " bytes failed");
    }
    b.cap = cap;
  }
  *out = b.ptr;
  return NX_OK;
}

template <typename T>
static int ws(nx_ctx *c, int slot, size_t count, T **out) {
  void *p = nullptr;
  NX_TRY(ws_get(c, slot, count * sizeof(T), &p));
  *out = static_cast<T *>(p);
  return NX_OK;
}

static int get_event(nx_ctx *c, hipEvent_t *e) {
  if (!c->event_pool.empty()) {
    *e = c->event_pool.back();
    c->event_pool.pop_back();
    return NX_OK;
  }
  NX_HIP(hipEventCreate(e));
  return NX_OK;
}

int begin_launch(nx_ctx *c, const char *name, int *stat_index) {
  *stat_index = -1;
  if (!c->profile) return NX_OK;
  int si = -1;
  for (size_t i = 0; i < c->stats.size(); ++i)
    if (c->stats[i].name == name) si = (int)i;
  if (si < 0) {
    c->stats.push_back(KernelStat{name, 0, 0.0});
    si = (int)c->stats.size() - 1;
  }
  PendingEvent pe{si, nullptr, nullptr};
  NX_TRY(get_event(c, &pe.start));
  NX_TRY(get_event(c, &pe.stop));
  NX_HIP(hipEventRecord(pe.start, c->stream));
  c->pending.push_back(pe);
  *stat_index = (int)c->pending.size() - 1;
  // a kernel started with go() binds both events to its own dispatch (the
  // start recorded here is then superseded); other work is bracketed by
  // the records on the stream
  c->launch_start = pe.start;
  c->launch_stop = pe.stop;
  c->launch_timed = false;
  return NX_OK;
}

int end_launch(nx_ctx *c, int pending_index) {
  if (pending_index < 0) return NX_OK;
  c->launch_start = c->launch_stop = nullptr;
  if (!c->launch_timed) NX_HIP(hipEventRecord(c->pending[pending_index].stop, c->stream));
  return NX_OK;
}

static int collect_profile(nx_ctx *c) {
  if (c->pending.empty()) return NX_OK;
  NX_HIP(hipStreamSynchronize(c->stream));
  for (auto &pe : c->pending) {
    float ms = 0.f;
    NX_HIP(hipEventElapsedTime(&ms, pe.start, pe.stop));
    c->stats[pe.stat].launches += 1;
    c->stats[pe.stat].total_ms += ms;
    c->event_pool.push_back(pe.start);
    c->event_pool.push_back(pe.stop);
  }
  c->pending.clear();
  return NX_OK;
}

static int set_device(nx_ctx *c) {
  NX_HIP(hipSetDevice(c->device));
  return NX_OK;
}

// one dense device allocation, recorded for release with the expert set
static int ex_alloc(nx_experts *ex, size_t bytes, uint8_t **out) {
  void *p = nullptr;
  if (bytes == 0) bytes = 256;
  if (hipMalloc(&p, bytes) != hipSuccess) {
    (void)hipGetLastError();
    return fail(NX_ERR_OOM, "device allocation of " + std::to_string(bytes) + " bytes failed");
  }
  // padding between rows and past the last row is read (times zero
  // activations) by the grouped GEMM's wide scale loads: keep it finite
  if (hipMemsetAsync(p, 0, bytes, ex->ctx->stream) != hipSuccess) {
    (void)hipGetLastError();
    (void)hipFree(p);
    return fail(NX_ERR_DEVICE, "clearing a device allocation failed");
  }
  ex->allocs.push_back(p);
  ex->device_bytes += bytes;
  *out = static_cast<uint8_t *>(p);
  return NX_OK;
}

// row layout of a plane of `rows` x `cols` in format fmt (no allocation)
static void plane_layout(int fmt, RolePlane &pl, int rows, int cols) {
  pl.rows = rows;
  pl.cols = cols;
  switch (fmt) {
  case NX_FMT_Q4_K:
    pl.nseg = cols / 256 * 4;
    pl.row_meta = (uint32_t)(cols / 256 * 16);
    break;
  case NX_FMT_Q8_0:
    pl.nseg = cols / 32;
    // whole dwords per row: the grouped GEMM loads two blocks' scales at once
    pl.row_meta = (uint32_t)((cols / 32 * 2 + 3) / 4 * 4);
    break;
  case NX_FMT_Q4_0:
    pl.nseg = (cols / 32 + 1) / 2;
    pl.row_meta = (uint32_t)(pl.nseg * 4);
    break;
  case NX_FMT_Q2_K:
    pl.nseg = cols / 256 * 4;
    pl.row_meta = (uint32_t)(pl.nseg * 8);
    break;
  case NX_FMT_F16:
  case NX_FMT_BF16:
    pl.nseg = (cols + 15) / 16;
    pl.row_meta = 0;
    break;
  default:  // F32
    pl.nseg = (cols + 7) / 8;
    pl.row_meta = 0;
    break;
  }
  // two 16-byte code chunks per segment, one for Q2_K's 2-bit codes; rows of
  // more than 64 segments are stored in panels of 64 (nx_device.hpp), the
  // last one zero-padded, so their bytes per row count whole panels
  const int np = panel_count(pl.nseg);
  pl.row_qs = (uint32_t)np * panel_row_bytes(pl.nseg, fmt == NX_FMT_Q2_K ? 16 : 32);
  if (pl.row_meta) {
    // scale bytes per segment: Q4_K 16 per block of 4, Q8_0 2, Q4_0 4, Q2_K 8
    const int mu = fmt == NX_FMT_Q8_0 ? 2 : (fmt == NX_FMT_Q2_K ? 8 : 4);
    pl.row_meta = (uint32_t)np * panel_row_bytes(pl.nseg, mu);
  }
  // strides rounded to 256 B so every expert's planes start aligned
  pl.qs_stride = ((size_t)rows * pl.row_qs + 255) / 256 * 256;
  pl.meta_stride = ((size_t)rows * pl.row_meta + 255) / 256 * 256;
}

static int init_plane(nx_experts *ex, RolePlane &pl, int count, int rows, int cols) {
  plane_layout(ex->fmt, pl, rows, cols);
  NX_TRY(ex_alloc(ex, pl.qs_stride * count, &pl.qs));
  if (pl.row_meta) NX_TRY(ex_alloc(ex, pl.meta_stride * count, &pl.meta));
  return NX_OK;
}

static int check_ctx(nx_ctx *c) {
  if (!c) return fail(NX_ERR_INVALID_ARG, "null context");
  return set_device(c);
}

}  // namespace nx

using namespace nx;

extern "C" {

const char *nx_last_error(void) { return g_err.c_str(); }

int nx_version(void) { return 1; }

int nx_device_count(int *count) {
  if (!count) return fail(NX_ERR_INVALID_ARG, "null count");
  *count = 0;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return NX_OK;
  }
  int good = 0;
  for (int d = 0; d < n; ++d) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, d) == hipSuccess && std::strstr(prop.gcnArchName, "gfx950"))
      ++good;
  }
  *count = good;
  return NX_OK;
}

int nx_ctx_create(int device, nx_ctx **out) {
  if (!out) return fail(NX_ERR_INVALID_ARG, "null output pointer");
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
    (void)hipGetLastError();
    return fail(NX_ERR_DEVICE, "no HIP device available");
  }
  if (device < 0 || device >= n) return fail(NX_ERR_INVALID_ARG, "device index out of range");
  hipDeviceProp_t prop;
  NX_HIP(hipGetDeviceProperties(&prop, device));
  if (!std::strstr(prop.gcnArchName, "gfx950"))
    return fail(NX_ERR_DEVICE, std::string("device is ") + prop.gcnArchName + ", this library is built for gfx950");
  NX_HIP(hipSetDevice(device));
  nx_ctx *c = new nx_ctx();
  c->device = device;
  c->num_cu = prop.multiProcessorCount;
  c->lds_per_cu = prop.maxSharedMemoryPerMultiProcessor;
  if (hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking) != hipSuccess) {
    delete c;
    return fail(NX_ERR_DEVICE, "hipStreamCreateWithFlags failed");
  }
  c->stream = c->own_stream;
  // the no-allocation entry point's scratch array on this device
  if (int rc = scratch_address(device, &c->scratch)) {
    (void)hipStreamDestroy(c->own_stream);
    delete c;
    return rc;
  }
  *out = c;
  return NX_OK;
}

int nx_ctx_destroy(nx_ctx *c) {
  if (!c) return NX_OK;
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  for (auto &b : c->ws)
    if (b.ptr) (void)hipFree(b.ptr);
  if (c->host_stage.ptr) (void)hipHostFree(c->host_stage.ptr);
  for (auto &pe : c->pending) {
    (void)hipEventDestroy(pe.start);
    (void)hipEventDestroy(pe.stop);
  }
  for (auto e : c->event_pool) (void)hipEventDestroy(e);
  if (c->own_stream) (void)hipStreamDestroy(c->own_stream);
  delete c;
  return NX_OK;
}

int nx_ctx_set_stream(nx_ctx *c, void *s) {
  NX_TRY(check_ctx(c));
  c->stream = s ? static_cast<hipStream_t>(s) : c->own_stream;
  return NX_OK;
}

int nx_ctx_get_stream(nx_ctx *c, void **s) {
  NX_TRY(check_ctx(c));
  if (!s) return fail(NX_ERR_INVALID_ARG, "null output pointer");
  *s = c->stream;
  return NX_OK;
}

int nx_sync(nx_ctx *c) {
  NX_TRY(check_ctx(c));
  NX_HIP(hipStreamSynchronize(c->stream));
  return NX_OK;
}

int nx_mem_info(nx_ctx *c, size_t *free_b, size_t *total_b) {
  NX_TRY(check_ctx(c));
  size_t f = 0, t = 0;
  NX_HIP(hipMemGetInfo(&f, &t));
  if (free_b) *free_b = f;
  if (total_b) *total_b = t;
  return NX_OK;
}

int nx_profile_enable(nx_ctx *c, int enable) {
  NX_TRY(check_ctx(c));
  c->profile = enable != 0;
  return NX_OK;
}

int nx_profile_reset(nx_ctx *c) {
  NX_TRY(check_ctx(c));
  NX_TRY(collect_profile(c));
  c->stats.clear();
  return NX_OK;
}

int nx_profile_count(nx_ctx *c, int *n) {
  NX_TRY(check_ctx(c));
  NX_TRY(collect_profile(c));
  if (n) *n = (int)c->stats.size();
  return NX_OK;
}

int nx_profile_get(nx_ctx *c, int index, char *name, size_t cap, int *launches, double *total_ms) {
  NX_TRY(check_ctx(c));
  NX_TRY(collect_profile(c));
  if (index < 0 || index >= (int)c->stats.size()) return fail(NX_ERR_INVALID_ARG, "profile index out of range");
  const KernelStat &s = c->stats[index];
  if (name && cap) {
    std::strncpy(name, s.name.c_str(), cap - 1);
    name[cap - 1] = 0;
  }
  if (launches) *launches = s.launches;
  if (total_ms) *total_ms = s.total_ms;
  return NX_OK;
}

// ------------------------------------------------------------------- quant
int nx_quant_bytes(int fmt, size_t n, size_t *bytes) {
  FormatInfo fi;
  if (!format_info(fmt, &fi)) return fail(NX_ERR_INVALID_ARG, "unknown weight format " + std::to_string(fmt));
  if (!bytes) return fail(NX_ERR_INVALID_ARG, "null output pointer");
  *bytes = gguf_bytes(fmt, n);
  return NX_OK;
}

int nx_dequant_dev(nx_ctx *c, int fmt, const void *src, size_t src_bytes, size_t n, float *dst) {
  NX_TRY(check_ctx(c));
  FormatInfo fi;
  if (!format_info(fmt, &fi)) return fail(NX_ERR_INVALID_ARG, "unknown weight format " + std::to_string(fmt));
  if (n == 0) return NX_OK;
  if (!src || !dst) return fail(NX_ERR_INVALID_ARG, "null buffer");
  if (src_bytes < gguf_bytes(fmt, n))  // src/gguf/mod.rs:966-971 and siblings
    return fail(NX_ERR_TRUNCATED, std::string(fmt_name(fmt)) + " tensor payload is truncated");
  return launch_dequant(c, fmt, src, n, dst);
}

int nx_dequant(nx_ctx *c, int fmt, const void *src, size_t src_bytes, size_t n, float *dst) {
  NX_TRY(check_ctx(c));
  FormatInfo fi;
  if (!format_info(fmt, &fi)) return fail(NX_ERR_INVALID_ARG, "unknown weight format " + std::to_string(fmt));
  if (n == 0) return NX_OK;
  if (!src || !dst) return fail(NX_ERR_INVALID_ARG, "null buffer");
  const size_t need = gguf_bytes(fmt, n);
  if (src_bytes < need) return fail(NX_ERR_TRUNCATED, std::string(fmt_name(fmt)) + " tensor payload is truncated");
  uint8_t *d_src = nullptr;
  float *d_dst = nullptr;
  NX_TRY(ws(c, WS_XIN, need, &d_src));
  NX_TRY(ws(c, WS_OUT, n, &d_dst));
  NX_HIP(hipMemcpyAsync(d_src, src, need, hipMemcpyHostToDevice, c->stream));
  NX_TRY(launch_dequant(c, fmt, d_src, n, d_dst));
  NX_HIP(hipMemcpyAsync(dst, d_dst, n * sizeof(float), hipMemcpyDeviceToHost, c->stream));
  NX_HIP(hipStreamSynchronize(c->stream));
  return NX_OK;
}

int nx_quantize_dev(nx_ctx *c, int fmt, const float *src, size_t n, void *dst, size_t dst_bytes) {
  NX_TRY(check_ctx(c));
  FormatInfo fi;
  if (!format_info(fmt, &fi)) return fail(NX_ERR_INVALID_ARG, "unknown weight format " + std::to_string(fmt));
  if (n == 0) return NX_OK;
  if (!src || !dst) return fail(NX_ERR_INVALID_ARG, "null buffer");
  if (dst_bytes < gguf_bytes(fmt, n)) return fail(NX_ERR_SHAPE, "destination smaller than the quantized payload");
  return launch_quantize(c, fmt, src, n, dst);
}

int nx_quantize(nx_ctx *c, int fmt, const float *src, size_t n, void *dst, size_t dst_bytes) {
  NX_TRY(check_ctx(c));
  FormatInfo fi;
  if (!format_info(fmt, &fi)) return fail(NX_ERR_INVALID_ARG, "unknown weight format " + std::to_string(fmt));
  if (n == 0) return NX_OK;
  if (!src || !dst) return fail(NX_ERR_INVALID_ARG, "null buffer");
  const size_t need = gguf_bytes(fmt, n);
  if (dst_bytes < need) return fail(NX_ERR_SHAPE, "destination smaller than the quantized payload");
  float *d_src = nullptr;
  uint8_t *d_dst = nullptr;
  NX_TRY(ws(c, WS_XIN, n, &d_src));
  NX_TRY(ws(c, WS_OUT, need, &d_dst));
  NX_HIP(hipMemcpyAsync(d_src, src, n * sizeof(float), hipMemcpyHostToDevice, c->stream));
  NX_TRY(launch_quantize(c, fmt, d_src, n, d_dst));
  NX_HIP(hipMemcpyAsync(dst, d_dst, need, hipMemcpyDeviceToHost, c->stream));
  NX_HIP(hipStreamSynchronize(c->stream));
  return NX_OK;
}

// ------------------------------------------------------------------- routing
int nx_route_topk(nx_ctx *c, const float *logits, size_t logits_len, int T, int E, int k,
                  int score_mode, int32_t *experts, float *weights, int32_t *counts, int *lists) {
  NX_TRY(check_ctx(c));
  if (T < 0 || E < 0 || k < 0) return fail(NX_ERR_INVALID_ARG, "negative size");
  if (score_mode != NX_SCORE_SOFTMAX && score_mode != NX_SCORE_SIGMOID)
    return fail(NX_ERR_INVALID_ARG, "unknown score mode");
  if (T > 0 && k > 0 && (!experts || !weights || !counts))
    return fail(NX_ERR_INVALID_ARG, "null output buffer");
  for (size_t i = 0; i < (size_t)T * k; ++i) {
    experts[i] = -1;
    weights[i] = 0.0f;
  }
  for (int t = 0; t < T && counts; ++t) counts[t] = 0;
  int n = 0;
  if (T > 0 && E > 0 && k > 0) {  // src/engine/mod.rs:924-934
    if (!logits) return fail(NX_ERR_INVALID_ARG, "null logits");
    n = (int)std::min<size_t>((size_t)T, logits_len / (size_t)E);
  }
  if (lists) *lists = n;
  if (n == 0) return NX_OK;
  float *d_logits;
  int32_t *d_exp, *d_cnt;
  float *d_w;
  NX_TRY(ws(c, WS_LOGITS, (size_t)n * E, &d_logits));
  NX_TRY(ws(c, WS_ROUTE_EXPERT, (size_t)n * k, &d_exp));
  NX_TRY(ws(c, WS_ROUTE_WEIGHT, (size_t)n * k, &d_w));
  NX_TRY(ws(c, WS_ROUTE_COUNT, (size_t)n, &d_cnt));
  NX_HIP(hipMemcpyAsync(d_logits, logits, (size_t)n * E * 4, hipMemcpyHostToDevice, c->stream));
  NX_TRY(launch_route(c, d_logits, n, E, k, score_mode, d_exp, d_w, d_cnt));
  NX_HIP(hipMemcpyAsync(experts, d_exp, (size_t)n * k * 4, hipMemcpyDeviceToHost, c->stream));
  NX_HIP(hipMemcpyAsync(weights, d_w, (size_t)n * k * 4, hipMemcpyDeviceToHost, c->stream));
  NX_HIP(hipMemcpyAsync(counts, d_cnt, (size_t)n * 4, hipMemcpyDeviceToHost, c->stream));
  NX_HIP(hipStreamSynchronize(c->stream));
  return NX_OK;
}

// Shape checks of InferenceEngine::matvec (src/engine/mod.rs:776-789), with
// the input of T tokens taken as one [T x H] array.
static int check_logits(const float *w, size_t w_len, const float *x, size_t x_len, int T, int E,
                        int H, const float *out) {
  if (T < 0 || E < 0 || H < 0) return fail(NX_ERR_INVALID_ARG, "negative size");
  const size_t need_x = (size_t)T * H, need_w = (size_t)E * H;
  if (x_len != need_x)
    return fail(NX_ERR_SHAPE, "Matvec input shape mismatch: got " + std::to_string(x_len) +
                                  ", expected " + std::to_string(need_x));
  if (w_len < need_w)
    return fail(NX_ERR_SHAPE, "Matvec weight too small: got " + std::to_string(w_len) +
                                  ", expected at least " + std::to_string(need_w));
  // device offsets are 32-bit
  if (need_w * 4 > 0x7FFFFF00u || need_x * 4 > 0x7FFFFF00u || (size_t)T * E > 0x7FFFFFFFu)
    return fail(NX_ERR_UNSUPPORTED, "router weight, input or logits over 2 GiB");
  if (T > 0 && E > 0 && (!out || (H > 0 && (!w || !x))))
    return fail(NX_ERR_INVALID_ARG, "null buffer");
  return NX_OK;
}

int nx_router_logits_dev(nx_ctx *c, const float *w, size_t w_len, const float *x, size_t x_len,
                         int T, int E, int H, int exact, float *logits) {
  NX_TRY(check_ctx(c));
  NX_TRY(check_logits(w, w_len, x, x_len, T, E, H, logits));
  return launch_router_logits(c, w, x, T, E, H, exact != 0, logits);
}

int nx_router_logits(nx_ctx *c, const float *w, size_t w_len, const float *x, size_t x_len,
                     int T, int E, int H, int exact, float *logits) {
  NX_TRY(check_ctx(c));
  NX_TRY(check_logits(w, w_len, x, x_len, T, E, H, logits));
  if (T == 0 || E == 0) return NX_OK;
  const size_t nw = (size_t)E * H, nx_ = (size_t)T * H, no = (size_t)T * E;
  float *d_w, *d_x, *d_o;
  NX_TRY(ws(c, WS_ROUTER_W, std::max<size_t>(nw, 1), &d_w));
  NX_TRY(ws(c, WS_XIN, std::max<size_t>(nx_, 1), &d_x));
  NX_TRY(ws(c, WS_LOGITS, no, &d_o));
  if (nw) NX_HIP(hipMemcpyAsync(d_w, w, nw * 4, hipMemcpyHostToDevice, c->stream));
  if (nx_) NX_HIP(hipMemcpyAsync(d_x, x, nx_ * 4, hipMemcpyHostToDevice, c->stream));
  NX_TRY(launch_router_logits(c, d_w, d_x, T, E, H, exact != 0, d_o));
  NX_HIP(hipMemcpyAsync(logits, d_o, no * 4, hipMemcpyDeviceToHost, c->stream));
  NX_HIP(hipStreamSynchronize(c->stream));
  return NX_OK;
}

// kernel::rms_norm takes weight[i] for i < dim (a shorter weight panics there)
static int check_norm(const float *x, size_t x_len, const float *w, size_t w_len, int T, int H,
                      const float *out) {
  if (T < 0 || H < 0) return fail(NX_ERR_INVALID_ARG, "negative size");
  const size_t need_x = (size_t)T * H;
  if (x_len != need_x)
    return fail(NX_ERR_SHAPE, "RMSNorm input shape mismatch: got " + std::to_string(x_len) +
                                  ", expected " + std::to_string(need_x));
  if (w_len < (size_t)H)
    return fail(NX_ERR_SHAPE, "RMSNorm weight too small: got " + std::to_string(w_len) +
                                  ", expected at least " + std::to_string(H));
  if (need_x * 4 > 0x7FFFFF00u) return fail(NX_ERR_UNSUPPORTED, "RMSNorm input over 2 GiB");
  if (need_x > 0 && (!x || !w || !out)) return fail(NX_ERR_INVALID_ARG, "null buffer");
  return NX_OK;
}

int nx_rms_norm_dev(nx_ctx *c, const float *x, size_t x_len, const float *w, size_t w_len,
                    float eps, int T, int H, int exact, float *out) {
  NX_TRY(check_ctx(c));
  NX_TRY(check_norm(x, x_len, w, w_len, T, H, out));
  if (T == 0 || H == 0) return NX_OK;
  if (!exact) return launch_rms_fast(c, x, w, eps, T, H, out);
  if (rms_runs_fit(H, x, w, out)) return launch_rms_exact_runs(c, x, w, eps, T, H, out);
  float *d_s;
  NX_TRY(ws(c, WS_SUMSQ, (size_t)T, &d_s));
  NX_TRY(launch_sumsq_exact(c, x, T, H, d_s));
  return launch_rms_apply(c, x, d_s, w, eps, T, H, out);
}

int nx_rms_norm(nx_ctx *c, const float *x, size_t x_len, const float *w, size_t w_len, float eps,
                int T, int H, int exact, float *out) {
  NX_TRY(check_ctx(c));
  NX_TRY(check_norm(x, x_len, w, w_len, T, H, out));
  if (T == 0 || H == 0) return NX_OK;
  const size_t n = (size_t)T * H;
  float *d_x, *d_w, *d_o;
  NX_TRY(ws(c, WS_XIN, n, &d_x));
  NX_TRY(ws(c, WS_NORM_W, (size_t)H, &d_w));
  NX_TRY(ws(c, WS_OUT, n, &d_o));
  NX_HIP(hipMemcpyAsync(d_x, x, n * 4, hipMemcpyHostToDevice, c->stream));
  NX_HIP(hipMemcpyAsync(d_w, w, (size_t)H * 4, hipMemcpyHostToDevice, c->stream));
  NX_TRY(nx_rms_norm_dev(c, d_x, n, d_w, (size_t)H, eps, T, H, exact, d_o));
  NX_HIP(hipMemcpyAsync(out, d_o, n * 4, hipMemcpyDeviceToHost, c->stream));
  NX_HIP(hipStreamSynchronize(c->stream));
  return NX_OK;
}

int nx_permute(nx_ctx *c, const int32_t *experts, const int32_t *counts, int T, int k, int E,
               int32_t *ecount, int32_t *offsets, int32_t *ptok, int32_t *pslot, int32_t *inv) {
  NX_TRY(check_ctx(c));
  if (T < 0 || k < 0 || E <= 0) return fail(NX_ERR_INVALID_ARG, "invalid sizes");
  if (E > 1024) return fail(NX_ERR_UNSUPPORTED, "permutation supports at most 1024 experts");
  if (T > 0 && (!experts || !counts || !inv)) return fail(NX_ERR_INVALID_ARG, "null buffer");
  if (!ecount || !offsets) return fail(NX_ERR_INVALID_ARG, "null buffer");
  // host-side validation: every listed expert in range, at most once per token
  size_t pairs = 0;
  std::vector<int> seen(E, -1);
  for (int t = 0; t < T; ++t) {
    if (counts[t] < 0 || counts[t] > k) return fail(NX_ERR_INVALID_ARG, "route count out of range");
    for (int r = 0; r < counts[t]; ++r) {
      const int e = experts[(size_t)t * k + r];
      if (e < 0 || e >= E) return fail(NX_ERR_INVALID_ARG, "expert index out of range");
      if (seen[e] == t) return fail(NX_ERR_INVALID_ARG, "expert listed twice for one token");
      seen[e] = t;
    }
    pairs += counts[t];
  }
  if (pairs > 0 && (!ptok || !pslot)) return fail(NX_ERR_INVALID_ARG, "null buffer");
  int32_t *d_exp, *d_cnt, *d_ec, *d_off, *d_pt, *d_ps, *d_inv, *d_act;
  const size_t tk = std::max<size_t>((size_t)T * k, 1);
  NX_TRY(ws(c, WS_ROUTE_EXPERT, tk, &d_exp));
  NX_TRY(ws(c, WS_ROUTE_COUNT, std::max(T, 1), &d_cnt));
  NX_TRY(ws(c, WS_EXPERT_COUNT, E, &d_ec));
  NX_TRY(ws(c, WS_OFFSETS, E + 1, &d_off));
  NX_TRY(ws(c, WS_PERM_TOKEN, tk, &d_pt));
  NX_TRY(ws(c, WS_PERM_SLOT, tk, &d_ps));
  NX_TRY(ws(c, WS_INV_POS, tk, &d_inv));
  NX_TRY(ws(c, WS_ACTIVE, E + 1, &d_act));
  if (T > 0) {
    NX_HIP(hipMemcpyAsync(d_exp, experts, (size_t)T * k * 4, hipMemcpyHostToDevice, c->stream));
    NX_HIP(hipMemcpyAsync(d_cnt, counts, (size_t)T * 4, hipMemcpyHostToDevice, c->stream));
  }
  NX_TRY(launch_permute(c, d_exp, d_cnt, T, k, E, 0, d_ec, d_off, d_pt, d_ps, d_inv, d_act, nullptr,
                        0));
  NX_HIP(hipMemcpyAsync(ecount, d_ec, (size_t)E * 4, hipMemcpyDeviceToHost, c->stream));
  NX_HIP(hipMemcpyAsync(offsets, d_off, (size_t)(E + 1) * 4, hipMemcpyDeviceToHost, c->stream));
  if (pairs > 0) {
    NX_HIP(hipMemcpyAsync(ptok, d_pt, pairs * 4, hipMemcpyDeviceToHost, c->stream));
    NX_HIP(hipMemcpyAsync(pslot, d_ps, pairs * 4, hipMemcpyDeviceToHost, c->stream));
  }
  if (T > 0 && k > 0)
    NX_HIP(hipMemcpyAsync(inv, d_inv, (size_t)T * k * 4, hipMemcpyDeviceToHost, c->stream));
  NX_HIP(hipStreamSynchronize(c->stream));
  return NX_OK;
}

// ------------------------------------------------------------------- experts
int nx_experts_create(nx_ctx *c, int fmt, int E, int H, int F, nx_experts **out) {
  NX_TRY(check_ctx(c));
  if (!out) return fail(NX_ERR_INVALID_ARG, "null output pointer");
  *out = nullptr;
  FormatInfo fi;
  if (!format_info(fmt, &fi)) return fail(NX_ERR_INVALID_ARG, "unknown weight format " + std::to_string(fmt));
  if (E <= 0) return fail(NX_ERR_INVALID_ARG, "MoE expert weight lists must be non-empty and aligned");
  if (H <= 0 || F <= 0) return fail(NX_ERR_INVALID_ARG, "hidden and ff_dim must be positive");
  if (fmt != NX_FMT_F32 && (H % fi.block || F % fi.block))
    return fail(NX_ERR_UNSUPPORTED, std::string(fmt_name(fmt)) + " experts need hidden and ff_dim to be multiples of " +
                                        std::to_string(fi.block));
  nx_experts *ex = new nx_experts();
  ex->ctx = c;
  ex->device = c->device;
  ex->fmt = fmt;
  ex->E = E;
  ex->H = H;
  ex->F = F;
  int rc = init_plane(ex, ex->role[NX_ROLE_GATE], E, F, H);
  if (!rc) rc = init_plane(ex, ex->role[NX_ROLE_UP], E, F, H);
  if (!rc) rc = init_plane(ex, ex->role[NX_ROLE_DOWN], E, H, F);
  if (rc) {
    nx_experts_destroy(ex);
    return rc;
  }
  *out = ex;
  return NX_OK;
}

int nx_experts_add_shared(nx_ctx *c, nx_experts *ex, int Fs) {
  NX_TRY(check_ctx(c));
  if (!ex) return fail(NX_ERR_INVALID_ARG, "null expert set");
  if (ex->Fs) return fail(NX_ERR_INVALID_ARG, "expert set already has a shared expert");
  FormatInfo fi;
  format_info(ex->fmt, &fi);
  if (Fs <= 0) return fail(NX_ERR_INVALID_ARG, "shared ff_dim must be positive");
  if (ex->fmt != NX_FMT_F32 && Fs % fi.block)
    return fail(NX_ERR_UNSUPPORTED, "shared ff_dim must be a multiple of the block size");
  NX_TRY(init_plane(ex, ex->shared[NX_ROLE_GATE], 1, Fs, ex->H));
  NX_TRY(init_plane(ex, ex->shared[NX_ROLE_UP], 1, Fs, ex->H));
  NX_TRY(init_plane(ex, ex->shared[NX_ROLE_DOWN], 1, ex->H, Fs));
  ex->Fs = Fs;
  return NX_OK;
}

int nx_experts_load(nx_ctx *c, nx_experts *ex, int expert, int role, const void *src,
                    size_t src_bytes, int on_device) {
  NX_TRY(check_ctx(c));
  if (!ex || !src) return fail(NX_ERR_INVALID_ARG, "null argument");
  if (role < 0 || role > 2) return fail(NX_ERR_INVALID_ARG, "unknown role");
  RolePlane *pl;
  size_t qoff = 0, moff = 0;
  if (expert == NX_EXPERT_SHARED) {
    if (!ex->Fs) return fail(NX_ERR_INVALID_ARG, "expert set has no shared expert");
    pl = &ex->shared[role];
  } else {
    if (expert < 0 || expert >= ex->E) return fail(NX_ERR_INVALID_ARG, "expert index out of range");
    pl = &ex->role[role];
    qoff = pl->qs_stride * expert;
    moff = pl->meta_stride * expert;
  }
  const size_t n = (size_t)pl->rows * pl->cols;
  const size_t need = gguf_bytes(ex->fmt, n);
  if (src_bytes < need) return fail(NX_ERR_TRUNCATED, std::string(fmt_name(ex->fmt)) + " tensor payload is truncated");
  const void *d_src = src;
  void *tmp = nullptr;
  if (!on_device) {
    if (hipMalloc(&tmp, need) != hipSuccess) {
      (void)hipGetLastError();
      return fail(NX_ERR_OOM, "staging allocation failed");
    }
    hipError_t e = hipMemcpyAsync(tmp, src, need, hipMemcpyHostToDevice, c->stream);
    if (e != hipSuccess) {
      (void)hipFree(tmp);
      return fail(NX_ERR_DEVICE, std::string("hipMemcpyAsync: ") + hipGetErrorString(e));
    }
    d_src = tmp;
  }
  int rc = launch_repack(c, ex->fmt, d_src, *pl, pl->qs + qoff,
                         pl->meta ? pl->meta + moff : nullptr);
  hipError_t e = hipStreamSynchronize(c->stream);
  if (tmp) (void)hipFree(tmp);
  if (rc) return rc;
  if (e != hipSuccess) return fail(NX_ERR_DEVICE, std::string("hipStreamSynchronize: ") + hipGetErrorString(e));
  return NX_OK;
}

int nx_experts_info(const nx_experts *ex, int *fmt, int *E, int *H, int *F, int *Fs, size_t *bytes) {
  if (!ex) return fail(NX_ERR_INVALID_ARG, "null expert set");
  if (fmt) *fmt = ex->fmt;
  if (E) *E = ex->E;
  if (H) *H = ex->H;
  if (F) *F = ex->F;
  if (Fs) *Fs = ex->Fs;
  if (bytes) *bytes = ex->device_bytes;
  return NX_OK;
}

// The set may outlive its context (its context pointer is not followed
// here): hipFree waits for the device's work in flight before it frees.
int nx_experts_destroy(nx_experts *ex) {
  if (!ex) return NX_OK;
  (void)hipSetDevice(ex->device);
  for (void *p : ex->allocs) (void)hipFree(p);
  delete ex;
  return NX_OK;
}

// ------------------------------------------------------------ dense matrices
int nx_matrix_create(nx_ctx *c, int fmt, int rows, int cols, nx_matrix **out) {
  NX_TRY(check_ctx(c));
  if (!out) return fail(NX_ERR_INVALID_ARG, "null output pointer");
  *out = nullptr;
  FormatInfo fi;
  if (!format_info(fmt, &fi)) return fail(NX_ERR_INVALID_ARG, "unknown weight format " + std::to_string(fmt));
  if (rows <= 0 || cols <= 0) return fail(NX_ERR_INVALID_ARG, "matrix rows and cols must be positive");
  if (fmt != NX_FMT_F32 && cols % fi.block)
    return fail(NX_ERR_UNSUPPORTED, std::string(fmt_name(fmt)) + " matrices need cols to be a multiple of " +
                                        std::to_string(fi.block));
  nx_experts *ex = new nx_experts();
  ex->ctx = c;
  ex->device = c->device;
  ex->fmt = fmt;
  ex->E = 1;
  ex->H = rows;
  ex->F = cols;
  RolePlane &pl = ex->role[NX_ROLE_DOWN];
  int rc = NX_OK;
  // narrow rows are addressed through one 32-bit buffer range per plane
  plane_layout(fmt, pl, rows, cols);
  if (pl.qs_stride > 0xFFFFFF00ull || pl.meta_stride > 0xFFFFFF00ull)
    rc = fail(NX_ERR_UNSUPPORTED, "matrix plane over 4 GiB resident");
  else if (!gemv_row_fits(fmt, pl.nseg))
    rc = fail(NX_ERR_UNSUPPORTED, std::string(fmt_name(fmt)) + " rows of " + std::to_string(cols) +
                                      " weights are too long for the register-resident GEMV");
  if (!rc) rc = init_plane(ex, pl, 1, rows, cols);
  if (rc) {
    nx_experts_destroy(ex);
    return rc;
  }
  *out = new nx_matrix{ex, rows, cols};
  return NX_OK;
}

int nx_matrix_load(nx_ctx *c, nx_matrix *m, const void *src, size_t src_bytes, int on_device) {
  NX_TRY(check_ctx(c));
  if (!m || !src) return fail(NX_ERR_INVALID_ARG, "null argument");
  // InferenceEngine::matvec's weight check, counted in weight elements
  FormatInfo fi;
  format_info(m->ex->fmt, &fi);
  const size_t have = m->ex->fmt == NX_FMT_F32 ? src_bytes / 4 : src_bytes / fi.block_bytes * fi.block;
  const size_t need = (size_t)m->rows * m->cols;
  if (have < need)
    return fail(NX_ERR_SHAPE, "Matvec weight too small: got " + std::to_string(have) +
                                  ", expected at least " + std::to_string(need));
  return nx_experts_load(c, m->ex, 0, NX_ROLE_DOWN, src, src_bytes, on_device);
}

int nx_matrix_info(const nx_matrix *m, int *fmt, int *rows, int *cols, size_t *device_bytes) {
  if (!m) return fail(NX_ERR_INVALID_ARG, "null matrix");
  if (fmt) *fmt = m->ex->fmt;
  if (rows) *rows = m->rows;
  if (cols) *cols = m->cols;
  if (device_bytes) *device_bytes = m->ex->device_bytes;
  return NX_OK;
}

int nx_matrix_destroy(nx_matrix *m) {
  if (!m) return NX_OK;
  nx_experts_destroy(m->ex);
  delete m;
  return NX_OK;
}

static int check_matvec(const nx_matrix *m, const float *x, size_t x_len, int T, const float *y) {
  if (!m) return fail(NX_ERR_INVALID_ARG, "null matrix");
  if (T < 0) return fail(NX_ERR_INVALID_ARG, "negative size");
  const size_t need_x = (size_t)T * m->cols;
  if (x_len != need_x)
    return fail(NX_ERR_SHAPE, "Matvec input shape mismatch: got " + std::to_string(x_len) +
                                  ", expected " + std::to_string(need_x));
  if (T > 0 && (!x || !y)) return fail(NX_ERR_INVALID_ARG, "null buffer");
  return NX_OK;
}

int nx_matvec_dev(nx_ctx *c, const nx_matrix *m, const float *d_x, size_t x_len, int T, float *d_y) {
  NX_TRY(check_ctx(c));
  NX_TRY(check_matvec(m, d_x, x_len, T, d_y));
  if (T == 0) return NX_OK;
  return launch_gemv_matrix(c, m->ex->fmt, m->ex->role[NX_ROLE_DOWN], d_x, T, d_y);
}

int nx_matvec(nx_ctx *c, const nx_matrix *m, const float *x, size_t x_len, int T, float *y) {
  NX_TRY(check_ctx(c));
  NX_TRY(check_matvec(m, x, x_len, T, y));
  if (T == 0) return NX_OK;
  const size_t ny = (size_t)T * m->rows;
  float *d_x, *d_y;
  NX_TRY(ws(c, WS_MAT_X, x_len, &d_x));
  NX_TRY(ws(c, WS_MAT_Y, ny, &d_y));
  NX_HIP(hipMemcpyAsync(d_x, x, x_len * 4, hipMemcpyHostToDevice, c->stream));
  NX_TRY(launch_gemv_matrix(c, m->ex->fmt, m->ex->role[NX_ROLE_DOWN], d_x, T, d_y));
  NX_HIP(hipMemcpyAsync(y, d_y, ny * 4, hipMemcpyDeviceToHost, c->stream));
  NX_HIP(hipStreamSynchronize(c->stream));
  return NX_OK;
}

// ------------------------------------------------------------------- forward
int nx_moe_forward_dev(nx_ctx *c, const nx_experts *ex, const float *d_x, const float *d_logits,
                       int T, int k, int score_mode, int path, float *d_out) {
  return moe_forward(c, ex, d_x, d_logits, T, k, score_mode, path, d_out, nullptr);
}

}  // extern "C"

int nx::moe_forward(nx_ctx *c, const nx_experts *ex, const float *d_x, const float *d_logits,
                    int T, int k, int score_mode, int path, float *d_out,
                    const float *d_residual) {
  NX_TRY(check_ctx(c));
  if (!ex) return fail(NX_ERR_INVALID_ARG, "null expert set");
  if (ex->ctx != c) return fail(NX_ERR_INVALID_ARG, "expert set belongs to another context");
  if (T < 0) return fail(NX_ERR_INVALID_ARG, "negative token count");
  if (score_mode != NX_SCORE_SOFTMAX && score_mode != NX_SCORE_SIGMOID)
    return fail(NX_ERR_INVALID_ARG, "unknown score mode");
  if (path < NX_PATH_AUTO || path > NX_PATH_MFMA_SPLIT) return fail(NX_ERR_INVALID_ARG, "unknown path");
  if (k <= 0) return fail(NX_ERR_NO_ROUTES, "MoE router produced no routes");  // src/engine/mod.rs:989-991
  if (T == 0) return NX_OK;
  if (!d_x || !d_logits || !d_out) return fail(NX_ERR_INVALID_ARG, "null buffer");
  const int E = ex->E, H = ex->H;
  if (E > 1024) return fail(NX_ERR_UNSUPPORTED, "at most 1024 experts");
  if (k > 64) return fail(NX_ERR_UNSUPPORTED, "top_k above 64");
  const bool shared = ex->Fs > 0;
  const size_t tk = (size_t)T * k;
  const size_t pairs_total = tk + (shared ? (size_t)T : 0);

  int32_t *d_exp, *d_cnt, *d_ec, *d_off, *d_pt, *d_ps, *d_inv, *d_act;
  float *d_w, *d_ypair;
  NX_TRY(ws(c, WS_ROUTE_EXPERT, tk, &d_exp));
  NX_TRY(ws(c, WS_ROUTE_WEIGHT, tk, &d_w));
  NX_TRY(ws(c, WS_ROUTE_COUNT, (size_t)T, &d_cnt));
  NX_TRY(ws(c, WS_EXPERT_COUNT, (size_t)E, &d_ec));
  NX_TRY(ws(c, WS_OFFSETS, (size_t)E + 1, &d_off));
  NX_TRY(ws(c, WS_PERM_TOKEN, tk, &d_pt));
  NX_TRY(ws(c, WS_PERM_SLOT, tk, &d_ps));
  NX_TRY(ws(c, WS_INV_POS, tk, &d_inv));
  NX_TRY(ws(c, WS_ACTIVE, (size_t)E + 1, &d_act));
  // the routes this call writes become the context's last routes only once
  // every launch of the call is enqueued: a later workspace failure can move
  // the slots carved above, and a failed call leaves no routes to read back
  c->last_exp = nullptr;
  auto remember_routes = [&] {
    c->last_exp = d_exp;
    c->last_w = d_w;
    c->last_cnt = d_cnt;
    c->last_T = T;
    c->last_k = k;
    return NX_OK;
  };

  int use = path;
  if (ex->fmt == NX_FMT_F16 || ex->fmt == NX_FMT_BF16) {
    // no MFMA operand path for these formats
    if (use == NX_PATH_MFMA_F16 || use == NX_PATH_MFMA_BF16 || use == NX_PATH_MFMA_SPLIT)
      return fail(NX_ERR_UNSUPPORTED, std::string(fmt_name(ex->fmt)) + " experts run on the GEMV path only");
    use = NX_PATH_GEMV;
  }
  if (ex->fmt == NX_FMT_Q2_K && (use == NX_PATH_MFMA_F16 || use == NX_PATH_MFMA_BF16)) {
    // Q2_K: the GEMV and the split-activation MFMA path (no grouped GEMM)
    return fail(NX_ERR_UNSUPPORTED,
                "Q2_K experts run on the GEMV and the split-activation MFMA path only");
  }
  // AUTO takes bf16 operands on the grouped GEMM: fp16's range ends at
  // 65504, which SwiGLU activations of real models can pass; bf16 keeps
  // float32's range, runs as fast here, and stays within the MFMA bar.
  if (use == NX_PATH_AUTO) {
    // Tokens per active expert, with the active count expected under
    // uniform routing, E (1 - (1 - k/E)^T).
    const double kk = std::min(1.0, (double)k / E);
    const double act = std::max(1.0, E * (1.0 - std::pow(1.0 - kk, (double)T)));
    const double tpe = (double)T * k / act;
    if (ex->fmt == NX_FMT_Q2_K) {
      // The GEMV or the split-activation path (Q2_K has no grouped GEMM).
      // Measured (ms, GEMV / split): Mixtral 2 tokens 0.101 / 0.122, 4:
      // 0.173 / 0.188, 8: 0.243 / 0.193, 32: 0.939 / 0.238, 128: 2.82 /
      // 0.534; Qwen3 4 tokens 0.048 / 0.048, 8: 0.093 / 0.065, 512: 1.84 /
      // 0.265; DeepSeek with its shared expert 2 tokens 0.119 / 0.137, 4:
      // 0.307 / 0.218, 64: 44.1 / 1.52.
      if (shared)
        use = (ex->Fs == ex->F && T >= 4) ? NX_PATH_MFMA_SPLIT : NX_PATH_GEMV;
      else
        use = (tpe >= 1.8 || ((long)T * k >= 64 && tpe >= 1.2)) ? NX_PATH_MFMA_SPLIT
                                                                 : NX_PATH_GEMV;
    } else if (ex->fmt == NX_FMT_Q4_K && shared && ex->Fs == ex->F) {
      // A shared expert sees every token: the GEMV walks it a token pair at
      // a time, the split-activation path 16 tokens at a time.  Measured
      // (DeepSeek shapes, ms, GEMV / split / grouped GEMM): 2 tokens 0.115 /
      // 0.173 / 0.268, 4: 0.270 / 0.264 / 0.321, 8: 0.887 / 0.508 / 0.588,
      // 16: 3.69 / 0.904 / 0.996, 32: - / 1.31 / 1.52, 64: - / 1.76 / 2.04;
      // the grouped GEMM (64-pair tiles at these counts) from the routed
      // experts' 8 tokens each: 192 tokens (6 each) split 2.08-2.18 / GEMM
      // 2.11, 256 tokens (8 each) 2.19-2.29 / 2.13.
      if (tpe >= 8.0)
        use = NX_PATH_MFMA_BF16;
      else
        use = T >= 4 ? NX_PATH_MFMA_SPLIT : NX_PATH_GEMV;
    } else if ((ex->fmt == NX_FMT_Q4_K ||
                ((ex->fmt == NX_FMT_Q4_0 || ex->fmt == NX_FMT_Q8_0) && mfv_supports(ex))) &&
               !shared) {
      // Measured crossovers (Mixtral and Qwen3 shapes): the GEMV re-reads an
      // expert's weights per pair of its tokens and wins below ~2 tokens per
      // expert; the split-activation MFMA path reads them once per 16 tokens
      // and wins up to ~12 (Mixtral: 0.31 against 0.36 ms at 8 tokens per
      // expert, 0.45 against 0.36 at 16; Qwen3: 0.17 / 0.20 at 8, 0.24 /
      // 0.21 at 16); the grouped GEMM beyond.  Q4_0 (ms, GEMV / split /
      // grouped GEMM): Mixtral 2 tokens per expert 0.183 / 0.233 / 0.290,
      // 4: 0.368 / 0.253 / 0.295, 8: - / 0.272 / 0.297, 16: - / 0.343 /
      // 0.299; Qwen3 1.2: 0.079 / 0.069 / 0.095, 4: 0.285 / 0.135 / 0.160.
      // Q8_0: Mixtral 2 tokens per expert 0.287 / 0.317 / 0.351, 4: 0.600 /
      // 0.344 / 0.359, 8: - / 0.366 / 0.379, 16: - / 0.435 / 0.383; Qwen3
      // 1.2: 0.083 / 0.081 / 0.103, 4: 0.347 / 0.169 / 0.184, 8: - / 0.175 /
      // 0.188, 16: - / 0.247 / 0.192.  (With a shared expert Q4_0 and Q8_0
      // keep the rule below: at DeepSeek's shape the split path and the
      // grouped GEMM are within 4% from 16 tokens.)
      if (tpe >= 12.0)
        use = NX_PATH_MFMA_BF16;
      else if (tpe >= 3.0 || ((long)T * k >= 64 && tpe >= 1.2))
        use = NX_PATH_MFMA_SPLIT;
      else
        use = NX_PATH_GEMV;
    } else if (ex->fmt == NX_FMT_F32) {
      // f32 weights keep their precision on the GEMV; the bf16 grouped GEMM
      // only once experts see 32 tokens on average
      const long active_max = std::min<long>(E, (long)T * k);
      use = ((long)T * k >= 32 * active_max) ? NX_PATH_MFMA_BF16 : NX_PATH_GEMV;
    } else {
      // The grouped GEMM from ~3 tokens per routed expert (Mixtral Q8_0 and
      // Q4_0 at 8 and 16 tokens, Qwen3 Q8_0 at 32), or from 6 tokens when a
      // shared expert sees them all: the GEMV passes over the shared expert
      // per pair of tokens and over the routed experts per token group
      // (DeepSeek shapes with a shared expert: GEMV 0.29 / 0.81 / 10.5 ms
      // at 4 / 8 / 32 tokens, grouped GEMM 0.36 / 0.61 / 1.44 ms).
      use = (tpe >= 3.0 || (shared && T >= 6)) ? NX_PATH_MFMA_BF16 : NX_PATH_GEMV;
    }
  }

  if (use == NX_PATH_GEMV) {
    NX_TRY(ws(c, WS_YPAIR, pairs_total * H, &d_ypair));
    // one token: the gate/up kernel routes it itself (no router launch)
    const bool route_in_gemv = NX_ROUTE_IN_GEMV && T == 1 && E <= NX_ROUTE_IN_GEMV_MAX_E && k <= 64;
    if (!route_in_gemv && route_permute_fusable(T, E, k)) {
      NX_TRY(launch_route_permute(c, d_logits, T, E, k, score_mode, d_exp, d_w, d_cnt, d_ec, d_off,
                                  d_pt, d_ps, d_inv, d_act, 0, nullptr, nullptr, 0));
    } else if (!route_in_gemv) {
      NX_TRY(launch_route(c, d_logits, T, E, k, score_mode, d_exp, d_w, d_cnt));
      NX_TRY(launch_permute(c, d_exp, d_cnt, T, k, E, 0, d_ec, d_off, d_pt, d_ps, d_inv, d_act,
                            nullptr, 0));
    }
    const int fmax = std::max(ex->F, ex->Fs);
    const int act_stride = (fmax + 7) / 8 * 8;
    float *d_actv;
    NX_TRY(ws(c, WS_ACT, pairs_total * act_stride, &d_actv));
    GemvPlan gp{ex, T, k, d_x, d_pt, d_off, d_act, d_actv, act_stride, d_ypair,
                d_w, d_cnt, d_inv, d_out, d_residual};
    gp.pslot = d_ps;
    if (route_in_gemv)
      gp.route = {d_logits, score_mode, d_exp, d_cnt, d_ec, d_off, d_pt, d_ps, d_inv, d_act, d_w};
    NX_TRY(launch_gemv_gateup(c, gp));
    NX_TRY(launch_gemv_down(c, gp));
    return remember_routes();
  }

  if (use == NX_PATH_MFMA_SPLIT) {
    if (!mfv_supports(ex))
      return fail(NX_ERR_UNSUPPORTED,
                  "the split-activation MFMA path takes Q4_K experts, or Q4_0 experts whose "
                  "hidden and FFN widths are multiples of 256");
    if (shared && ex->Fs != ex->F)
      return fail(NX_ERR_UNSUPPORTED,
                  "the split-activation MFMA path takes a shared expert as wide as the routed ones");
    const int max_tiles = mfv_max_tiles(T, k, E, shared);
    int32_t *d_tiles;
    NX_TRY(ws(c, WS_TILES, 2 + 2 * (size_t)max_tiles, &d_tiles));
    // (the fused router lists no shared-expert tiles)
    if (!shared && route_permute_fusable(T, E, k)) {
      NX_TRY(launch_route_permute(c, d_logits, T, E, k, score_mode, d_exp, d_w, d_cnt, d_ec, d_off,
                                  d_pt, d_ps, d_inv, d_act, kMfvTileM, d_tiles, nullptr, 0));
    } else {
      NX_TRY(launch_route(c, d_logits, T, E, k, score_mode, d_exp, d_w, d_cnt));
      NX_TRY(launch_permute(c, d_exp, d_cnt, T, k, E, kMfvTileM, d_ec, d_off, d_pt, d_ps, d_inv,
                            d_act, d_tiles, shared ? T : 0));
    }
    MfvPlan mp{ex, T, k, d_x, d_pt, d_off, d_tiles, max_tiles, d_w, d_cnt, d_inv, d_out, d_residual};
    NX_TRY(launch_mfv(c, mp));
    return remember_routes();
  }

  // grouped GEMM on MFMA
  const bool bf16 = use == NX_PATH_MFMA_BF16;
  // gate/up and down take M-tiles of their own heights: one tile list each
  const long active_max = std::min<long>(E, (long)T * k);
  auto tiles_bound = [&](int tm) {
    return (int)(((long)T * k + tm - 1) / tm + active_max + (shared ? ((long)T + tm - 1) / tm : 0));
  };
  const int tm = gemm_tile_m(ex->fmt, true, T, k, E), tm_down = gemm_tile_m(ex->fmt, false, T, k, E);
  const int max_tiles = tiles_bound(tm), max_tiles_down = tiles_bound(tm_down);
  int32_t *d_tiles, *d_tiles_down;
  NX_TRY(ws(c, WS_TILES, 2 + 2 * (size_t)max_tiles, &d_tiles));
  NX_TRY(ws(c, WS_TILES_DOWN, 2 + 2 * (size_t)max_tiles_down, &d_tiles_down));
  NX_TRY(launch_route(c, d_logits, T, E, k, score_mode, d_exp, d_w, d_cnt));
  NX_TRY(launch_permute(c, d_exp, d_cnt, T, k, E, tm, d_ec, d_off, d_pt, d_ps, d_inv, d_act,
                        d_tiles, shared ? T : 0, tm_down, d_tiles_down));
  void *d_xh, *d_acth;
  // operands in the kernels' K order, rows padded to whole scale windows
  const int x_stride = gemm_kpad(ex->fmt, H);
  const int act_stride = gemm_kpad(ex->fmt, std::max(ex->F, ex->Fs));
  if ((size_t)T * x_stride * 2 >= (1u << 31) || pairs_total * act_stride * 2 >= (1u << 31))
    return fail(NX_ERR_UNSUPPORTED, "activation buffers above 2 GiB");
  NX_TRY(ws_get(c, WS_XH, (size_t)T * x_stride * 2, &d_xh));
  NX_TRY(launch_to_half(c, ex->fmt, d_x, T, H, x_stride, bf16, d_xh));
  NX_TRY(ws_get(c, WS_ACT, pairs_total * act_stride * 2, &d_acth));
  // the down pass splits K when that fills the CUs' rounds better; each
  // split writes its own partial sums, added by the combine
  const int ksplit =
      gemm_down_ksplit(ex->fmt, std::max(ex->F, ex->Fs), H, max_tiles_down,
                       gemm_wg_per_cu(ex->fmt, tm_down) * c->num_cu);
  // the bf16 path keeps its per-pair partial sums in bf16 too (half the
  // bytes the down pass writes and the combine reads; two columns per store,
  // so rows of even length)
  const bool ybf = bf16 && H % 2 == 0;
  const size_t y_elems = (size_t)ksplit * pairs_total * H;
  NX_TRY(ws(c, WS_YPAIR, ybf ? (y_elems + 1) / 2 : y_elems, &d_ypair));
  GemmPlan mp{ex,        T,       k,         bf16, d_x,          d_pt,           d_off,
              d_act,     d_tiles, max_tiles, tm,   d_tiles_down, max_tiles_down, tm_down,
              d_acth,    act_stride, d_ypair, ybf, d_xh,         x_stride,       pairs_total,
              ksplit};
  NX_TRY(launch_gemm_gateup(c, mp));
  NX_TRY(launch_gemm_down(c, mp));
  if (ybf)
    NX_TRY(launch_combine_bf16(c, reinterpret_cast<const uint16_t *>(d_ypair), d_w, d_cnt, d_inv,
                               T, k, H, shared, d_out, ksplit, pairs_total * (size_t)H,
                               d_residual));
  else
    NX_TRY(launch_combine(c, d_ypair, d_w, d_cnt, d_inv, T, k, H, shared, d_out, ksplit,
                          pairs_total * (size_t)H, d_residual));
  return remember_routes();
}

extern "C" {

int nx_moe_forward_noalloc(nx_ctx *c, const nx_experts *ex, const float *d_x,
                           const float *d_logits, int T, int k, int score_mode, int path,
                           float *d_out) {
  NX_TRY(check_ctx(c));
  if (!c->scratch) return fail(NX_ERR_DEVICE, "no scratch array on this context's device");
  // profiling creates HIP events: this entry point takes no resources at all
  if (c->profile)
    return fail(NX_ERR_INVALID_ARG, "nx_moe_forward_noalloc does not run with profiling enabled");
  c->scratch_mode = true;
  c->scratch_used = 0;
  for (auto &s : c->scratch_slot) s = DevBuf{};
  const int rc = moe_forward(c, ex, d_x, d_logits, T, k, score_mode, path, d_out, nullptr);
  c->scratch_mode = false;
  return rc;
}

int nx_moe_last_routes(nx_ctx *c, int T, int k, int32_t *experts, float *weights,
                       int32_t *counts) {
  NX_TRY(check_ctx(c));
  if (!c->last_exp)
    return fail(NX_ERR_INVALID_ARG, "no routes recorded: no forward has completed on this context");
  if (T != c->last_T || k != c->last_k)
    return fail(NX_ERR_SHAPE, "the last forward routed " + std::to_string(c->last_T) +
                                  " tokens with top_k " + std::to_string(c->last_k));
  if (!experts || !weights || !counts) return fail(NX_ERR_INVALID_ARG, "null buffer");
  const size_t tk = (size_t)T * k;
  NX_HIP(hipMemcpyAsync(experts, c->last_exp, tk * 4, hipMemcpyDeviceToHost, c->stream));
  NX_HIP(hipMemcpyAsync(weights, c->last_w, tk * 4, hipMemcpyDeviceToHost, c->stream));
  NX_HIP(hipMemcpyAsync(counts, c->last_cnt, (size_t)T * 4, hipMemcpyDeviceToHost, c->stream));
  NX_HIP(hipStreamSynchronize(c->stream));
  return NX_OK;
}

int nx_moe_forward(nx_ctx *c, const nx_experts *ex, const float *x, const float *logits, int T,
                   int k, int score_mode, int path, float *out) {
  NX_TRY(check_ctx(c));
  if (!ex) return fail(NX_ERR_INVALID_ARG, "null expert set");
  if (k <= 0) return fail(NX_ERR_NO_ROUTES, "MoE router produced no routes");
  if (T < 0) return fail(NX_ERR_INVALID_ARG, "negative token count");
  if (T == 0) return NX_OK;
  if (!x || !logits || !out) return fail(NX_ERR_INVALID_ARG, "null buffer");
  const size_t nx_ = (size_t)T * ex->H, nl = (size_t)T * ex->E;
  float *d_x, *d_l, *d_o;
  NX_TRY(ws(c, WS_XIN, nx_, &d_x));
  NX_TRY(ws(c, WS_LOGITS, nl, &d_l));
  NX_TRY(ws(c, WS_OUT, nx_, &d_o));
  NX_HIP(hipMemcpyAsync(d_x, x, nx_ * 4, hipMemcpyHostToDevice, c->stream));
  NX_HIP(hipMemcpyAsync(d_l, logits, nl * 4, hipMemcpyHostToDevice, c->stream));
  NX_TRY(nx_moe_forward_dev(c, ex, d_x, d_l, T, k, score_mode, path, d_o));
  NX_HIP(hipMemcpyAsync(out, d_o, nx_ * 4, hipMemcpyDeviceToHost, c->stream));
  NX_HIP(hipStreamSynchronize(c->stream));
  return NX_OK;
}

}  // extern "C"

// tokens up to which the exact block runs its prologue as one launch
#ifndef NX_BLOCK_PROLOGUE_MAX_T
#define NX_BLOCK_PROLOGUE_MAX_T 64
#endif
constexpr int BLOCK_PROLOGUE_MAX_T = NX_BLOCK_PROLOGUE_MAX_T;

// One MoE block: normed = rms_norm(hidden), logits = W_r . normed,
// hidden += MoE(normed, logits).  The FFN half of decode_with_cache
// (src/engine/mod.rs:1129-1142) with the MoE layer in place of the dense FFN.
int nx_moe_block_dev(nx_ctx *c, const nx_experts *ex, float *d_hidden, const float *d_norm_w,
                     size_t norm_len, float eps, const float *d_router_w, size_t router_len,
                     int T, int k, int score_mode, int path, int exact) {
  NX_TRY(check_ctx(c));
  if (!ex) return fail(NX_ERR_INVALID_ARG, "null expert set");
  if (T < 0) return fail(NX_ERR_INVALID_ARG, "negative token count");
  const int E = ex->E, H = ex->H;
  const size_t n = (size_t)T * H;
  NX_TRY(check_norm(d_hidden, n, d_norm_w, norm_len, T, H, d_hidden));
  NX_TRY(check_logits(d_router_w, router_len, d_hidden, n, T, E, H, d_hidden));
  if (T == 0) return NX_OK;
  float *d_n, *d_l;
  NX_TRY(ws(c, WS_NORMED, n, &d_n));
  NX_TRY(ws(c, WS_BLK_LOGITS, (size_t)T * E, &d_l));
  if (exact && T <= BLOCK_PROLOGUE_MAX_T &&
      block_prologue_fits(H, d_hidden, d_norm_w, d_router_w, d_n)) {
    // one launch: each workgroup repeats its token's (parallel, latency-bound)
    // sum-of-squares chain instead of waiting on a separate kernel
    NX_TRY(launch_block_prologue(c, d_hidden, d_norm_w, eps, d_router_w, T, E, H, d_n, d_l));
  } else {
    NX_TRY(nx_rms_norm_dev(c, d_hidden, n, d_norm_w, norm_len, eps, T, H, exact, d_n));
    NX_TRY(launch_router_logits(c, d_router_w, d_n, T, E, H, exact != 0, d_l));
  }
  // the residual add (hidden + layer output, one rounding) happens in the
  // combine's final write
  return moe_forward(c, ex, d_n, d_l, T, k, score_mode, path, d_hidden, d_hidden);
}

int nx_moe_block(nx_ctx *c, const nx_experts *ex, float *hidden, const float *norm_w,
                 size_t norm_len, float eps, const float *router_w, size_t router_len, int T,
                 int k, int score_mode, int path, int exact) {
  NX_TRY(check_ctx(c));
  if (!ex) return fail(NX_ERR_INVALID_ARG, "null expert set");
  if (T < 0) return fail(NX_ERR_INVALID_ARG, "negative token count");
  const int E = ex->E, H = ex->H;
  const size_t n = (size_t)T * H;
  NX_TRY(check_norm(hidden, n, norm_w, norm_len, T, H, hidden));
  NX_TRY(check_logits(router_w, router_len, hidden, n, T, E, H, hidden));
  if (T == 0) return NX_OK;
  float *d_h, *d_nw, *d_rw;
  NX_TRY(ws(c, WS_BLK_HIDDEN, n, &d_h));
  NX_TRY(ws(c, WS_NORM_W, (size_t)H, &d_nw));
  NX_TRY(ws(c, WS_ROUTER_W, (size_t)E * H, &d_rw));
  NX_HIP(hipMemcpyAsync(d_h, hidden, n * 4, hipMemcpyHostToDevice, c->stream));
  NX_HIP(hipMemcpyAsync(d_nw, norm_w, (size_t)H * 4, hipMemcpyHostToDevice, c->stream));
  NX_HIP(hipMemcpyAsync(d_rw, router_w, (size_t)E * H * 4, hipMemcpyHostToDevice, c->stream));
  NX_TRY(nx_moe_block_dev(c, ex, d_h, d_nw, (size_t)H, eps, d_rw, (size_t)E * H, T, k, score_mode,
                          path, exact));
  NX_HIP(hipMemcpyAsync(hidden, d_h, n * 4, hipMemcpyDeviceToHost, c->stream));
  NX_HIP(hipStreamSynchronize(c->stream));
  return NX_OK;
}
