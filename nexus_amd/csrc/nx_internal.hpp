// nx_internal.hpp — host-side internals of libnexus_hip.so (context, resident
// expert layout, workspace, launch helpers).  Not part of the C ABI.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <vector>

#include "../../include/nexus_hip.h"

namespace nx {

int fail(int code, const std::string &msg);
void clear_error();

#define NX_HIP(call)                                                                       \
  do {                                                                                     \
    hipError_t nx_e_ = (call);                                                             \
    if (nx_e_ != hipSuccess)                                                               \
      return ::nx::fail(NX_ERR_DEVICE, std::string(#call) + ": " + hipGetErrorString(nx_e_)); \
  } while (0)

#define NX_TRY(expr)        \
  do {                      \
    int nx_rc_ = (expr);    \
    if (nx_rc_) return nx_rc_; \
  } while (0)

// Resident per-format layout.  A GGUF block of `block` elements and
// `block_bytes` bytes is split into a code plane (qs_bytes per block) and a
// scale plane (meta_bytes per block); the code plane of each row is cut into
// 32-byte segments stored half-interleaved, rows of more than 64 segments in
// panels of 64 segments (nx_device.hpp).  Q4_K: 144 B =
// 128 B codes + 16 B {d, dmin, scales12}; Q8_0: 34 B = 32 B codes + 2 B d;
// Q4_0: 18 B = 16 B codes + 2 B d; F32: rows padded to 8 floats, no scales.
struct FormatInfo {
  int fmt;
  int block;       // elements per block
  int block_bytes; // GGUF bytes per block
  int qs_bytes;    // code-plane bytes per block
  int meta_bytes;  // scale-plane bytes per block
};
bool format_info(int fmt, FormatInfo *fi);

// One matrix role (gate / up / down) for all experts of a set:
// expert e's codes start at qs + e * qs_stride, scales at meta + e * meta_stride.
struct RolePlane {
  uint8_t *qs = nullptr;
  uint8_t *meta = nullptr;
  size_t qs_stride = 0;    // bytes per expert (code plane)
  size_t meta_stride = 0;  // bytes per expert (scale plane)
  int rows = 0;
  int cols = 0;        // logical columns
  int nseg = 0;        // 32-byte code segments per row
  // bytes per row: nseg * 32 (codes) when a row is one panel, else whole
  // zero-padded panels of 64 segments (plane bytes = rows * row_qs)
  uint32_t row_qs = 0;    // code-plane bytes per row
  uint32_t row_meta = 0;  // scale-plane bytes per row
};

struct KernelStat {
  std::string name;
  int launches = 0;
  double total_ms = 0.0;
};

struct PendingEvent {
  int stat;
  hipEvent_t start, stop;
};

// Device scratch owned by a context; grown on demand, never shrunk.
struct DevBuf {
  void *ptr = nullptr;
  size_t cap = 0;
};

}  // namespace nx

struct nx_ctx {
  int device = 0;
  hipStream_t own_stream = nullptr;
  hipStream_t stream = nullptr;
  int num_cu = 0;
  size_t lds_per_cu = 0;  // bytes of LDS per CU
  // workspace
  nx::DevBuf ws[32];
  // The library's static device scratch array on this context's device
  // (hipGetSymbolAddress at context creation), used instead of ws by
  // nx_moe_forward_noalloc: while scratch_mode is set, ws_get carves each
  // slot from it (256-byte aligned, bump order) and never allocates.
  uint8_t *scratch = nullptr;
  bool scratch_mode = false;
  size_t scratch_used = 0;
  nx::DevBuf scratch_slot[32];
  // route arrays of the last forward (for nx_moe_last_routes)
  const int32_t *last_exp = nullptr;
  const float *last_w = nullptr;
  const int32_t *last_cnt = nullptr;
  int last_T = 0, last_k = 0;
  // host-visible staging for blocking calls
  nx::DevBuf host_stage;
  // profiling
  bool profile = false;
  std::vector<nx::KernelStat> stats;
  std::vector<nx::PendingEvent> pending;
  std::vector<hipEvent_t> event_pool;
  // events of the launch in progress (profiling): a kernel started with
  // nx::go takes them into its dispatch, which records them at the kernel's
  // own start and end
  hipEvent_t launch_start = nullptr, launch_stop = nullptr;
  bool launch_timed = false;
};

// one dense weight matrix (rows x cols, row-major as GGUF stores it), held
// as a one-expert set whose down-role plane is the matrix
struct nx_matrix {
  nx_experts *ex = nullptr;
  int rows = 0, cols = 0;
};

struct nx_experts {
  nx_ctx *ctx = nullptr;  // compared, never followed, once the set exists
  int device = 0;         // the device its planes live on
  int fmt = 0;
  int E = 0, H = 0, F = 0, Fs = 0;
  nx::RolePlane role[3];
  nx::RolePlane shared[3];
  size_t device_bytes = 0;
  std::vector<void *> allocs;
};

namespace nx {

// workspace slots
enum WsSlot {
  WS_ROUTE_EXPERT = 0,
  WS_ROUTE_WEIGHT,
  WS_ROUTE_COUNT,
  WS_EXPERT_COUNT,
  WS_OFFSETS,
  WS_PERM_TOKEN,
  WS_PERM_SLOT,
  WS_INV_POS,
  WS_ACTIVE,   // [E + 1]: active expert ids, then n_active at index E
  WS_ACT,      // SwiGLU activations
  WS_YPAIR,    // per-pair expert outputs
  WS_XIN,      // device copy of inputs for blocking calls
  WS_LOGITS,
  WS_OUT,
  WS_TILES,    // grouped-GEMM tile list
  WS_XH,       // half-precision copy of activations for the MFMA path
  WS_ROUTER_W, // device copy of the router weight for blocking calls
  WS_NORMED,   // RMSNorm output of a block
  WS_BLK_LOGITS,
  WS_BLK_OUT,
  WS_SUMSQ,
  WS_NORM_W,   // device copy of the norm weight for blocking calls
  WS_BLK_HIDDEN,
  WS_MAT_X,    // device copy of matvec inputs for blocking calls
  WS_MAT_Y,
  WS_MFV_PART, // gate/up partial sums of the split-activation MFMA path
  WS_TILES_DOWN, // grouped-GEMM tile list of the down pass
  WS_PERM_CHUNK, // per-chunk expert counts of the many-workgroup permutation
  WS_COUNT
};
static_assert(WS_COUNT <= 32, "workspace slots of a context");

int ws_get(nx_ctx *c, int slot, size_t bytes, void **out);

// Launch bookkeeping: records HIP events around `launch` when profiling.
int begin_launch(nx_ctx *c, const char *name, int *stat_index);
int end_launch(nx_ctx *c, int stat_index);

// Starts kernel `k` on the context's stream.  While profiling, the dispatch
// records the launch's events (hipExtLaunchKernelGGL), so the measured time
// is the kernel's execution alone: an event pair recorded around the launch
// would add the records' own latency to it.
template <typename K, typename... Args>
void go(nx_ctx *c, K k, dim3 grid, dim3 block, uint32_t lds, Args... args) {
  if (c->launch_start) {
    hipExtLaunchKernelGGL(k, grid, block, lds, c->stream, c->launch_start, c->launch_stop, 0,
                          args...);
    c->launch_timed = true;
  } else {
    hipLaunchKernelGGL(k, grid, block, lds, c->stream, args...);
  }
}

template <typename F>
int launch(nx_ctx *c, const char *name, F &&fn) {
  int si = -1;
  NX_TRY(begin_launch(c, name, &si));
  fn();
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    c->launch_start = c->launch_stop = nullptr;
    return fail(NX_ERR_DEVICE, std::string("launch ") + name + ": " + hipGetErrorString(e));
  }
  return end_launch(c, si);
}

// ---- launchers implemented in the kernel files ----
int launch_dequant(nx_ctx *c, int fmt, const void *d_src, size_t n, float *d_dst);
int launch_quantize(nx_ctx *c, int fmt, const float *d_src, size_t n, void *d_dst);
int launch_repack(nx_ctx *c, int fmt, const void *d_src, const RolePlane &pl, uint8_t *qs,
                  uint8_t *meta);

int launch_route(nx_ctx *c, const float *d_logits, int T, int E, int k, int score_mode,
                 int32_t *d_expert, float *d_weight, int32_t *d_count);
// d_tiles (optional): [0] = tile count, then (expert, first pair) per tile
// of tile_m pairs; shared_T > 0 appends ceil(shared_T / tile_m) tiles of the
// shared expert (expert id E)
int launch_permute(nx_ctx *c, const int32_t *d_expert, const int32_t *d_count, int T, int k,
                   int E, int tile_m, int32_t *d_ecount, int32_t *d_offsets, int32_t *d_ptok,
                   int32_t *d_pslot, int32_t *d_inv, int32_t *d_active, int32_t *d_tiles,
                   int shared_T, int tile_m2 = 0, int32_t *d_tiles2 = nullptr);
// router + permutation in one workgroup, for small batches; d_tiles
// (optional) as for launch_permute, without shared-expert tiles
bool route_permute_fusable(int T, int E, int k);
int launch_route_permute(nx_ctx *c, const float *d_logits, int T, int E, int k, int score_mode,
                         int32_t *d_expert, float *d_weight, int32_t *d_count, int32_t *d_ecount,
                         int32_t *d_offsets, int32_t *d_ptok, int32_t *d_pslot, int32_t *d_inv,
                         int32_t *d_active, int tile_m, int32_t *d_tiles, int *d_counters,
                         int n_counters);
// logits[t][e] = sum_c w[e][c] x[t][c]; exact: the reference's sequential
// order with separately rounded products and sums
int launch_router_logits(nx_ctx *c, const float *d_w, const float *d_x, int T, int E, int H,
                         bool exact, float *d_out);
// per-row sequential sum of squares (rms_norm's variance sum, bit-exact)
int launch_sumsq_exact(nx_ctx *c, const float *d_x, int T, int H, float *d_out);
// exact RMSNorm + router logits of T tokens in one launch (block prologue);
// block_prologue_fits: the row shape and alignment it takes
int launch_block_prologue(nx_ctx *c, const float *d_x, const float *d_nw, float eps,
                          const float *d_w, int T, int E, int H, float *d_xn, float *d_logits);
bool block_prologue_fits(int H, const void *x, const void *nw, const void *w, const void *xn);
// exact RMSNorm in one launch for rows of whole float4 up to 7168
bool rms_runs_fit(int H, const void *x, const void *w, const void *out);
int launch_rms_exact_runs(nx_ctx *c, const float *d_x, const float *d_w, float eps, int T, int H,
                          float *d_out);
int launch_rms_apply(nx_ctx *c, const float *d_x, const float *d_sumsq, const float *d_w,
                     float eps, int T, int H, float *d_out);
int launch_rms_fast(nx_ctx *c, const float *d_x, const float *d_w, float eps, int T, int H,
                    float *d_out);
// out[t] = sum_r w[t,r] * y[pair(t,r)] (+ y[shared row t]); y is the sum of
// nsplit partial buffers split_stride floats apart; with a residual,
// out = residual + that sum (out may be the residual itself).  d_inv null:
// the routed rows are stored in route order (pair(t,r) = t * k + r)
int launch_combine(nx_ctx *c, const float *d_ypair, const float *d_weight, const int32_t *d_count,
                   const int32_t *d_inv, int T, int k, int H, bool shared, float *d_out,
                   int nsplit = 1, size_t split_stride = 0, const float *d_residual = nullptr);
// the same, over bf16 per-pair rows (the bf16 grouped GEMM's down pass)
int launch_combine_bf16(nx_ctx *c, const uint16_t *d_ypair, const float *d_weight,
                        const int32_t *d_count, const int32_t *d_inv, int T, int k, int H,
                        bool shared, float *d_out, int nsplit, size_t split_stride,
                        const float *d_residual);

struct GemvPlan {
  const nx_experts *ex;
  int T, k;
  const float *x;            // [T][H]
  const int32_t *perm_token;  // [pairs]
  const int32_t *offsets;     // [E+1]
  const int32_t *active;      // [E] ids then n_active at [E]
  float *act;                 // [pairs_total][act_stride]
  int act_stride;
  float *ypair;               // [pairs_total][H]
  // combine inputs for the down projection
  const float *rw;
  const int32_t *rcnt;
  const int32_t *inv;
  float *out;
  const float *residual = nullptr;  // out = residual + layer output when set
  // pair -> route slot t * k + r ([T * k]); with one token the down pass
  // writes each routed pair's rows at its route slot, so the combine looks
  // up no pair indices
  const int32_t *pslot = nullptr;
  // One token routed inside the gate/up kernel from logits [E] (E at most
  // kFusedRouteMaxE), which also writes the arrays the router and
  // permutation kernels would (expert, weight, count, ecount, offsets,
  // perm_token, perm_slot, inv, active); perm_token, offsets and active
  // above then point at those same arrays for the down pass.
  struct FusedRoute {
    const float *logits = nullptr;
    int score_mode = 0;
    int32_t *exp = nullptr, *cnt = nullptr, *ecount = nullptr, *off = nullptr, *ptok = nullptr,
            *pslot = nullptr, *inv = nullptr, *active = nullptr;
    float *w = nullptr;
  } route;
};
constexpr int kFusedRouteMaxE = 256;
int launch_gemv_gateup(nx_ctx *c, const GemvPlan &p);
// out[t][r] = sum_c W[r][c] x[t][c] for one resident matrix (x rows pl.cols
// floats apart, out rows pl.rows floats apart)
int launch_gemv_matrix(nx_ctx *c, int fmt, const RolePlane &pl, const float *x, int T, float *out);
// whether a row of nseg segments fits the register-resident GEMV
bool gemv_row_fits(int fmt, int nseg);
int launch_gemv_down(nx_ctx *c, const GemvPlan &p);

struct GemmPlan {
  const nx_experts *ex;
  int T, k;
  bool bf16;
  const float *x;
  const int32_t *perm_token;
  const int32_t *offsets;
  const int32_t *active;
  const int32_t *tiles;  // tile list from the permutation kernel (gate/up M-tiles)
  int max_tiles;         // grid bound for the tile list
  int tile_m;            // gate/up M-tile height
  const int32_t *tiles_down;  // the down pass's tile list (its own M-tile height)
  int max_tiles_down;
  int tile_m_down;
  void *act;             // [pairs_total][act_stride] half precision
  int act_stride;
  float *ypair;
  bool ypair_bf16;       // ypair holds bf16 partial sums (uint16_t elements)
  void *xh;              // [T][x_stride] half precision copy of x, operand order
  int x_stride;
  size_t pairs_total;    // rows of act / ypair
  int ksplit;            // down pass K splits (ypair holds ksplit partial sums)
};
// the layer forward behind nx_moe_forward_dev; d_residual (optional) is added
// to the output in the combine (d_out may equal d_residual)
int moe_forward(nx_ctx *c, const nx_experts *ex, const float *d_x, const float *d_logits, int T,
                int k, int score_mode, int path, float *d_out, const float *d_residual);
// few-token grouped matvec on MFMA (Q4_K): gate/up over K slices, SwiGLU of
// the summed slices, down over K slices, then the combine (summing the down
// slices in order) into out (+ residual)
struct MfvPlan {
  const nx_experts *ex;
  int T, k;
  const float *x;             // [T][H], 16-byte aligned
  const int32_t *perm_token;  // [pairs]
  const int32_t *offsets;     // [E+1]
  const int32_t *tiles;       // tile list of the permutation with tile_m = kMfvTileM
  int max_tiles;              // grid bound for the tile list
  const float *rw;            // combine inputs
  const int32_t *rcnt;
  const int32_t *inv;
  float *out;
  const float *residual;
};
int launch_mfv(nx_ctx *c, const MfvPlan &p);
// whether the split-activation path takes these experts: Q4_K, or Q4_0
// with hidden and FFN widths that are multiples of 256
bool mfv_supports(const nx_experts *ex);
int mfv_max_tiles(int T, int k, int E, bool shared);
constexpr int kMfvTileM = 16;
// grouped-GEMM M-tile height of a pass for a batch
int gemm_tile_m(int fmt, bool gateup, int T, int k, int E);
int gemm_wg_per_cu(int fmt, int tile_m);
int gemm_down_ksplit(int fmt, int F, int H, int tiles, int slots);
// width of a row of GEMM operands (operand order pads to whole scale windows)
int gemm_kpad(int fmt, int cols);
int launch_to_half(nx_ctx *c, int fmt, const float *x, int T, int H, int kpad, bool bf16, void *out);
int launch_gemm_gateup(nx_ctx *c, const GemmPlan &p);
int launch_gemm_down(nx_ctx *c, const GemmPlan &p);

}  // namespace nx
