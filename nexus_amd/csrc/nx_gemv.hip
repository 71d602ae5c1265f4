// nx_gemv.hip — decode path: fused dequant-in-register GEMV over the resident
// quantized experts, fp32 accumulate.
//
// Replaces the three InferenceEngine::matvec calls, the SwiGLU and the
// weighted accumulate of dispatch_moe_ffn (src/engine/mod.rs:994-1021,
// 775-801) for the tokens routed to each expert.
//
// A row group of L = LPR * KSPLIT lanes owns a run of rows.  Lane i of the
// group owns segments i, i+L, ... of every row (see nx_device.hpp), so the
// activations it needs are loaded into registers once per token group and
// reused for all rows.  Rows are processed U at a time in a two-stage
// software pipeline: the code and scale loads of the next U rows are issued
// before the current U rows are decoded and reduced (DPP adds within a
// wave's row group).
//
// Gate/up (k_gemv_gateup): one workgroup per (expert slot, row block) on a
// one-dimensional grid (slot = the i-th active expert from the permutation,
// then one slot for the shared expert); the epilogue applies SwiGLU and
// stores the activation row of each pair.
//
// Down + combine (k_gemv_down): grid x = row blocks only.  Each half of a
// 512-thread workgroup walks every (slot, token group, row stage) of its
// slots over the workgroup's rows as one continuous pipeline, so the weight
// stream does not drain between experts.  Each wave
// leaves its per-row partial sums in LDS (or, for very many pairs, in a
// global scratch area private to the workgroup); after one barrier the
// workgroup forms out[t] = sum_r w[t,r] * y[pair(t,r)] (+ shared) for its
// rows in route order — the reference's accumulation order, with no atomics
// and no communication between workgroups.
//
// Down rows longer than 64 segments (Mixtral's F = 14336: 224) take the
// per-slot kernel in K slices instead: one wave per (row, slice of 64
// segments), one workgroup per (slot, slice, row block), the slot's
// activations prepared once per workgroup into LDS; the slices' partial sums go to the route-order combine
// kernel, which adds them in slice order.  Weight codes are loaded with the
// non-temporal policy: they are read once, and the activation, scale and
// route arrays that every workgroup rereads stay in the caches.
#include <map>
#include <mutex>
#include <utility>

#include "nx_device.hpp"
#include "nx_internal.hpp"
#include "nx_route_dev.hpp"

// Pipeline depths (stages; S - 1 in flight while one is decoded) of the
// per-slot kernel: two-matrix gate/up rows and one-matrix (down) rows.
#ifndef NX_GEMV_GATEUP_STAGES
#define NX_GEMV_GATEUP_STAGES 2
#endif
#ifndef NX_GEMV_PLAIN_STAGES
#define NX_GEMV_PLAIN_STAGES 2
#endif
// down rows longer than 64 segments split into K slices (per-slot kernel)
#ifndef NX_GEMV_DOWN_SPLIT
#define NX_GEMV_DOWN_SPLIT 1
#endif
// rows per pipeline stage of the one-matrix (down) per-slot kernel
#ifndef NX_GEMV_PLAIN_ROWS
#define NX_GEMV_PLAIN_ROWS 2
#endif
// most slots (active experts + shared) the down pass combines inside its
// workgroups; more go through the per-slot kernel and the combine kernel
#ifndef NX_GEMV_COMBINE_SLOTS
#define NX_GEMV_COMBINE_SLOTS 2
#endif
// cache policy of the weight-code loads (2: non-temporal, streamed past the
// caches so the small activation and route arrays stay resident)
#ifndef NX_GEMV_WEIGHT_CPOL
#define NX_GEMV_WEIGHT_CPOL 2
#endif

namespace nx {

namespace {

struct GemvArgs {
  const uint8_t *qs0, *qs1, *meta0, *meta1;  // role bases (gate, up) or (down, -)
  size_t qs_stride, meta_stride;             // per expert
  uint32_t row_qs, row_meta;                 // bytes per row
  const uint8_t *sqs0, *sqs1, *smeta0, *smeta1;
  uint32_t srow_qs, srow_meta;
  int rows, cols, nseg;
  int srows, scols, snseg;
  const float *x;
  int x_stride;
  const int32_t *perm_token;  // gate/up: pair -> token
  const int32_t *pslot;       // pair -> route slot (one-token down pass)
  const int32_t *offsets;
  const int32_t *active;
  int E, T, k, has_shared;
  float *out;
  int out_stride;
  int rows_per_group;
  // down projection: combine inputs, pair count, global partial-sum area
  const float *rw;
  const int32_t *rcnt;
  const int32_t *inv;
  float *final_out;
  const float *residual;  // final_out = residual + combine when set
  int npairs;
  float *gpart;
  // down rows in K slices (PLAIN, one wave per row): slice s covers segments
  // 64 s .. 64 s + 63 and writes its partial sums kslice_stride floats after
  // slice s - 1's
  int kslices;
  size_t kslice_stride;
  // row blocks per (slot, slice): the per-slot kernel's grid is
  // one-dimensional, workgroup b = (slot * kslices + slice) * kgx + row block
  // (a two-dimensional grid of the same workgroups ran the Mixtral down pass
  // about 1 us slower)
  int kgx;
  // one token (T == 1): slot s < n_active is the s-th active expert and owns
  // pair s, so the expert id and the active count load together and the
  // activation row needs no lookup
  int one_token;
  // gate/up of one token with the routing done in the kernel: every
  // workgroup routes the token from route_logits [E]; workgroup (0, 0) also
  // writes the route and permutation arrays the down pass reads
  const float *route_logits;
  int score_mode;
  int32_t *r_exp, *r_cnt, *r_ecount, *r_off, *r_ptok, *r_pslot, *r_inv, *r_active;
  float *r_w;
};


__device__ __forceinline__ uint4 bload16w(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, NX_GEMV_WEIGHT_CPOL);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// Logical row q of a row group -> matrix row base + q * step, present while
// below end.
struct RowMap {
  int base, step, end;
  __device__ __forceinline__ int row(int q) const { return base + q * step; }
  __device__ __forceinline__ bool valid(int q) const { return base + q * step < end; }
};

// Workgroup-uniform description of one expert slot.
struct SlotView {
  int pair0, count, rows, cols, nseg;
  const uint8_t *q0, *q1, *m0, *m1;
  uint32_t rq, rm;
  bool routed;
};

// active: the active expert list (global, or the workgroup's own routing in
// LDS); null for a dense matrix, one slot over all T tokens.  e_one >= 0: one
// token, slot < n_active is expert e_one (loaded by the caller) with pair slot.
__device__ __forceinline__ SlotView slot_view(const GemvArgs &a, int slot, int n_active,
                                              const int32_t *active, const int32_t *offsets,
                                              int e_one = -1) {
  SlotView v;
  if (slot < n_active) {
    int e = 0;
    v.pair0 = 0;
    v.count = a.T;
    if (e_one >= 0) {
      e = e_one;
      v.pair0 = slot;
      v.count = 1;
    } else if (active) {
      e = active[slot];
      v.pair0 = offsets[e];
      v.count = offsets[e + 1] - v.pair0;
    }
    v.rows = a.rows;
    v.cols = a.cols;
    v.nseg = a.nseg;
    v.q0 = a.qs0 + (size_t)e * a.qs_stride;
    v.q1 = a.qs1 + (size_t)e * a.qs_stride;
    v.m0 = a.meta0 + (size_t)e * a.meta_stride;
    v.m1 = a.meta1 + (size_t)e * a.meta_stride;
    v.rq = a.row_qs;
    v.rm = a.row_meta;
    v.routed = true;
  } else {
    v.pair0 = a.T * a.k;
    v.count = a.T;
    v.rows = a.srows;
    v.cols = a.scols;
    v.nseg = a.snseg;
    v.q0 = a.sqs0;
    v.q1 = a.sqs1;
    v.m0 = a.smeta0;
    v.m1 = a.smeta1;
    v.rq = a.srow_qs;
    v.rm = a.srow_meta;
    v.routed = false;
  }
  // every field is wave-uniform (the slot is); say so, or buffer resources
  // built from them become per-lane values and loads waterfall loops
  auto ufirst = [](auto x) { return __builtin_amdgcn_readfirstlane(x); };
  auto uptr = [](const uint8_t *p) {
    const uint64_t w = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)w);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(w >> 32));
    return reinterpret_cast<const uint8_t *>(((uint64_t)hi << 32) | lo);
  };
  v.pair0 = ufirst(v.pair0);
  v.count = ufirst(v.count);
  v.rows = ufirst(v.rows);
  v.cols = ufirst(v.cols);
  v.nseg = ufirst(v.nseg);
  v.q0 = uptr(v.q0);
  v.q1 = uptr(v.q1);
  v.m0 = uptr(v.m0);
  v.m1 = uptr(v.m1);
  v.rq = ufirst(v.rq);
  v.rm = ufirst(v.rm);
  return v;
}

// Buffer resource for a wave-uniform base and size: both read back through
// readfirstlane, so the resource stays in scalar registers even where the
// compiler lost track of their uniformity (a per-lane resource would turn
// every load into a waterfall loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc_u(const void *base, uint32_t bytes) {
  const uint64_t w = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)w);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(w >> 32));
  return make_rsrc(reinterpret_cast<const void *>(((uint64_t)hi << 32) | lo),
                   __builtin_amdgcn_readfirstlane(bytes));
}

// Register-resident pieces of one row group's work: its segments of a row,
// the activations for NT tokens over those segments, and U rows of codes and
// scales for NMAT matrices.
template <int FMT, int L, int SPL, int NT, int U, int NMAT>
struct RowGroup {
  using S = Seg<FMT>;
  using Meta = typename S::Meta;
  using XS = typename S::X;
  static constexpr int EPS = S::EPS;

  struct Stage {
    uint4 q[U][NMAT][SPL][2];
    Meta m[U][NMAT][SPL];
  };

  int li;      // lane index within the row group
  int seg0;    // first segment of the row group's K slice (0: whole rows)
  XS xv[SPL][NT];  // activations of this lane's segments, per token
  typename S::Run run[NT];  // running integer dot sums, per token

  __device__ __forceinline__ void init(int lane_index, int first_segment = 0) {
    li = lane_index;
    seg0 = first_segment;
#pragma unroll
    for (int t = 0; t < NT; ++t) run_init(run[t]);
  }

  // Issue the loads of logical rows q0 .. q0+U-1 (matrix rows rm.row(q)) of
  // view v; rows at or past rm.end (and absent segments) read as zero.  The
  // planes are in panels of 64 segments (nx_device.hpp).  When a row group
  // spans whole waves (L >= 64) with one segment per lane, a wave's segments
  // are one panel and the rows are wave-uniform: each row gets its own buffer
  // resource at its part of that panel (size 0 past the end), built on the
  // scalar unit, and the lane offsets stay constant.  Otherwise the lanes
  // add their rows' panel offsets to plane-wide resources.
  __device__ __forceinline__ void load(Stage &st, const SlotView &v, int r0, int row_end) const {
    load(st, v, RowMap{0, 1, row_end}, r0);
  }
  __device__ __forceinline__ void load(Stage &st, const SlotView &v, const RowMap &rm,
                                       int q0) const {
    constexpr int CH = code_chunks<FMT>();
    constexpr int CU = 16 * CH;  // code bytes per segment
    uint32_t off0[SPL], off1[SPL], moff[SPL];
#pragma unroll
    for (int m = 0; m < SPL; ++m) {
      const int j = seg0 + li + m * L;
      const bool jv = j < v.nseg;
      off0[m] = jv ? (CH == 1 ? (uint32_t)(j & 63) * 16u : seg_off(j, 0, v.nseg)) : OOB;
      off1[m] = jv ? seg_off(j, 1, v.nseg) : OOB;
      moff[m] = S::meta_off(j, jv);
    }
    if constexpr (L >= 64 && SPL == 1) {
      // the row is wave-uniform: say so, or the resources below become
      // per-lane values and every load a waterfall loop
      const RowMap m{__builtin_amdgcn_readfirstlane(rm.base), __builtin_amdgcn_readfirstlane(rm.step),
                     __builtin_amdgcn_readfirstlane(rm.end)};
      const int q0u = __builtin_amdgcn_readfirstlane(q0);
      // the wave's panel (seg0 and L are whole groups of 64)
      const int g = __builtin_amdgcn_readfirstlane((seg0 + li) >> 6);
      const uint32_t pq = panel_row_bytes(v.nseg, CU), pm = panel_row_bytes(v.nseg, S::MU);
      const uint8_t *bq0 = v.q0 + (size_t)g * v.rows * pq;
      const uint8_t *bq1 = v.q1 + (size_t)g * v.rows * pq;
      const uint8_t *bm0 = v.m0 + (size_t)g * v.rows * pm;
      const uint8_t *bm1 = v.m1 + (size_t)g * v.rows * pm;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int r = m.row(q0u + u);
        const bool rv = r < m.end;
        const uint32_t nq = rv ? pq : 0u, nm = rv ? pm : 0u;
        const __amdgpu_buffer_rsrc_t rq0 = make_rsrc_u(bq0 + (size_t)r * pq, nq);
        const __amdgpu_buffer_rsrc_t rq1 = make_rsrc_u(bq1 + (size_t)r * pq, nq);
        const __amdgpu_buffer_rsrc_t rm0 = make_rsrc_u(bm0 + (size_t)r * pm, nm);
        const __amdgpu_buffer_rsrc_t rm1 = make_rsrc_u(bm1 + (size_t)r * pm, nm);
#pragma unroll
        for (int mt = 0; mt < NMAT; ++mt) {
          st.q[u][mt][0][0] = bload16w(mt == 0 ? rq0 : rq1, off0[0]);
          st.q[u][mt][0][1] = CH == 2 ? bload16w(mt == 0 ? rq0 : rq1, off1[0]) : make_uint4(0, 0, 0, 0);
          st.m[u][mt][0] = S::load_meta(mt == 0 ? rm0 : rm1, moff[0]);
        }
      }
    } else {
      const __amdgpu_buffer_rsrc_t rq0 = make_rsrc_u(v.q0, (uint32_t)v.rows * v.rq);
      const __amdgpu_buffer_rsrc_t rq1 = make_rsrc_u(v.q1, (uint32_t)v.rows * v.rq);
      const __amdgpu_buffer_rsrc_t rm0 = make_rsrc_u(v.m0, (uint32_t)v.rows * v.rm);
      const __amdgpu_buffer_rsrc_t rm1 = make_rsrc_u(v.m1, (uint32_t)v.rows * v.rm);
      // each segment index m's panel, wave-uniform (rows of one panel below
      // 64 lanes; one panel per m from 64), and the panel row bytes
      const uint32_t prq = panel_row_bytes(v.nseg, CU), prm = panel_row_bytes(v.nseg, S::MU);
      uint32_t pbq[SPL], pbm[SPL];
#pragma unroll
      for (int m = 0; m < SPL; ++m) {
        const int g = __builtin_amdgcn_readfirstlane((seg0 + li + m * L) >> 6);
        pbq[m] = panel_row_off(0, g, v.rows, v.nseg, CU);
        pbm[m] = panel_row_off(0, g, v.rows, v.nseg, S::MU);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int r = rm.row(q0 + u);
        const bool rv = r < rm.end;
#pragma unroll
        for (int m = 0; m < SPL; ++m) {
          const uint32_t rqo = rv ? pbq[m] + (uint32_t)r * prq : OOB;
          const uint32_t rmo = rv ? pbm[m] + (uint32_t)r * prm : OOB;
#pragma unroll
          for (int mt = 0; mt < NMAT; ++mt) {
            st.q[u][mt][m][0] = bload16w(mt == 0 ? rq0 : rq1, rqo + off0[m]);
            st.q[u][mt][m][1] =
                CH == 2 ? bload16w(mt == 0 ? rq0 : rq1, rqo + off1[m]) : make_uint4(0, 0, 0, 0);
            st.m[u][mt][m] = S::load_meta(mt == 0 ? rm0 : rm1, rmo + moff[m]);
          }
        }
      }
    }
  }

  // Activations of tokens t0 .. t0+NT-1 of view v over this lane's segments.
  // row_of(t) gives the row of the activation matrix for token t of the slot;
  // one buffer resource per row, sized to the row, so columns past the row
  // (padding, absent segments) and absent tokens read as zero.
  // Raw activations of this lane's segments for one token group: loaded by
  // load_x_issue, converted into the operands by load_x_prep.  Between the
  // two, loads issued later (weights) stay in flight while the conversion
  // waits only for the activations, which went out first.
  using XRaw = float[SPL][NT][EPS];
  template <class RowOf>
  __device__ __forceinline__ void load_x_issue(XRaw &x, const float *xbase, int xstride,
                                               const SlotView &v, int t0, RowOf row_of) const {
    // the token group is wave-uniform (see slot_view)
    const int t0u = __builtin_amdgcn_readfirstlane(t0);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const bool tv = t0u + t < v.count;
      const float *xrow = xbase;
      if (tv) xrow = xbase + (size_t)__builtin_amdgcn_readfirstlane(row_of(t0u + t)) * xstride;
      const __amdgpu_buffer_rsrc_t xr = make_rsrc_u(xrow, tv ? (uint32_t)v.cols * 4u : 0u);
#pragma unroll
      for (int m = 0; m < SPL; ++m) {
        const int j = seg0 + li + m * L;
        const bool jv = j < v.nseg;
#pragma unroll
        for (int e = 0; e < EPS; e += 4) {
          const uint32_t xo = jv ? (uint32_t)S::xidx(j, e) * 4u : OOB;
          if constexpr (FMT == NX_FMT_F32 || FMT == NX_FMT_F16 || FMT == NX_FMT_BF16) {
            // rows of any length: element-wise so that each load is wholly in or out
#pragma unroll
            for (int i = 0; i < 4; ++i) x[m][t][e + i] = __uint_as_float(bload4(xr, xo + 4u * i));
          } else {
            const uint4 f = bload16(xr, xo);
            x[m][t][e] = __uint_as_float(f.x);
            x[m][t][e + 1] = __uint_as_float(f.y);
            x[m][t][e + 2] = __uint_as_float(f.z);
            x[m][t][e + 3] = __uint_as_float(f.w);
          }
        }
      }
    }
  }
  __device__ __forceinline__ void load_x_prep(const XRaw &x) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int m = 0; m < SPL; ++m) S::prep(x[m][t], xv[m][t]);
  }
  // one buffer resource per row, sized to the row, so columns past the row
  // (padding, absent segments) and absent tokens read as zero.
  template <class RowOf>
  __device__ __forceinline__ void load_x(const float *xbase, int xstride, const SlotView &v, int t0,
                                         RowOf row_of) {
    XRaw x;
    load_x_issue(x, xbase, xstride, v, t0, row_of);
    load_x_prep(x);
  }

  // Workgroup-cooperative activations, for row groups of one whole wave
  // (L == 64, SPL == 1): every wave of the workgroup owns the same 64
  // segments, so the workgroup builds each segment's operand once in LDS.
  // Thread tid loads quarter tid%4 of segment tid/4 (coop_issue, before the
  // weight loads so that its loads are not queued behind them), then the
  // quads build the operands (coop_finish) and every lane copies its own.
  static constexpr int XQ = EPS / 4;                        // values per quarter
  static constexpr int XW = (int)((sizeof(XS) + 15) / 16);  // 16-byte words per operand

  template <class RowOf>
  __device__ __forceinline__ void coop_issue(float (&xq)[NT][XQ], const float *xbase, int xstride,
                                             const SlotView &v, int t0, RowOf row_of,
                                             int tid) const {
    const int sgm = seg0 + (tid >> 2), q = tid & 3;
    const bool jv = sgm < v.nseg;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const bool tv = t0 + t < v.count;
      const float *xrow = xbase;
      if (tv) xrow = xbase + (size_t)row_of(t0 + t) * xstride;
      const __amdgpu_buffer_rsrc_t xr = make_rsrc_u(xrow, tv ? (uint32_t)v.cols * 4u : 0u);
#pragma unroll
      for (int e = 0; e < XQ; e += 4) {
        const uint4 f = bload16(xr, jv ? (uint32_t)S::xidx(sgm, q * XQ + e) * 4u : OOB);
        xq[t][e] = __uint_as_float(f.x);
        xq[t][e + 1] = __uint_as_float(f.y);
        xq[t][e + 2] = __uint_as_float(f.z);
        xq[t][e + 3] = __uint_as_float(f.w);
      }
    }
  }
  __device__ __forceinline__ void coop_finish(const float (&xq)[NT][XQ], uint4 *xsh, int tid) {
    const int sgm = tid >> 2, q = tid & 3;
    __syncthreads();  // the previous token group's operands have been copied
#pragma unroll
    for (int t = 0; t < NT; ++t)
      S::prep_quarter(xq[t], q, reinterpret_cast<XS *>(xsh + (t * 64 + sgm) * XW));
    __syncthreads();
#pragma unroll
    for (int t = 0; t < NT; ++t) xv[0][t] = *reinterpret_cast<const XS *>(xsh + (t * 64 + li) * XW);
  }

  // Dot products of the staged rows with the activations, summed over the
  // row group's LPR lanes (the total lands in the group's last lane).
  template <int LPR>
  __device__ __forceinline__ void compute(const Stage &st, float (&acc)[U][NMAT][NT]) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[u][mt][t] = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
        for (int m = 0; m < SPL; ++m) {
          S::template dot<NT>(st.q[u][mt][m][0], st.q[u][mt][m][1], st.m[u][mt][m],
                              seg0 + li + m * L, xv[m], run, acc[u][mt]);
          // keep each segment's decode local: without this the scheduler
          // hoists the work of the whole stage and runs out of registers
          __builtin_amdgcn_sched_barrier(0);
        }
    group_sum_n<LPR, U * NMAT * NT>(&acc[0][0][0]);
  }
};

// Wave 0 of a gate/up workgroup routes the launch's one token (route_select:
// top-k with ties to the lower index) from the logits route_load gave, and
// finds what the permutation kernel would give it: the routed experts sorted
// by id are the active list, each owning one pair at its rank.  Every
// workgroup needs only the active list (s_active, s_n in LDS).  Workgroup 0
// also writes the arrays the later kernels and the route query read, with
// the values k_route_permute gives one token.
template <int EPL>
__device__ __forceinline__ void fused_route(const GemvArgs &a, int lane,
                                            const float (&lv)[kFusedRouteMaxE / 64],
                                            int32_t *s_active, int32_t *s_n) {
  // only the workgroup that writes the routes needs their weights
  const bool writer = blockIdx.x == 0;
  int e, n;
  float w;
  route_select<EPL>(lv, a.E, a.k, a.score_mode, lane, &e, &w, &n, writer);
  // this route's rank among the routed experts in ascending id order (n is
  // wave-uniform, so every lane takes part in each read)
  int rank = 0;
  for (int r = 0; r < n; ++r) rank += __builtin_amdgcn_readlane(e, r) < e ? 1 : 0;
  if (lane < n) s_active[rank] = e;
  if (lane == 0) *s_n = n;
  if (!writer) return;
  if (lane < n) {
    a.r_active[rank] = e;
    a.r_ptok[rank] = 0;
    a.r_pslot[rank] = lane;
  }
  if (lane < a.k) {
    a.r_exp[lane] = e;
    a.r_w[lane] = w;
    a.r_inv[lane] = lane < n ? rank : -1;
  }
  if (lane == 0) {
    a.r_cnt[0] = n;
    a.r_active[a.E] = n;
  }
  // per expert x <= E: the routed experts below x (its offset) and at x
  for (int x = lane; x <= a.E; x += 64) {
    int below = 0, hit = 0;
    for (int r = 0; r < n; ++r) {
      const int er = __builtin_amdgcn_readlane(e, r);
      below += er < x ? 1 : 0;
      hit += er == x ? 1 : 0;
    }
    a.r_off[x] = below;
    if (x < a.E) a.r_ecount[x] = hit;
  }
}

// PLAIN: one matrix (the down projection of one slot per workgroup), no
// SwiGLU; activations are per pair (row pair0 + t of x) and each row's dot
// product goes to out[pair][row] for the combine kernel.
template <int FMT, int LPR, int KSPLIT, int SPL, int NT, bool PLAIN = false>
__global__ __launch_bounds__(256, 2) void k_gemv_gateup(const GemvArgs a) {
  constexpr int L = LPR * KSPLIT;
  constexpr int GROUPS = 256 / L;
  constexpr int NMAT = PLAIN ? 1 : 2;
  // rows per pipeline stage: one matrix leaves the registers for twice the
  // rows; two tokens' activations in registers (no shared LDS operands, or
  // two segments per lane) leave room for one row per stage (two rows
  // spilled, and one is faster: Qwen3 gate/up at 2 tokens 20.5 -> 16.4 us)
  constexpr int U = PLAIN && SPL == 1 && L == 64 ? NX_GEMV_PLAIN_ROWS
                    : (!PLAIN && NT == 2 && (L < 64 || SPL == 2)) ? 1
                                                                  : 2;
  // stages (S - 1 of them in flight while one is decoded)
  constexpr int S = PLAIN ? NX_GEMV_PLAIN_STAGES : (NT == 1 && SPL == 1 ? NX_GEMV_GATEUP_STAGES : 2);
  using RG = RowGroup<FMT, L, SPL, NT, U, NMAT>;
  const int tid = threadIdx.x, lane = tid & 63;
  // wave index, known to the compiler as wave-uniform
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // row group of this thread; with KSPLIT > 1, waves grp KSPLIT ..
  // grp KSPLIT + KSPLIT - 1 share its rows, each over its own segments
  const int grp = KSPLIT > 1 ? wave / KSPLIT : (LPR == 64 ? wave : tid / LPR);

  // one wave per row group: the workgroup shares the activation operands
  constexpr bool COOP = L == 64 && SPL == 1 && FMT != NX_FMT_F32 && FMT != NX_FMT_F16 &&
                        FMT != NX_FMT_BF16;
  __shared__ uint4 xsh[COOP ? NT * 64 * RG::XW : 1];
  // slot, K slice (PLAIN with kslices > 1; else whole rows) and row block:
  // workgroup = (slot, slice, row block)
  const int kslices = PLAIN ? a.kslices : 1;
  const int sk = (int)blockIdx.x / a.kgx;
  const int bx = (int)blockIdx.x - sk * a.kgx;
  const int slot = sk / kslices;
  const int kslice = sk - slot * kslices;
  const int rpg = a.rows_per_group;
  RG g;
  g.init(KSPLIT == 1 ? (lane % LPR) : tid % L, kslice * L * SPL);
  float xq[NT][RG::XQ];  // activation quarters in flight (COOP)
  bool x_issued = false;  // set only by the in-kernel routing (NT == 1)

  const int32_t *active = a.active, *offsets = a.offsets, *perm_token = a.perm_token;
  int n_active;
  // one token: this slot's expert, loaded together with the active count
  // (slot <= E, so the load is in range even for an absent slot), and for
  // the down pass the route slot its rows are written at (clamped to the
  // T * k = k route slots; only a routed slot uses it)
  int e_one = -1, ps_one = 0;
  if constexpr (!PLAIN && NT == 1) {
    // one token routed here: ids of the routed experts in ascending order
    // (the permutation's active list), each with one pair at its rank
    __shared__ int32_t s_active[64];
    __shared__ int32_t s_n;
    if (a.route_logits) {  // kernel-uniform
      // the logits go out first: loads complete in issue order, so the
      // routing then waits for them alone, not for the activations too
      float lv[kFusedRouteMaxE / 64];
      if (wave == 0) route_load(a.route_logits, a.E, lane, lv);
      if constexpr (COOP) {
        // every slot of the one token reads activation row 0 over rows of
        // a.cols (gate/up and the shared expert alike): load it while the
        // token is routed
        SlotView v0;
        v0.count = 1;
        v0.cols = a.cols;
        v0.nseg = a.nseg;
        g.coop_issue(xq, a.x, a.x_stride, v0, 0, [](int) { return 0; }, tid);
        x_issued = true;
      }
      if (wave == 0) {  // as few keys per lane as the experts need
        if (a.E <= 64)
          fused_route<1>(a, lane, lv, s_active, &s_n);
        else if (a.E <= 128)
          fused_route<2>(a, lane, lv, s_active, &s_n);
        else
          fused_route<4>(a, lane, lv, s_active, &s_n);
      }
      __syncthreads();
      n_active = s_n;
      // this slot's expert (one pair, at the slot's rank)
      if (slot < n_active) e_one = s_active[slot];
    } else {
      if (a.one_token) e_one = a.active[min(slot, a.E)];
      n_active = a.active[a.E];
    }
  } else {
    // (in-kernel routing takes one token, which runs the NT == 1 instances)
    if (a.one_token) {
      e_one = a.active[min(slot, a.E)];
      if (PLAIN && a.pslot) ps_one = a.pslot[min(slot, a.k - 1)];
    }
    n_active = a.active ? a.active[a.E] : 1;
  }
  const int n_slots = n_active + (a.has_shared ? 1 : 0);
  if (slot >= n_slots) return;  // workgroup-uniform
  float *const out = a.out + (size_t)kslice * a.kslice_stride;
  // first output row of the slot: its pair, or (one-token down pass) the
  // routed pair's route slot
  const int orow0 = (PLAIN && e_one >= 0 && a.pslot && slot < n_active) ? ps_one : -1;
  // KSPLIT > 1: per-wave partial sums of up to RED_ROWS rows, summed across
  // the group's waves once per RED_ROWS rows (two barriers), not per stage
  constexpr int RED_ROWS = 32;
  static_assert(RED_ROWS % U == 0, "a stage's rows share one run of partials");
  __shared__ float red[KSPLIT > 1 ? 4 * RED_ROWS * NMAT * NT : 1];

  const SlotView v = slot_view(a, slot, n_active, active, offsets, e_one);
  // this group's logical rows 0 .. nq-1: the workgroup owns one contiguous
  // run of GROUPS * rpg rows, and its row groups take every GROUPS-th row of
  // it (row = run start + q * GROUPS + group), so that at each stage the
  // waves read neighbouring rows
  const int wg0 = bx * GROUPS * rpg;
  const RowMap rm{wg0 + grp, GROUPS, min(v.rows, wg0 + GROUPS * rpg)};
  const int nq = rm.end > rm.base ? (rm.end - rm.base + GROUPS - 1) / GROUPS : 0;
  // activation row of token t of the slot (one token: row 0, no lookup)
  auto row_of = [&](int t) {
    return PLAIN ? v.pair0 + t
                 : (v.routed && e_one < 0 ? perm_token[v.pair0 + t] : (e_one >= 0 ? 0 : t));
  };

  // with KSPLIT > 1 finish has barriers, so the stage sequence must be
  // workgroup-uniform: one row group per workgroup runs its nq rows; with
  // several, every group runs rows_per_group rows (rows past the end load as
  // zeros and are not written)
  const int qlim = (KSPLIT > 1 && GROUPS > 1) ? rpg : nq;

  typename RG::Stage st[S];
  for (int t0 = 0; t0 < v.count; t0 += NT) {
    if constexpr (COOP) {
      if (!x_issued) g.coop_issue(xq, a.x, a.x_stride, v, t0, row_of, tid);
      x_issued = false;
#pragma unroll
      for (int i = 0; i < S - 1; ++i) g.load(st[i], v, rm, i * U);
      g.coop_finish(xq, xsh, tid);
    } else if constexpr (!PLAIN) {
      // the activations go out first, then the weight stages: loads
      // complete in issue order, so the conversion waits only for the
      // activations while the weights stay in flight (Qwen3 one-token
      // gate/up 12.1 -> 11.3 us)
      typename RG::XRaw xr;
      g.load_x_issue(xr, a.x, a.x_stride, v, t0, row_of);
#pragma unroll
      for (int i = 0; i < S - 1; ++i) g.load(st[i], v, rm, i * U);
      g.load_x_prep(xr);
    } else {
      // down: the weight stages first (activations first measured slower
      // here: DeepSeek one-token down 17.9 -> 18.5 us)
#pragma unroll
      for (int i = 0; i < S - 1; ++i) g.load(st[i], v, rm, i * U);
      g.load_x(a.x, a.x_stride, v, t0, row_of);
    }

    auto finish = [&](const typename RG::Stage &st, int q0) {
      float acc[U][NMAT][NT];
      g.template compute<LPR>(st, acc);
      const bool writer = (g.li % LPR) == LPR - 1;
      if constexpr (KSPLIT > 1) {
        // the wave's partials of rows q0 .. q0 + U - 1 (lane 63 holds them)
        const int sr = q0 % RED_ROWS;
        if (lane == 63) {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
              for (int t = 0; t < NT; ++t)
                red[((wave * RED_ROWS + sr + u) * NMAT + mt) * NT + t] = acc[u][mt][t];
        }
        // a full run of partials, or the group's last stage (both
        // workgroup-uniform: every group runs the same stage sequence)
        if (sr + U == RED_ROWS || q0 + U >= qlim) {
          __syncthreads();
          const int qb = q0 + U - (sr + U);  // first row of the run
          for (int i = tid % L; i < (sr + U) * NT; i += L) {
            const int rl = i / NT, t = i - rl * NT;
            if (!rm.valid(qb + rl) || t0 + t >= v.count) continue;
            const int r = rm.row(qb + rl);
            float sm[NMAT];
#pragma unroll
            for (int mt = 0; mt < NMAT; ++mt) {
              float s = 0.f;
#pragma unroll
              for (int w = 0; w < KSPLIT; ++w)
                s += red[(((grp * KSPLIT + w) * RED_ROWS + rl) * NMAT + mt) * NT + t];
              sm[mt] = s;
            }
            out[(size_t)((orow0 >= 0 ? orow0 : v.pair0) + t0 + t) * a.out_stride + r] =
                PLAIN ? sm[0] : silu_mul(sm[0], sm[NMAT - 1]);
          }
          __syncthreads();
        }
        return;
      }
      if (writer) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (!rm.valid(q0 + u)) continue;
          const int r = rm.row(q0 + u);
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            if (t0 + t >= v.count) continue;
            if constexpr (PLAIN)
              out[(size_t)((orow0 >= 0 ? orow0 : v.pair0) + t0 + t) * a.out_stride + r] = acc[u][0][t];
            else
              out[(size_t)((orow0 >= 0 ? orow0 : v.pair0) + t0 + t) * a.out_stride + r] =
                  silu_mul(acc[u][0][t], acc[u][NMAT - 1][t]);
          }
        }
      }
    };

    for (int q = 0; q < qlim; q += S * U) {
#pragma unroll
      for (int i = 0; i < S; ++i) {
        const int qq = q + i * U;
        if (qq >= qlim) break;
        g.load(st[(i + S - 1) % S], v, rm, qq + (S - 1) * U);
        finish(st[i], qq);
      }
    }
  }
}

// Down projection of every pair over this workgroup's rows, then the combine.
// The workgroup is DOWN_SG halves of 256 threads; half h runs slots h,
// h + DOWN_SG, ... over the same rows, so the experts of a token are
// streamed side by side.  YLDS: partial sums in LDS (dynamic,
// [KSPLIT][npairs][wg_rows]); otherwise in a.gpart at this workgroup's own
// offset.
constexpr int DOWN_SG = 2;

template <int FMT, int LPR, int KSPLIT, int SPL, int NT, bool YLDS>
__global__ __launch_bounds__(256 * DOWN_SG, 1) void k_gemv_down(const GemvArgs a) {
  constexpr int L = LPR * KSPLIT;
  constexpr int GROUPS = 256 / L;
  constexpr int U = 2;  // rows per pipeline stage
  // pipeline stages: three where the registers allow (one segment per lane)
  constexpr int S = (SPL == 1 && L >= 64) ? 3 : 2;
  using RG = RowGroup<FMT, L, SPL, NT, U, 1>;
  extern __shared__ float ypart_lds[];
  const int tid = threadIdx.x, tl = tid & 255, lane = tl & 63;
  // half and wave index, known to the compiler as wave-uniform
  const int half = __builtin_amdgcn_readfirstlane(tid >> 8);
  const int wave = __builtin_amdgcn_readfirstlane(tl >> 6);
  const int grp = KSPLIT > 1 ? wave / KSPLIT : (LPR == 64 ? wave : tl / LPR);
  const int kpart = KSPLIT == 1 ? 0 : wave % KSPLIT;  // which partial this wave leaves

  const int n_active = a.active[a.E];
  const int n_slots = n_active + (a.has_shared ? 1 : 0);
  const int npairs = a.npairs;
  const int wg_rows = GROUPS * a.rows_per_group;
  const int rb0 = blockIdx.x * wg_rows;
  const int nr = min(a.rows, rb0 + wg_rows) - rb0;
  const int row_begin = rb0 + grp * a.rows_per_group;
  const int row_end = min(a.rows, row_begin + a.rows_per_group);
  float *ybuf = YLDS ? ypart_lds : a.gpart + (size_t)blockIdx.x * KSPLIT * npairs * wg_rows;

  RG g;
  g.init(KSPLIT == 1 ? (lane % LPR) : tl % L);
  const bool writer = (g.li % LPR) == LPR - 1;

  // Stage positions: (slot, first token of the group, first row).  The
  // sequence runs over rows fastest, then token groups, then this half's
  // slots.
  struct Pos {
    int si, t0, r;
  };
  auto advance = [&](Pos &p, SlotView &v) {
    p.r += U;
    if (p.r >= row_end) {
      p.r = row_begin;
      p.t0 += NT;
      if (p.t0 >= v.count) {
        p.t0 = 0;
        p.si += DOWN_SG;
        if (p.si < n_slots) v = slot_view(a, p.si, n_active, a.active, a.offsets);
      }
    }
  };
  // what finishing a stage needs of its slot and position
  struct StageInfo {
    int si, t0, r, pair0, count, cols, nseg;
  };
  auto finish = [&](const typename RG::Stage &st, const StageInfo &p) {
    float acc[U][1][NT];
    g.template compute<LPR>(st, acc);
    if (writer) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int r = p.r + u;
        if (r >= row_end) continue;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          if (p.t0 + t >= p.count) continue;
          ybuf[((size_t)kpart * npairs + p.pair0 + p.t0 + t) * wg_rows + (r - rb0)] = acc[u][0][t];
        }
      }
    }
  };

  if (row_begin < row_end && half < n_slots) {  // uniform within the row group
    // S-stage register pipeline over the sequence of (slot, token group,
    // rows) positions: stage i is decoded while the next S - 1 are in flight
    Pos pl{half, 0, row_begin};  // next position to issue
    SlotView vl = slot_view(a, half, n_active, a.active, a.offsets);
    typename RG::Stage st[S];
    StageInfo info[S];
    bool valid[S];
    auto issue = [&](int j) {
      valid[j] = pl.si < n_slots;
      if (valid[j]) {
        info[j] = StageInfo{pl.si, pl.t0, pl.r, vl.pair0, vl.count, vl.cols, vl.nseg};
        g.load(st[j], vl, pl.r, row_end);
        advance(pl, vl);
      }
    };
    // Loads complete in issue order as far as the wait counts go: the first
    // group's activations go out first, then the first weight stages, and
    // only then does the conversion wait (for the activations alone).  Later
    // groups load theirs before the next stage is issued.
    {
      typename RG::XRaw xr;
      g.load_x_issue(xr, a.x, a.x_stride, vl, 0, [&](int t) { return vl.pair0 + t; });
#pragma unroll
      for (int i = 0; i < S - 1; ++i) issue(i);
      g.load_x_prep(xr);
    }
    int xsi = half, xt0 = 0;  // the token group whose activations are prepared
    bool done = false;
    while (!done) {
#pragma unroll
      for (int i = 0; i < S; ++i) {
        if (!valid[i]) {
          done = true;
          break;
        }
        const StageInfo &p = info[i];
        if (p.si != xsi || p.t0 != xt0) {
          SlotView vx;
          vx.pair0 = p.pair0;
          vx.count = p.count;
          vx.cols = p.cols;
          vx.nseg = p.nseg;
          g.load_x(a.x, a.x_stride, vx, p.t0, [&](int t) { return p.pair0 + t; });
          xsi = p.si;
          xt0 = p.t0;
        }
        issue((i + S - 1) % S);
        finish(st[i], p);
      }
    }
  }

  // combine this workgroup's rows: out[t][h] = sum_r w[t,r] * y[pair(t,r)][h]
  // (+ shared), in route order; y = the KSPLIT partials summed in wave order
  __syncthreads();
  const int T = a.T;
  for (int i = tid; i < nr * T; i += 256 * DOWN_SG) {
    const int t = i / nr, hl = i - t * nr;
    auto y = [&](int p) {
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < KSPLIT; ++w) s += ybuf[((size_t)w * npairs + p) * wg_rows + hl];
      return s;
    };
    const int n = a.rcnt[t];
    float acc = 0.0f;
    for (int r = 0; r < n; ++r) {
      const int p = a.inv[(size_t)t * a.k + r];
      acc = acc + __fmul_rn(a.rw[(size_t)t * a.k + r], y(p));
    }
    if (a.has_shared) acc = acc + y(T * a.k + t);
    const size_t o = (size_t)t * a.rows + rb0 + hl;
    a.final_out[o] = a.residual ? a.residual[o] + acc : acc;
  }
}

using KernelFn = void (*)(GemvArgs);

struct Shape {
  int lpr, ksplit, spl;
};

// kernels: gate/up; down with the workgroup-local combine; down rows per
// slot (grid.y), combined afterwards by k_combine
enum GemvKind { KIND_GATEUP, KIND_DOWN_COMBINE, KIND_DOWN_ROWS };

// kernel instance for (format, tokens per group, shape, kind, partials in LDS)
template <int FMT, int NT, int LPR, int KSPLIT, int SPL>
KernelFn inst(int kind, bool ylds) {
  if (kind == KIND_GATEUP) return k_gemv_gateup<FMT, LPR, KSPLIT, SPL, NT>;
  if (kind == KIND_DOWN_ROWS) return k_gemv_gateup<FMT, LPR, KSPLIT, SPL, NT, true>;
  return ylds ? k_gemv_down<FMT, LPR, KSPLIT, SPL, NT, true>
              : k_gemv_down<FMT, LPR, KSPLIT, SPL, NT, false>;
}

template <int FMT, int NT>
KernelFn pick_shape(int gateup, bool ylds, const Shape &s) {
  // two segments per lane exist only where choose_shape allows them
  constexpr bool two = 2 * Seg<FMT>::EPS * NT <= 64;
  if (s.ksplit == 1) {
    if (s.lpr == 16 && s.spl == 1) return inst<FMT, NT, 16, 1, 1>(gateup, ylds);
    if (s.lpr == 32 && s.spl == 1) return inst<FMT, NT, 32, 1, 1>(gateup, ylds);
    if (s.lpr == 64 && s.spl == 1) return inst<FMT, NT, 64, 1, 1>(gateup, ylds);
    if constexpr (two)
      if (s.lpr == 64 && s.spl == 2) return inst<FMT, NT, 64, 1, 2>(gateup, ylds);
  } else if (s.ksplit == 2) {
    if (s.spl == 1) return inst<FMT, NT, 64, 2, 1>(gateup, ylds);
  } else {
    if (s.spl == 1) return inst<FMT, NT, 64, 4, 1>(gateup, ylds);
    if constexpr (two)
      if (s.spl == 2) return inst<FMT, NT, 64, 4, 2>(gateup, ylds);
  }
  return nullptr;
}

template <int FMT>
KernelFn pick_fmt(int gateup, bool ylds, int nt, const Shape &s) {
  return nt == 1 ? pick_shape<FMT, 1>(gateup, ylds, s) : pick_shape<FMT, 2>(gateup, ylds, s);
}

KernelFn pick(int fmt, int gateup, bool ylds, int nt, const Shape &s) {
  switch (fmt) {
  case NX_FMT_Q4_K: return pick_fmt<NX_FMT_Q4_K>(gateup, ylds, nt, s);
  case NX_FMT_Q8_0: return pick_fmt<NX_FMT_Q8_0>(gateup, ylds, nt, s);
  case NX_FMT_Q4_0: return pick_fmt<NX_FMT_Q4_0>(gateup, ylds, nt, s);
  case NX_FMT_Q2_K: return pick_fmt<NX_FMT_Q2_K>(gateup, ylds, nt, s);
  case NX_FMT_F32: return pick_fmt<NX_FMT_F32>(gateup, ylds, nt, s);
  case NX_FMT_F16: return pick_fmt<NX_FMT_F16>(gateup, ylds, nt, s);
  case NX_FMT_BF16: return pick_fmt<NX_FMT_BF16>(gateup, ylds, nt, s);
  }
  return nullptr;
}

int elems_per_segment(int fmt) {
  switch (fmt) {
  case NX_FMT_Q4_K: return 64;
  case NX_FMT_Q8_0: return 32;
  case NX_FMT_Q4_0: return 64;
  case NX_FMT_Q2_K: return 64;
  case NX_FMT_F16:
  case NX_FMT_BF16: return 16;
  default: return 8;
  }
}

// lanes per row / waves per row / segments per lane for a row of nseg segments
bool choose_shape(int nseg, int eps, int nt, Shape *s) {
  // activation registers per lane: two segments per lane only while that
  // stays within 64 registers (the 4-bit formats spill beyond it)
  const int budget = 64;
  if (nseg <= 16) *s = {16, 1, 1};
  else if (nseg <= 32) *s = {32, 1, 1};
  else if (nseg <= 64) *s = {64, 1, 1};
  else if (nseg <= 128 && 2 * eps * nt <= budget) *s = {64, 1, 2};
  else if (nseg <= 128) *s = {64, 2, 1};
  else if (nseg <= 256) *s = {64, 4, 1};
  else if (nseg <= 512 && 2 * eps * nt <= budget) *s = {64, 4, 2};
  else return false;
  return true;
}

// tokens per group (two when there are several, unless a row that long only
// fits one token's activations in registers) and the shape for it
bool choose_tokens_shape(int nseg, int eps, int T, int *nt, Shape *s) {
  if (T > 1 && choose_shape(nseg, eps, 2, s)) {
    *nt = 2;
    return true;
  }
  *nt = 1;
  return choose_shape(nseg, eps, 1, s);
}

// Rows per row group, from rpg up, for which the grid of ceil(rows / (rpg *
// gpw)) x grid_y workgroups fits `cap` resident workgroups (or rpg itself
// when no length does).
long fit_one_round(long rows, long rpg, int gpw, long grid_y, long cap) {
  for (long r = rpg; r <= rows; ++r) {
    if ((rows + r * gpw - 1) / (r * gpw) * grid_y <= cap) return r;
    if ((rows + r * gpw - 1) / (r * gpw) == 1) break;
  }
  return rpg;
}

// Resident workgroups per CU of a kernel at a block size.  The occupancy
// query costs microseconds of host time per call and its answer is fixed per
// kernel, so it is asked once.
int wg_per_cu_of(KernelFn fn, int threads) {
  static std::mutex mu;
  static std::map<std::pair<const void *, int>, int> cache;
  const auto key = std::make_pair(reinterpret_cast<const void *>(fn), threads);
  {
    std::lock_guard<std::mutex> lk(mu);
    const auto it = cache.find(key);
    if (it != cache.end()) return it->second;
  }
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, key.first, threads, 0) != hipSuccess ||
      n < 1) {
    (void)hipGetLastError();
    n = 1;
  }
  std::lock_guard<std::mutex> lk(mu);
  cache[key] = n;
  return n;
}

// partial sums of the down kernel stay in LDS up to this size per workgroup
constexpr size_t kDownLdsMax = 64 * 1024;

// slots a launch may see: active experts (at most E, at most T*k) plus the
// shared expert
int slots_max_of(const nx_experts *ex, const GemvPlan &p) {
  const long routed = std::min<long>(ex->E, (long)p.T * p.k);
  return (int)routed + (ex->Fs > 0 ? 1 : 0);
}

int run_gemv(nx_ctx *c, const GemvPlan &p, bool gateup) {
  const nx_experts *ex = p.ex;
  const RolePlane &R0 = ex->role[gateup ? NX_ROLE_GATE : NX_ROLE_DOWN];
  const RolePlane &R1 = ex->role[gateup ? NX_ROLE_UP : NX_ROLE_DOWN];
  const bool has_shared = ex->Fs > 0;
  const RolePlane &S0 = ex->shared[gateup ? NX_ROLE_GATE : NX_ROLE_DOWN];
  const RolePlane &S1 = ex->shared[gateup ? NX_ROLE_UP : NX_ROLE_DOWN];

  GemvArgs a{};
  a.qs0 = R0.qs;
  a.qs1 = R1.qs;
  a.meta0 = R0.meta;
  a.meta1 = R1.meta;
  a.qs_stride = R0.qs_stride;
  a.meta_stride = R0.meta_stride;
  a.row_qs = R0.row_qs;
  a.row_meta = R0.row_meta;
  a.rows = R0.rows;
  a.cols = R0.cols;
  a.nseg = R0.nseg;
  if (has_shared) {
    a.sqs0 = S0.qs;
    a.sqs1 = S1.qs;
    a.smeta0 = S0.meta;
    a.smeta1 = S1.meta;
    a.srow_qs = S0.row_qs;
    a.srow_meta = S0.row_meta;
    a.srows = S0.rows;
    a.scols = S0.cols;
    a.snseg = S0.nseg;
  }
  a.perm_token = p.perm_token;
  a.pslot = p.T == 1 ? p.pslot : nullptr;
  a.offsets = p.offsets;
  a.active = p.active;
  a.E = ex->E;
  a.T = p.T;
  a.k = p.k;
  a.has_shared = has_shared ? 1 : 0;
  if (gateup) {
    a.x = p.x;
    a.x_stride = ex->H;
    a.out = p.act;
    a.out_stride = p.act_stride;
    if (p.route.logits) {
      if (p.T != 1 || ex->E > kFusedRouteMaxE || p.k > 64)
        return fail(NX_ERR_INVALID_ARG, "in-kernel routing takes one token and at most 256 experts");
      a.route_logits = p.route.logits;
      a.score_mode = p.route.score_mode;
      a.r_exp = p.route.exp;
      a.r_w = p.route.w;
      a.r_cnt = p.route.cnt;
      a.r_ecount = p.route.ecount;
      a.r_off = p.route.off;
      a.r_ptok = p.route.ptok;
      a.r_pslot = p.route.pslot;
      a.r_inv = p.route.inv;
      a.r_active = p.route.active;
    }
  } else {
    a.x = p.act;
    a.x_stride = p.act_stride;
  }

  const int nseg = a.nseg > a.snseg ? a.nseg : a.snseg;
  // Down rows longer than one wave's 64 segments (Mixtral's 14336 columns:
  // 224 segments) are cut into K slices of 64 segments, the code plane's
  // layout groups: one wave per (row, slice), each workgroup on one (slot,
  // slice) so it prepares only that slice's activations, and the combine
  // adds the slices' partial sums in slice order.
  const bool down_split = NX_GEMV_DOWN_SPLIT && !gateup && nseg > 64;
  const int kslices = down_split ? (nseg + 63) / 64 : 1;
  a.kslices = kslices;
  int nt;
  Shape sh;
  if (!choose_tokens_shape(down_split ? 64 : nseg, elems_per_segment(ex->fmt), p.T, &nt, &sh))
    return fail(NX_ERR_UNSUPPORTED, "row length too large for the register-resident GEMV");
  const int L = sh.lpr * sh.ksplit;
  const int groups_per_wg = 256 / L;
  const int slots_max = (ex->E < p.T * p.k ? ex->E : p.T * p.k) + (has_shared ? 1 : 0);
  const int rows = a.rows > a.srows ? a.rows : a.srows;
  // The down pass combines its rows inside the workgroup when there are at
  // most two slots (one token's top-2: the halves of the workgroup run them
  // side by side); beyond that, and for K slices, the slots go to grid.y like
  // gate/up, each writing its rows per pair, and the combine runs as its own
  // kernel.
  const bool down_rows = !gateup && (down_split || slots_max_of(ex, p) > NX_GEMV_COMBINE_SLOTS);
  const int kind = gateup ? KIND_GATEUP : (down_rows ? KIND_DOWN_ROWS : KIND_DOWN_COMBINE);
  const bool per_slot = gateup || down_rows;
  // residency is register-bound (eight waves per CU by launch bounds)
  const int threads = per_slot ? 256 : 256 * DOWN_SG;
  KernelFn probe = pick(ex->fmt, kind, true, nt, sh);
  if (!probe) return fail(NX_ERR_UNSUPPORTED, "no GEMV kernel instance for this shape");
  const int wg_per_cu = wg_per_cu_of(probe, threads);
  // gate/up spreads slots over grid.y; down runs all slots inside each
  // workgroup.  Size the row runs so the launch is one round of resident
  // workgroups with equal work each.
  const long work_rows = per_slot ? (long)rows * slots_max * kslices : (long)rows;
  const long groups = (long)c->num_cu * wg_per_cu * groups_per_wg;
  long rpg = (work_rows + groups - 1) / groups;
  if (rpg < 1) rpg = 1;
  const long grid_y = per_slot ? (long)slots_max * kslices : 1;
  // Q4_K and Q8_0 gate/up rows of one wave each (no cross-wave sums): twice
  // the rows per group, half the workgroups, while those still cover every
  // CU.  Measured, one token (us per layer step): Mixtral Q4_K 40.7 -> 40.4,
  // Q8_0 68.5 -> 66.9; Qwen3 and DeepSeek unchanged; Q4_0 40.1 -> 43.1 and
  // Q2_K 37.6 -> 41.4, so not those; the same for the down passes: Qwen3
  // 20.8 -> 19.8 but DeepSeek 53.4 -> 54.8, Q4_0 and Q2_K 3-4 us slower.
  // Q4_K down rows of at most 16 lanes (Qwen3's 768-wide experts) or in K
  // slices (Mixtral's 14336) take the longer runs too (one token: Qwen3
  // 20.7 -> 19.7 us, Mixtral 40.4 -> 39.9 us; DeepSeek, Q8_0 unchanged).
  const bool longer =
      sh.ksplit == 1 &&
      (gateup ? (ex->fmt == NX_FMT_Q4_K || ex->fmt == NX_FMT_Q8_0)
              : (ex->fmt == NX_FMT_Q4_K && (sh.lpr <= 16 || kslices > 1)));
  if (longer) {
    const long rpw2 = 2 * rpg * groups_per_wg;
    if ((rows + rpw2 - 1) / rpw2 * grid_y >= c->num_cu) rpg *= 2;
  }
  // whole row blocks per slot round the grid up: lengthen the runs until
  // it fits one round (a workgroup left over for a second round runs alone
  // and nearly doubles the launch)
  rpg = fit_one_round(rows, rpg, groups_per_wg, grid_y, (long)c->num_cu * wg_per_cu);
  a.rows_per_group = (int)rpg;
  a.one_token = p.T == 1 ? 1 : 0;
  const long rows_per_wg = rpg * groups_per_wg;
  const unsigned gx = (unsigned)((rows + rows_per_wg - 1) / rows_per_wg);
  a.kgx = (int)gx;

  if (gateup) {
    const dim3 grid(gx * (unsigned)slots_max);
    return launch(c, "gemv_gateup",
                  [&] { go(c, probe, grid, dim3(256), 0, a); });
  }
  if (down_rows) {
    const size_t pairs_total = (size_t)p.T * p.k + (has_shared ? (size_t)p.T : 0);
    float *ypair = p.ypair;
    if (kslices > 1) {
      void *yp = nullptr;
      NX_TRY(ws_get(c, WS_YPAIR, (size_t)kslices * pairs_total * ex->H * sizeof(float), &yp));
      ypair = static_cast<float *>(yp);
    }
    a.out = ypair;
    a.out_stride = ex->H;
    a.kslice_stride = pairs_total * ex->H;
    const dim3 grid(gx * (unsigned)(slots_max * kslices));
    NX_TRY(launch(c, "gemv_down", [&] { go(c, probe, grid, dim3(256), 0, a); }));
    // one token: the rows are in route order (see a.pslot), no pair lookup
    return launch_combine(c, ypair, p.rw, p.rcnt, a.pslot ? nullptr : p.inv, p.T, p.k, ex->H,
                          has_shared, p.out,
                          kslices, a.kslice_stride, p.residual);
  }

  a.rw = p.rw;
  a.rcnt = p.rcnt;
  a.inv = p.inv;
  a.final_out = p.out;
  a.residual = p.residual;
  a.npairs = (int)((long)p.T * p.k + (has_shared ? p.T : 0));
  const size_t part_bytes = (size_t)sh.ksplit * a.npairs * rows_per_wg * sizeof(float);
  const bool ylds = part_bytes <= kDownLdsMax;
  KernelFn fn = pick(ex->fmt, KIND_DOWN_COMBINE, ylds, nt, sh);
  if (!fn) return fail(NX_ERR_UNSUPPORTED, "no GEMV kernel instance for this shape");
  if (!ylds) {
    void *gp = nullptr;
    NX_TRY(ws_get(c, WS_YPAIR, part_bytes * gx, &gp));
    a.gpart = static_cast<float *>(gp);
  }
  const unsigned lds = ylds ? (unsigned)part_bytes : 0u;
  return launch(c, "gemv_down_combine",
                [&] { go(c, fn, dim3(gx), dim3(threads), lds, a); });
}

// One matrix over T tokens: the per-slot kernel with a single dense slot.
int run_gemv_matrix(nx_ctx *c, int fmt, const RolePlane &pl, const float *x, int T, float *out) {
  GemvArgs a{};
  a.kslices = 1;
  a.qs0 = a.qs1 = pl.qs;
  a.meta0 = a.meta1 = pl.meta;
  a.qs_stride = pl.qs_stride;
  a.meta_stride = pl.meta_stride;
  a.row_qs = pl.row_qs;
  a.row_meta = pl.row_meta;
  a.rows = pl.rows;
  a.cols = pl.cols;
  a.nseg = pl.nseg;
  a.E = 1;
  a.T = T;
  a.k = 1;
  a.x = x;
  a.x_stride = pl.cols;
  a.out = out;
  a.out_stride = pl.rows;
  int nt;
  Shape sh;
  if (!choose_tokens_shape(pl.nseg, elems_per_segment(fmt), T, &nt, &sh))
    return fail(NX_ERR_UNSUPPORTED, "row length too large for the register-resident GEMV");
  KernelFn fn = pick(fmt, KIND_DOWN_ROWS, true, nt, sh);
  if (!fn) return fail(NX_ERR_UNSUPPORTED, "no GEMV kernel instance for this shape");
  const int wg_per_cu = wg_per_cu_of(fn, 256);
  const int groups_per_wg = 256 / (sh.lpr * sh.ksplit);
  const long groups = (long)c->num_cu * wg_per_cu * groups_per_wg;
  long rpg = (pl.rows + groups - 1) / groups;
  if (rpg < 1) rpg = 1;
  rpg = fit_one_round(pl.rows, rpg, groups_per_wg, 1, (long)c->num_cu * wg_per_cu);
  a.rows_per_group = (int)rpg;
  const long rows_per_wg = rpg * groups_per_wg;
  const unsigned gx = (unsigned)((pl.rows + rows_per_wg - 1) / rows_per_wg);
  a.kgx = (int)gx;
  return launch(c, "gemv_matrix",
                [&] { go(c, fn, dim3(gx), dim3(256), 0, a); });
}

}  // namespace

int launch_gemv_matrix(nx_ctx *c, int fmt, const RolePlane &pl, const float *x, int T, float *out) {
  return run_gemv_matrix(c, fmt, pl, x, T, out);
}
bool gemv_row_fits(int fmt, int nseg) {
  int nt;
  Shape sh;
  return choose_tokens_shape(nseg, elems_per_segment(fmt), 1, &nt, &sh);
}
int launch_gemv_gateup(nx_ctx *c, const GemvPlan &p) { return run_gemv(c, p, true); }
int launch_gemv_down(nx_ctx *c, const GemvPlan &p) { return run_gemv(c, p, false); }

}  // namespace nx
