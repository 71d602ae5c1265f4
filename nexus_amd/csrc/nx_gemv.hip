// nx_gemv.hip — decode path: fused dequant-in-register GEMV over the resident
// quantized experts, fp32 accumulate.
//
// Replaces the three InferenceEngine::matvec calls, the SwiGLU and the
// weighted accumulate of dispatch_moe_ffn (src/engine/mod.rs:994-1021,
// 775-801) for the tokens routed to each expert.  Gate/up grid: x = row
// blocks, y = expert slot (the i-th active expert from the permutation, then
// one slot for the shared expert).  Down grid: row blocks only; each
// workgroup runs every slot over its rows and then combines them.
//
// A row group of L = LPR * KSPLIT lanes owns a run of rows.  Lane i of the
// group owns segments i, i+L, ... of every row (see nx_device.hpp), so the
// activations it needs are loaded into registers once per token group and
// reused for all rows.  Rows are processed U at a time in a two-stage
// software pipeline: the code and scale loads of the next U rows are issued
// before the current U rows are decoded and reduced (DPP adds within the
// group, an LDS sum across waves when KSPLIT > 1).
//
// The down projection writes each pair's output rows, then the same
// workgroup forms out[t] = sum_r w[t,r] * y[pair(t,r)] (+ shared) for its
// rows in route order — the reference's accumulation order, with no atomics
// and no communication between workgroups.
#include "nx_device.hpp"
#include "nx_internal.hpp"

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
  const int32_t *offsets;
  const int32_t *active;
  int E, T, k, has_shared;
  float *out;
  int out_stride;
  int rows_per_group;
  uint32_t mask_lo, mask_hi;  // 0x0F0F0F0F / 0xF0F0F0F0 (Q8_0: 0x80808080 in mask_hi)
  // combine (down projection)
  const float *rw;
  const int32_t *rcnt;
  const int32_t *inv;
  float *final_out;
};

template <int FMT, int LPR, int KSPLIT, int SPL, int NT, bool GATEUP>
__global__ __launch_bounds__(256, 2) void k_gemv(const GemvArgs a) {
  using S = Seg<FMT>;
  using Meta = typename S::Meta;
  constexpr int EPS = S::EPS, NXS = S::NXS;
  constexpr int NMAT = GATEUP ? 2 : 1;
  constexpr int L = LPR * KSPLIT;
  constexpr int GROUPS = 256 / L;
  constexpr int U = GATEUP ? 2 : 4;  // rows per pipeline stage
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = KSPLIT == 1 ? (lane % LPR) : tid;
  const int grp = KSPLIT == 1 ? (tid / LPR) : 0;

  const int n_active = a.active[a.E];
  const int n_slots = n_active + (a.has_shared ? 1 : 0);
  if (GATEUP && (int)blockIdx.y >= n_slots) return;  // workgroup-uniform
  __shared__ float red[KSPLIT > 1 ? 4 * U * NMAT * NT : 1];

  // gate/up: one slot per workgroup row; down: every slot, in order
  for (int si = 0; si < (GATEUP ? 1 : n_slots); ++si) {
  const int slot = GATEUP ? (int)blockIdx.y : si;
  // ---- slot -> expert, pair range, matrix bases (workgroup-uniform)
  int pair0, count, rows, cols, nseg;
  const uint8_t *q0p, *q1p, *m0p, *m1p;
  uint32_t rq, rm;
  bool routed;
  if (slot < n_active) {
    const int e = a.active[slot];
    pair0 = a.offsets[e];
    count = a.offsets[e + 1] - pair0;
    rows = a.rows;
    cols = a.cols;
    nseg = a.nseg;
    q0p = a.qs0 + (size_t)e * a.qs_stride;
    q1p = a.qs1 + (size_t)e * a.qs_stride;
    m0p = a.meta0 + (size_t)e * a.meta_stride;
    m1p = a.meta1 + (size_t)e * a.meta_stride;
    rq = a.row_qs;
    rm = a.row_meta;
    routed = true;
  } else {
    pair0 = a.T * a.k;
    count = a.T;
    rows = a.srows;
    cols = a.scols;
    nseg = a.snseg;
    q0p = a.sqs0;
    q1p = a.sqs1;
    m0p = a.smeta0;
    m1p = a.smeta1;
    rq = a.srow_qs;
    rm = a.srow_meta;
    routed = false;
  }
  const int row_begin = (blockIdx.x * GROUPS + grp) * a.rows_per_group;
  const int row_end = min(rows, row_begin + a.rows_per_group);

  // buffer resources over this expert's matrices (loads past the end read 0)
  const __amdgpu_buffer_rsrc_t rq0 = make_rsrc(q0p, (uint32_t)rows * rq);
  const __amdgpu_buffer_rsrc_t rq1 = make_rsrc(q1p, (uint32_t)rows * rq);
  const __amdgpu_buffer_rsrc_t rm0 = make_rsrc(m0p, (uint32_t)rows * rm);
  const __amdgpu_buffer_rsrc_t rm1 = make_rsrc(m1p, (uint32_t)rows * rm);

  // this lane's segments and their byte offsets inside a row (OOB if none)
  int jseg[SPL];
  bool jv[SPL];
  uint32_t off0[SPL], off1[SPL], moff[SPL];
#pragma unroll
  for (int m = 0; m < SPL; ++m) {
    jseg[m] = li + m * L;
    jv[m] = jseg[m] < nseg;
    off0[m] = jv[m] ? seg_off(jseg[m], 0, nseg) : OOB;
    off1[m] = jv[m] ? seg_off(jseg[m], 1, nseg) : OOB;
    moff[m] = S::meta_off(jseg[m], jv[m]);
  }

  struct Stage {
    uint4 q[U][NMAT][SPL][2];
    Meta m[U][NMAT][SPL];
  };
  // rows past row_end load zeros (their offsets are out of range) and are
  // never stored
  auto load = [&](Stage &st, int r0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool rv = r0 + u < row_end;
      const uint32_t rqo = rv ? (uint32_t)(r0 + u) * rq : OOB;
      const uint32_t rmo = rv ? (uint32_t)(r0 + u) * rm : OOB;
#pragma unroll
      for (int mt = 0; mt < NMAT; ++mt) {
#pragma unroll
        for (int m = 0; m < SPL; ++m) {
          st.q[u][mt][m][0] = bload16(mt == 0 ? rq0 : rq1, rqo + off0[m]);
          st.q[u][mt][m][1] = bload16(mt == 0 ? rq0 : rq1, rqo + off1[m]);
          st.m[u][mt][m] = S::load_meta(mt == 0 ? rm0 : rm1, rmo + moff[m]);
        }
      }
    }
  };

  for (int t0 = 0; t0 < count; t0 += NT) {
    // ---- activations of NT tokens for this lane's segments
    float x[SPL][NT][EPS];
    float xs[SPL][NT][NXS];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      // one buffer resource per token row, sized to the row: columns past
      // the row (padding, absent segments) and absent tokens read as zero
      const bool tv = t0 + t < count;
      const float *xrow = a.x;
      if (tv) {
        const int p = pair0 + t0 + t;
        const int row = GATEUP ? (routed ? a.perm_token[p] : (t0 + t)) : p;
        xrow = a.x + (size_t)row * a.x_stride;
      }
      const __amdgpu_buffer_rsrc_t xr = make_rsrc(xrow, tv ? (uint32_t)cols * 4u : 0u);
#pragma unroll
      for (int m = 0; m < SPL; ++m) {
#pragma unroll
        for (int v = 0; v < EPS; v += 4) {
          const uint32_t xo = jv[m] ? (uint32_t)S::xidx(jseg[m], v) * 4u : OOB;
          if constexpr (FMT == NX_FMT_F32) {
            // rows of odd length: element-wise so that each load is wholly in or out
#pragma unroll
            for (int e = 0; e < 4; ++e) x[m][t][v + e] = __uint_as_float(bload4(xr, xo + 4u * e));
          } else {
            const uint4 f = bload16(xr, xo);
            x[m][t][v] = __uint_as_float(f.x);
            x[m][t][v + 1] = __uint_as_float(f.y);
            x[m][t][v + 2] = __uint_as_float(f.z);
            x[m][t][v + 3] = __uint_as_float(f.w);
          }
        }
        S::xsums(x[m][t], xs[m][t]);
      }
    }

    auto compute = [&](const Stage &st, int r0) {
      float acc[U][NMAT][NT];
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
          for (int m = 0; m < SPL; ++m)
          {
            S::template dot<NT>(st.q[u][mt][m][0], st.q[u][mt][m][1], st.m[u][mt][m], jseg[m],
                                x[m], xs[m], acc[u][mt], a.mask_lo, a.mask_hi);
            // keep each segment's decode local: without this the scheduler
            // hoists every byte conversion of the stage and runs out of registers
            __builtin_amdgcn_sched_barrier(0);
          }
      group_sum_n<LPR, U * NMAT * NT>(&acc[0][0][0]);
      bool writer = (li % LPR) == LPR - 1;
      if constexpr (KSPLIT > 1) {
        if (lane == 63) {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
              for (int t = 0; t < NT; ++t) red[((wave * U + u) * NMAT + mt) * NT + t] = acc[u][mt][t];
        }
        __syncthreads();
        writer = tid == 255;
        if (writer) {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
              for (int t = 0; t < NT; ++t) {
                float s = 0.f;
#pragma unroll
                for (int w = 0; w < KSPLIT; ++w) s += red[((w * U + u) * NMAT + mt) * NT + t];
                acc[u][mt][t] = s;
              }
        }
        __syncthreads();
      }
      if (writer) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int r = r0 + u;
          if (r >= row_end) continue;
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            if (t0 + t >= count) continue;
            const float v = GATEUP ? silu_mul(acc[u][0][t], acc[u][NMAT - 1][t]) : acc[u][0][t];
            a.out[(size_t)(pair0 + t0 + t) * a.out_stride + r] = v;
          }
        }
      }
    };

    Stage A, B;
    load(A, row_begin);
    for (int r = row_begin; r < row_end; r += 2 * U) {
      load(B, r + U);
      compute(A, r);
      load(A, r + 2 * U);
      compute(B, r + U);
    }
  }

  }  // slot loop

  if constexpr (!GATEUP) {
    // combine this workgroup's rows: out[t][h] = sum_r w[t,r] * y[pair(t,r)][h]
    // (+ shared), in route order; the y rows were written by this workgroup
    __syncthreads();
    const int rb0 = blockIdx.x * GROUPS * a.rows_per_group;
    const int nr = min(a.rows, rb0 + GROUPS * a.rows_per_group) - rb0;
    for (int i = tid; i < nr * a.T; i += 256) {
      const int t = i / nr, h = rb0 + (i - t * nr);
      const int n = a.rcnt[t];
      float acc = 0.0f;
      for (int r = 0; r < n; ++r) {
        const int p = a.inv[(size_t)t * a.k + r];
        acc = acc + __fmul_rn(a.rw[(size_t)t * a.k + r], a.out[(size_t)p * a.out_stride + h]);
      }
      if (a.has_shared) acc = acc + a.out[((size_t)a.T * a.k + t) * a.out_stride + h];
      a.final_out[(size_t)t * a.rows + h] = acc;
    }
  }
}

using KernelFn = void (*)(GemvArgs);

struct Shape {
  int lpr, ksplit, spl;
};

template <int FMT, bool GATEUP, int NT>
KernelFn pick_shape(const Shape &s) {
  if (s.ksplit == 1) {
    if (s.lpr == 16 && s.spl == 1) return k_gemv<FMT, 16, 1, 1, NT, GATEUP>;
    if (s.lpr == 32 && s.spl == 1) return k_gemv<FMT, 32, 1, 1, NT, GATEUP>;
    if (s.lpr == 64 && s.spl == 1) return k_gemv<FMT, 64, 1, 1, NT, GATEUP>;
    if (s.lpr == 64 && s.spl == 2) return k_gemv<FMT, 64, 1, 2, NT, GATEUP>;
  } else {
    if (s.spl == 1) return k_gemv<FMT, 64, 4, 1, NT, GATEUP>;
    if (s.spl == 2) return k_gemv<FMT, 64, 4, 2, NT, GATEUP>;
  }
  return nullptr;
}

template <int FMT>
KernelFn pick_fmt(bool gateup, int nt, const Shape &s) {
  if (gateup) return nt == 1 ? pick_shape<FMT, true, 1>(s) : pick_shape<FMT, true, 2>(s);
  return nt == 1 ? pick_shape<FMT, false, 1>(s) : pick_shape<FMT, false, 2>(s);
}

KernelFn pick(int fmt, bool gateup, int nt, const Shape &s) {
  switch (fmt) {
  case NX_FMT_Q4_K: return pick_fmt<NX_FMT_Q4_K>(gateup, nt, s);
  case NX_FMT_Q8_0: return pick_fmt<NX_FMT_Q8_0>(gateup, nt, s);
  case NX_FMT_Q4_0: return pick_fmt<NX_FMT_Q4_0>(gateup, nt, s);
  case NX_FMT_F32: return pick_fmt<NX_FMT_F32>(gateup, nt, s);
  }
  return nullptr;
}

int elems_per_segment(int fmt) {
  switch (fmt) {
  case NX_FMT_Q4_K: return 64;
  case NX_FMT_Q8_0: return 32;
  case NX_FMT_Q4_0: return 64;
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
  else if (nseg <= 256) *s = {64, 4, 1};
  else if (nseg <= 512 && 2 * eps * nt <= budget) *s = {64, 4, 2};
  else return false;
  return true;
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
  } else {
    a.x = p.act;
    a.x_stride = p.act_stride;
    a.out = p.ypair;
    a.out_stride = ex->H;
  }

  const int nseg = a.nseg > a.snseg ? a.nseg : a.snseg;
  const int nt = p.T > 1 ? 2 : 1;
  Shape sh;
  if (!choose_shape(nseg, elems_per_segment(ex->fmt), nt, &sh))
    return fail(NX_ERR_UNSUPPORTED, "row length too large for the register-resident GEMV");
  const int L = sh.lpr * sh.ksplit;
  const int groups_per_wg = 256 / L;
  const int slots_max = (ex->E < p.T * p.k ? ex->E : p.T * p.k) + (has_shared ? 1 : 0);
  const int rows = a.rows > a.srows ? a.rows : a.srows;
  KernelFn fn = pick(ex->fmt, gateup, nt, sh);
  if (!fn) return fail(NX_ERR_UNSUPPORTED, "no GEMV kernel instance for this shape");
  int wg_per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&wg_per_cu, reinterpret_cast<const void *>(fn),
                                                   256, 0) != hipSuccess ||
      wg_per_cu < 1) {
    (void)hipGetLastError();
    wg_per_cu = 1;
  }
  // gate/up spreads slots over grid.y; down runs all slots inside each
  // workgroup.  Size the row runs so the launch is about one round of
  // resident workgroups, each with a long software pipeline.
  const long work_rows = gateup ? (long)rows * slots_max : (long)rows;
  const int step = gateup ? 4 : 8;  // rows per pipeline round (2 stages x U)
  const long groups = (long)c->num_cu * wg_per_cu * groups_per_wg;
  long rpg = (work_rows + groups - 1) / groups;
  rpg = (rpg + step - 1) / step * step;
  if (rpg < step) rpg = step;
  a.rows_per_group = (int)rpg;
  a.mask_lo = 0x0F0F0F0Fu;
  a.mask_hi = ex->fmt == NX_FMT_Q8_0 ? 0x80808080u : 0xF0F0F0F0u;
  const long rows_per_wg = rpg * groups_per_wg;
  const unsigned gx = (unsigned)((rows + rows_per_wg - 1) / rows_per_wg);
  if (!gateup) {
    a.rw = p.rw;
    a.rcnt = p.rcnt;
    a.inv = p.inv;
    a.final_out = p.out;
  }
  const char *name = gateup ? "gemv_gateup" : "gemv_down_combine";
  const dim3 grid(gx, gateup ? (unsigned)slots_max : 1u);
  return launch(c, name, [&] { hipLaunchKernelGGL(fn, grid, dim3(256), 0, c->stream, a); });
}

}  // namespace

int launch_gemv_gateup(nx_ctx *c, const GemvPlan &p) { return run_gemv(c, p, true); }
int launch_gemv_down(nx_ctx *c, const GemvPlan &p) { return run_gemv(c, p, false); }

}  // namespace nx
