// nx_gemv.hip — decode path: fused dequant-in-register GEMV over the resident
// quantized experts, fp32 accumulate.
//
// Replaces the three InferenceEngine::matvec calls and the SwiGLU of
// dispatch_moe_ffn (src/engine/mod.rs:996-1017, 775-801) for the tokens routed
// to each expert.  Launch grid: x = row blocks, y = expert slot (the i-th
// active expert from the permutation, plus one slot for the shared expert).
//
// A "row group" of KSPLIT wavefronts owns a run of rows.  Lane g of the group
// always loads the same chunks of every row (c = g + m * 64 * KSPLIT), so the
// activations it needs are loaded into registers once per token group and
// reused for every row; each row costs the lane CPL 16-byte code loads (plus
// the small scale vectors) and the dot products, followed by a wavefront
// butterfly and, for KSPLIT > 1, an LDS sum across the group's waves.
//
// Q4_K: the dot product is evaluated as d*sc*sum(q*x) - dmin*m*sum(x) per
// 16-element half chunk, sum(x) being precomputed with the activations.
#include "nx_device.hpp"
#include "nx_internal.hpp"

namespace nx {

namespace {

struct GemvArgs {
  const uint8_t *qs[2];
  const uint8_t *meta[2];
  size_t qs_stride, meta_stride;  // per expert
  size_t row_qs, row_meta;        // per row
  const uint8_t *sqs[2];
  const uint8_t *smeta[2];
  size_t srow_qs, srow_meta;
  int rows, cols, nch;      // routed experts
  int srows, scols, snch;   // shared expert
  const float *x;
  int x_stride;
  const int32_t *perm_token;  // gate/up: pair -> token (null for down)
  const int32_t *offsets;
  const int32_t *active;
  int E, T, k, has_shared;
  float *out;
  int out_stride;
  int rows_per_group;
};

template <int FMT, int KSPLIT, int CPL, int NT, bool GATEUP>
__global__ __launch_bounds__(256) void k_gemv(const GemvArgs a) {
  using Fm = Fmt<FMT>;
  constexpr int NMAT = GATEUP ? 2 : 1;
  constexpr int LANES = 64 * KSPLIT;
  constexpr int GROUPS = 4 / KSPLIT;
  constexpr int U = KSPLIT == 1 ? 2 : 4;  // rows in flight per iteration
  constexpr int XPC = Fm::XPC;
  constexpr int NXS = Fm::NXS;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int gid = KSPLIT == 1 ? lane : (int)threadIdx.x;
  const int group = KSPLIT == 1 ? wave : 0;

  // ---- slot -> expert, pair range, matrix bases
  const int slot = blockIdx.y;
  const int n_active = a.active[a.E];
  int pair0, count, rows, cols, nch;
  const uint8_t *qs[NMAT];
  const uint8_t *meta[NMAT];
  size_t rq, rm;
  bool routed;
  if (slot < n_active) {
    const int e = a.active[slot];
    pair0 = a.offsets[e];
    count = a.offsets[e + 1] - pair0;
    rows = a.rows;
    cols = a.cols;
    nch = a.nch;
#pragma unroll
    for (int m = 0; m < NMAT; ++m) {
      qs[m] = a.qs[m] + (size_t)e * a.qs_stride;
      meta[m] = a.meta[m] + (size_t)e * a.meta_stride;
    }
    rq = a.row_qs;
    rm = a.row_meta;
    routed = true;
  } else if (a.has_shared && slot == n_active) {
    pair0 = a.T * a.k;
    count = a.T;
    rows = a.srows;
    cols = a.scols;
    nch = a.snch;
#pragma unroll
    for (int m = 0; m < NMAT; ++m) {
      qs[m] = a.sqs[m];
      meta[m] = a.smeta[m];
    }
    rq = a.srow_qs;
    rm = a.srow_meta;
    routed = false;
  } else {
    return;  // workgroup-uniform
  }
  const int row_begin = (blockIdx.x * GROUPS + group) * a.rows_per_group;
  if (KSPLIT > 1 && row_begin >= rows) return;  // workgroup-uniform when KSPLIT > 1
  const int row_end = min(rows, row_begin + a.rows_per_group);

  __shared__ float red[KSPLIT > 1 ? 4 * U * NMAT * NT : 1];

  for (int t0 = 0; t0 < count; t0 += NT) {
    // ---- activations for NT tokens into registers
    float x[NT][CPL][XPC];
    float xs[NT][CPL][NXS];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const bool tv = t0 + j < count;
      const float *xrow = a.x;
      if (tv) {
        const int p = pair0 + t0 + j;
        if (GATEUP) {
          const int tok = routed ? a.perm_token[p] : (t0 + j);
          xrow = a.x + (size_t)tok * a.x_stride;
        } else {
          xrow = a.x + (size_t)p * a.x_stride;
        }
      }
#pragma unroll
      for (int m = 0; m < CPL; ++m) {
        const int c = gid + m * LANES;
        const bool cv = tv && c < nch;
        if constexpr (FMT == NX_FMT_F32) {
#pragma unroll
          for (int v = 0; v < XPC; ++v) {
            const int xi = Fm::xidx(c, v);
            x[j][m][v] = (cv && xi < cols) ? xrow[xi] : 0.f;
          }
        } else {
#pragma unroll
          for (int v = 0; v < XPC; v += 4) {
            float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
            if (cv) f = *reinterpret_cast<const float4 *>(xrow + Fm::xidx(c, v));
            x[j][m][v] = f.x;
            x[j][m][v + 1] = f.y;
            x[j][m][v + 2] = f.z;
            x[j][m][v + 3] = f.w;
          }
        }
        Fm::xsums(x[j][m], xs[j][m]);
      }
    }

    // ---- rows
    for (int r0 = row_begin; r0 < row_end; r0 += U) {
      uint4 q[U][NMAT][CPL];
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
          for (int m = 0; m < CPL; ++m) {
            const int c = gid + m * LANES;
            const int r = r0 + u;
            q[u][mt][m] = make_uint4(0, 0, 0, 0);
            if (r < row_end && c < nch)
              q[u][mt][m] = *reinterpret_cast<const uint4 *>(qs[mt] + (size_t)r * rq + (size_t)c * 16);
          }
      float acc[U][NMAT][NT];
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
          for (int j = 0; j < NT; ++j) acc[u][mt][j] = 0.f;
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
          for (int m = 0; m < CPL; ++m) {
            const int c = gid + m * LANES;
            const int r = r0 + u;
            if (r < row_end && c < nch) {
              typename Fm::Dec dec;
              Fm::decode(q[u][mt][m], meta[mt] + (size_t)r * rm, c, dec);
#pragma unroll
              for (int j = 0; j < NT; ++j) acc[u][mt][j] += Fm::dot(dec, x[j][m], xs[j][m]);
            }
          }
      // ---- reduce
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
          for (int j = 0; j < NT; ++j) acc[u][mt][j] = wave_sum(acc[u][mt][j]);
      if constexpr (KSPLIT > 1) {
        if (lane == 0) {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
              for (int j = 0; j < NT; ++j) red[((wave * U + u) * NMAT + mt) * NT + j] = acc[u][mt][j];
        }
        __syncthreads();
        if (wave == 0) {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
              for (int j = 0; j < NT; ++j) {
                float s = 0.f;
#pragma unroll
                for (int w = 0; w < KSPLIT; ++w) s += red[((w * U + u) * NMAT + mt) * NT + j];
                acc[u][mt][j] = s;
              }
        }
        __syncthreads();
        if (wave != 0) continue;
      }
      // ---- epilogue: lane u*NT + j writes row r0+u of token t0+j
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          const int r = r0 + u;
          if (lane == u * NT + j && r < row_end && t0 + j < count) {
            float v;
            if (GATEUP)
              v = silu_mul(acc[u][0][j], acc[u][NMAT - 1][j]);
            else
              v = acc[u][0][j];
            a.out[(size_t)(pair0 + t0 + j) * a.out_stride + r] = v;
          }
        }
    }
  }
}

using KernelFn = void (*)(GemvArgs);

template <int FMT, bool GATEUP>
KernelFn pick(int ksplit, int cpl, int nt) {
#define NX_K(KS, C, N) \
  if (ksplit == KS && cpl == C && nt == N) return k_gemv<FMT, KS, C, N, GATEUP>;
#define NX_KN(KS, C) NX_K(KS, C, 1) NX_K(KS, C, 2)
  NX_KN(1, 1) NX_KN(1, 2) NX_KN(1, 4) NX_KN(1, 8)
  NX_KN(4, 1) NX_KN(4, 2) NX_KN(4, 4) NX_KN(4, 8)
#undef NX_KN
#undef NX_K
  return nullptr;
}

KernelFn pick_fmt(int fmt, bool gateup, int ksplit, int cpl, int nt) {
  switch (fmt) {
  case NX_FMT_Q4_K: return gateup ? pick<NX_FMT_Q4_K, true>(ksplit, cpl, nt) : pick<NX_FMT_Q4_K, false>(ksplit, cpl, nt);
  case NX_FMT_Q8_0: return gateup ? pick<NX_FMT_Q8_0, true>(ksplit, cpl, nt) : pick<NX_FMT_Q8_0, false>(ksplit, cpl, nt);
  case NX_FMT_Q4_0: return gateup ? pick<NX_FMT_Q4_0, true>(ksplit, cpl, nt) : pick<NX_FMT_Q4_0, false>(ksplit, cpl, nt);
  case NX_FMT_F32: return gateup ? pick<NX_FMT_F32, true>(ksplit, cpl, nt) : pick<NX_FMT_F32, false>(ksplit, cpl, nt);
  }
  return nullptr;
}

int x_per_chunk(int fmt) {
  switch (fmt) {
  case NX_FMT_Q4_K: return 32;
  case NX_FMT_Q8_0: return 16;
  case NX_FMT_Q4_0: return 32;
  default: return 4;
  }
}

int chunks_per_row(int fmt, int cols) {
  switch (fmt) {
  case NX_FMT_Q4_K: return cols / 256 * 8;
  case NX_FMT_Q8_0: return cols / 32 * 2;
  case NX_FMT_Q4_0: return cols / 32;
  default: return (cols + 3) / 4;
  }
}

int run_gemv(nx_ctx *c, const GemmPlan *, const GemvPlan &p, bool gateup) {
  const nx_experts *ex = p.ex;
  const int ri = gateup ? NX_ROLE_GATE : NX_ROLE_DOWN;
  const RolePlane &R0 = ex->role[ri];
  const RolePlane &R1 = ex->role[gateup ? NX_ROLE_UP : NX_ROLE_DOWN];
  const bool has_shared = ex->Fs > 0;
  const RolePlane &S0 = ex->shared[ri];
  const RolePlane &S1 = ex->shared[gateup ? NX_ROLE_UP : NX_ROLE_DOWN];

  GemvArgs a{};
  a.qs[0] = R0.qs;
  a.meta[0] = R0.meta;
  a.qs[1] = R1.qs;
  a.meta[1] = R1.meta;
  a.qs_stride = R0.qs_stride;
  a.meta_stride = R0.meta_stride;
  FormatInfo fi;
  format_info(ex->fmt, &fi);
  a.row_qs = (size_t)R0.nblocks * fi.qs_bytes;
  a.row_meta = (size_t)R0.nblocks * fi.meta_bytes;
  a.rows = R0.rows;
  a.cols = R0.cols;
  a.nch = chunks_per_row(ex->fmt, R0.cols);
  if (has_shared) {
    a.sqs[0] = S0.qs;
    a.smeta[0] = S0.meta;
    a.sqs[1] = S1.qs;
    a.smeta[1] = S1.meta;
    a.srow_qs = (size_t)S0.nblocks * fi.qs_bytes;
    a.srow_meta = (size_t)S0.nblocks * fi.meta_bytes;
    a.srows = S0.rows;
    a.scols = S0.cols;
    a.snch = chunks_per_row(ex->fmt, S0.cols);
  }
  a.perm_token = gateup ? p.perm_token : nullptr;
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

  // ---- shape of the launch
  const int nch = a.nch > a.snch ? a.nch : a.snch;
  const int xpc = x_per_chunk(ex->fmt);
  const int nt = p.T > 1 ? 2 : 1;
  const int budget = 128;  // activation registers per lane
  int ksplit = 1;
  int cpl = (nch + 63) / 64;
  if (cpl * xpc * nt > budget || cpl > 8) {
    ksplit = 4;
    cpl = (nch + 255) / 256;
  }
  if (cpl > 8 || cpl * xpc * nt > 256)
    return fail(NX_ERR_UNSUPPORTED, "GEMV row length too large for the register-resident path");
  if (cpl == 3) cpl = 4;
  if (cpl > 4) cpl = 8;

  const int slots_max = (ex->E < p.T * p.k ? ex->E : p.T * p.k) + (has_shared ? 1 : 0);
  const int rows = a.rows > a.srows ? a.rows : a.srows;
  const int groups_per_wg = 4 / ksplit;
  const int U = ksplit == 1 ? 2 : 4;
  const long target_groups = (long)c->num_cu * 16;
  long rpg = ((long)rows * slots_max + target_groups - 1) / target_groups;
  if (rpg < U) rpg = U;
  if (rpg > 64) rpg = 64;
  rpg = (rpg + U - 1) / U * U;
  a.rows_per_group = (int)rpg;
  const long rows_per_wg = rpg * groups_per_wg;
  const unsigned gx = (unsigned)((rows + rows_per_wg - 1) / rows_per_wg);
  KernelFn fn = pick_fmt(ex->fmt, gateup, ksplit, cpl, nt);
  if (!fn) return fail(NX_ERR_UNSUPPORTED, "no GEMV kernel instance for this shape");
  const char *name = gateup ? "gemv_gateup" : "gemv_down";
  return launch(c, name, [&] {
    hipLaunchKernelGGL(fn, dim3(gx, (unsigned)slots_max), dim3(256), 0, c->stream, a);
  });
}

}  // namespace

int launch_gemv_gateup(nx_ctx *c, const GemvPlan &p) { return run_gemv(c, nullptr, p, true); }
int launch_gemv_down(nx_ctx *c, const GemvPlan &p) { return run_gemv(c, nullptr, p, false); }

}  // namespace nx
