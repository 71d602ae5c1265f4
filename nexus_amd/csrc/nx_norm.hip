// nx_norm.hip — RMSNorm of a decoder block on gfx950.
//
// kernel::rms_norm (src/kernel/mod.rs:199-209): variance = (sum of x_i^2) /
// dim with the sum taken left to right, rstd = 1 / sqrt(variance + eps), and
// out_i = (x_i * rstd) * w_i.  Exact mode runs the register-run chain below
// for rows of whole float4 up to 7168, else takes the sum of squares from the
// sequential chain kernel (the router-logit chain kernel with each row
// paired with itself) and applies it here; the division and the square root
// are the correctly rounded ones (the compiler's default for HIP), so the
// output is bit-identical to the reference's.  Fast mode sums in parallel.
//
// The block's residual add (InferenceEngine::add_inplace,
// src/engine/mod.rs:803-807: hidden_i = hidden_i + y_i) happens in the final
// write of the layer's combine.
#include "nx_device.hpp"
#include "nx_internal.hpp"
#include "nx_rows.hpp"

namespace nx {

namespace {

__device__ __forceinline__ float rstd_of(float sumsq, int H, float eps) {
#pragma clang fp contract(off)
  return 1.0f / __builtin_sqrtf(sumsq / (float)H + eps);
}

// out[t][i] = (x[t][i] * rstd_t) * w[i]; grid (ceil(H / 1024), T), each
// thread four elements with all loads issued before the first use
__global__ __launch_bounds__(256) void k_rms_apply(const float *__restrict__ x,
                                                   const float *__restrict__ sumsq,
                                                   const float *__restrict__ w, float eps, int H,
                                                   float *__restrict__ out) {
#pragma clang fp contract(off)
  const int t = blockIdx.y;
  const size_t row = (size_t)t * H;
  const int i0 = blockIdx.x * 1024 + threadIdx.x;
  float xv[4], wv[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int i = i0 + 256 * u;
    xv[u] = i < H ? x[row + i] : 0.f;
    wv[u] = i < H ? w[i] : 0.f;
  }
  const float r = rstd_of(sumsq[t], H, eps);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int i = i0 + 256 * u;
    if (i < H) out[row + i] = (xv[u] * r) * wv[u];
  }
}

// fast mode: one 1024-thread workgroup per token; parallel sum of squares
// (fma) with every load of the row issued up front, then the same
// normalisation from the registers
constexpr int RMS_FAST_PER = 8;  // elements per thread kept in registers (H <= 8192)

__global__ __launch_bounds__(1024) void k_rms_fast(const float *__restrict__ x,
                                                   const float *__restrict__ w, float eps, int H,
                                                   float *__restrict__ out) {
#pragma clang fp contract(off)
  __shared__ float part[16];
  const int t = blockIdx.x;
  const size_t row = (size_t)t * H;
  float xv[RMS_FAST_PER];
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < RMS_FAST_PER; ++u) {
    const int i = threadIdx.x + 1024 * u;
    xv[u] = i < H ? x[row + i] : 0.f;
  }
  // rows longer than the register tile: the rest is summed from memory
  for (int i = threadIdx.x + 1024 * RMS_FAST_PER; i < H; i += 1024)
    s = __builtin_fmaf(x[row + i], x[row + i], s);
#pragma unroll
  for (int u = 0; u < RMS_FAST_PER; ++u) s = __builtin_fmaf(xv[u], xv[u], s);
  s = group_sum<64>(s);
  if ((threadIdx.x & 63) == 63) part[threadIdx.x >> 6] = s;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) tot += part[i];
  const float r = rstd_of(tot, H, eps);
#pragma unroll
  for (int u = 0; u < RMS_FAST_PER; ++u) {
    const int i = threadIdx.x + 1024 * u;
    if (i < H) out[row + i] = (xv[u] * r) * w[i];
  }
  for (int i = threadIdx.x + 1024 * RMS_FAST_PER; i < H; i += 1024)
    out[row + i] = (x[row + i] * r) * w[i];
}

// Exact mode for rows of whole float4 up to 64 S4 float4 (S4 = 16: rows up
// to 4096; S4 = 28: up to 7168): one wave per token, the whole RMSNorm in
// one launch.  A sequential sum runs at the dependent-add latency only with
// its operands already in registers, so the wave stages its row through its
// own LDS buffer (coalesced 16-byte loads; one float4 of padding per run of
// S4, so the lanes reading their runs' k-th float4 hit different banks) and
// lane r squares run r (columns 4 S4 r ..) in its registers.  The runs are
// added in order, each lane adding its run to the sum handed over by
// readlane from the lane before: the left-to-right sum of the reference,
// bit for bit (a partial last run adds +0 to a sum that started at +0).  Then
// out = (x rstd) w from the staged row.  No barrier: a wave's LDS accesses
// complete in order.  Requires H % 4 == 0, 0 < H <= 256 S4 and 16-byte
// aligned rows.
template <int S4>
__global__ __launch_bounds__(256) void k_rms_runs(const float *__restrict__ x,
                                                  const float *__restrict__ w, float eps, int T,
                                                  int H, float *__restrict__ out) {
#pragma clang fp contract(off)
  __shared__ float4 xs[4][64 * (S4 + 1)];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;  // (wave-uniform; no barrier follows)
  const int H4 = H >> 2;
  const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
  auto pad = [](int i) { return i + i / S4; };  // float4 i of the row -> LDS slot
  float4 *my = xs[wave];
  const float4 *xr4 = reinterpret_cast<const float4 *>(x + (size_t)t * H);
  {
    // indices clamped into the row, values selected afterwards: no branch,
    // every load issued before the first wait
    float4 v[S4];
#pragma unroll
    for (int j = 0; j < S4; ++j) v[j] = xr4[min(j * 64 + lane, H4 - 1)];
#pragma unroll
    for (int j = 0; j < S4; ++j) {
      const int i = j * 64 + lane;
      if (i >= H4) v[j] = z4;
      my[pad(i)] = v[j];
    }
  }
  // the runs below read other lanes' staged float4s: keep every staging
  // store of the wave ahead of them (a wave's LDS accesses complete in order)
  __builtin_amdgcn_wave_barrier();
  float ss = 0.f;
  {
    float4 q[S4];
#pragma unroll
    for (int k = 0; k < S4; ++k) {
      const float4 a = my[pad(lane * S4 + k)];
      q[k] = make_float4(a.x * a.x, a.y * a.y, a.z * a.z, a.w * a.w);
    }
    const int nr = (H4 + S4 - 1) / S4;
    for (int r = 0; r < nr; ++r) {
      float acc = ss;
#pragma unroll
      for (int k = 0; k < S4; ++k) {
        acc = acc + q[k].x;
        acc = acc + q[k].y;
        acc = acc + q[k].z;
        acc = acc + q[k].w;
      }
      ss = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), r));
    }
  }
  const float r = rstd_of(ss, H, eps);
  const float4 *w4 = reinterpret_cast<const float4 *>(w);
  float4 *o4 = reinterpret_cast<float4 *>(out + (size_t)t * H);
#pragma unroll
  for (int j = 0; j < S4; ++j) {
    const int i = j * 64 + lane;
    if (i < H4) {
      const float4 a = my[pad(i)], b = w4[i];
      o4[i] = make_float4((a.x * r) * b.x, (a.y * r) * b.y, (a.z * r) * b.z, (a.w * r) * b.w);
    }
  }
}

}  // namespace

bool rms_runs_fit(int H, const void *x, const void *w, const void *out) {
  static_assert(kRmsRunsMaxH == 256 * 28, "k_rms_runs<28>: 64 runs of 28 float4s");
  auto al = [](const void *q) { return ((uintptr_t)q & 15) == 0; };
  return register_row_fits(H, kRmsRunsMaxH) && al(x) && al(w) && al(out);
}

int launch_rms_exact_runs(nx_ctx *c, const float *d_x, const float *d_w, float eps, int T, int H,
                          float *d_out) {
  if (T <= 0 || H <= 0) return NX_OK;
  if (!rms_runs_fit(H, d_x, d_w, d_out))
    return fail(NX_ERR_UNSUPPORTED, "exact RMSNorm: row shape or alignment not supported");
  const dim3 grid((unsigned)((T + 3) / 4));
  return launch(c, "rms_exact_runs", [&] {
    if (H <= 256 * 16)
      go(c, k_rms_runs<16>, grid, dim3(256), 0, d_x, d_w, eps, T, H, d_out);
    else
      go(c, k_rms_runs<28>, grid, dim3(256), 0, d_x, d_w, eps, T, H, d_out);
  });
}

int launch_rms_apply(nx_ctx *c, const float *d_x, const float *d_sumsq, const float *d_w,
                     float eps, int T, int H, float *d_out) {
  if (T <= 0 || H <= 0) return NX_OK;
  const dim3 grid((H + 1023) / 1024, T);
  return launch(c, "rms_apply", [&] {
    go(c, k_rms_apply, dim3(grid), dim3(256), 0, d_x, d_sumsq, d_w, eps, H, d_out);
  });
}

int launch_rms_fast(nx_ctx *c, const float *d_x, const float *d_w, float eps, int T, int H,
                    float *d_out) {
  if (T <= 0 || H <= 0) return NX_OK;
  return launch(c, "rms_fast", [&] {
    go(c, k_rms_fast, dim3(T), dim3(1024), 0, d_x, d_w, eps, H, d_out);
  });
}

}  // namespace nx
