// nx_norm.hip — RMSNorm of a decoder block on gfx950.
//
// kernel::rms_norm (src/kernel/mod.rs:199-209): variance = (sum of x_i^2) /
// dim with the sum taken left to right, rstd = 1 / sqrt(variance + eps), and
// out_i = (x_i * rstd) * w_i.  Exact mode takes the sum of squares from the
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

}  // namespace

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
