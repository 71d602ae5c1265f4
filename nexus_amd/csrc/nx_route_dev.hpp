// nx_route_dev.hpp — the one-token router as a device function, shared by the
// router kernels and by the gate/up GEMV (which routes a lone decode token
// itself instead of waiting on a router launch).
//
// InferenceEngine::route_moe_experts (src/engine/mod.rs:918-966): each finite
// logit becomes a 64-bit key (total-order-sortable f32 bits << 32 | ~expert),
// so a wave-wide max picks the largest logit and, among identical bit
// patterns, the lowest expert index; non-finite logits are never selected.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/nexus_hip.h"

namespace nx {

__device__ __forceinline__ uint32_t sortable(float f) {
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float unsortable(uint32_t s) {
  return __uint_as_float((s & 0x80000000u) ? (s & 0x7FFFFFFFu) : ~s);
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = __shfl_xor((uint32_t)v, m, 64);
  const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), m, 64);
  return ((uint64_t)hi << 32) | lo;
}

// Routes one token with one wavefront.  On return lane r < *n holds the r-th
// route (expert *e, weight *w); lanes >= *n hold e = -1, w = 0.  With
// weights false (wave-uniform) only the selection is made and *w is 0.
template <int EPL>
__device__ __forceinline__ void route_one(const float *__restrict__ row, int E, int k,
                                          int score_mode, int lane, int *e_out, float *w_out,
                                          int *n_out, bool weights = true) {
  uint64_t key[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + 64 * i;
    key[i] = 0;
    if (e < E) {
      const float l = row[e];
      if (isfinite(l)) key[i] = ((uint64_t)sortable(l) << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)e);
    }
  }
  const int kk = k < E ? k : E;
  uint64_t mine = 0;  // lane r keeps the r-th selection
  int n = 0;
  for (int r = 0; r < kk; ++r) {
    uint64_t best = 0;
#pragma unroll
    for (int i = 0; i < EPL; ++i) best = key[i] > best ? key[i] : best;
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) {
      const uint64_t o = shfl_xor_u64(best, m);
      best = o > best ? o : best;
    }
    if (best == 0) break;  // no finite logits left (uniform across the wave)
#pragma unroll
    for (int i = 0; i < EPL; ++i)
      if (key[i] == best) key[i] = 0;
    if (lane == r) mine = best;
    ++n;
  }
  float l = 0.f, w = 0.f;
  int e = -1;
  if (lane < n) {
    l = unsortable((uint32_t)(mine >> 32));
    e = (int)(0xFFFFFFFFu - (uint32_t)mine);
  }
  *e_out = e;
  *n_out = n;
  *w_out = 0.f;
  if (!weights) return;
  const float l0 = __shfl(l, 0, 64);  // largest selected logit
  if (lane < n) {
    if (score_mode == NX_SCORE_SOFTMAX) {
      w = (float)exp((double)(l - l0));
    } else {
      const float ex = (float)exp(-(double)l);
      w = 1.0f / (1.0f + ex);
    }
  }
  // sequential f32 sum in route order (Iterator::sum)
  float sum = -0.0f;
  for (int r = 0; r < n; ++r) sum = sum + __shfl(w, r, 64);
  if (sum > 0.0f && lane < n) w = w / sum;
  *w_out = w;
}

}  // namespace nx
