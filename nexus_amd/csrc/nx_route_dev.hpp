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

// v of another lane of the same 16-lane row, by a DPP lane pattern (every
// lane reads a lane inside its row, so none reads out of range)
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, 0xF, 0xF, false);
  return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}

__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int l) {
  const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)v, l);
  const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// maximum over the wave, in every lane: within each 16-lane row by DPP
// (swap neighbours, swap pairs, mirror halves of 8, mirror the row), then
// across the four rows from lanes 0, 16, 32, 48
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  v = max_u64(v, dpp_u64<0xB1>(v));   // quad_perm [1, 0, 3, 2]
  v = max_u64(v, dpp_u64<0x4E>(v));   // quad_perm [2, 3, 0, 1]
  v = max_u64(v, dpp_u64<0x141>(v));  // row_half_mirror
  v = max_u64(v, dpp_u64<0x140>(v));  // row_mirror
  return max_u64(max_u64(readlane_u64(v, 0), readlane_u64(v, 16)),
                 max_u64(readlane_u64(v, 32), readlane_u64(v, 48)));
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
    best = wave_max_u64(best);
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
  // largest selected logit (lane 0's)
  const float l0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(l), 0));
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
  for (int r = 0; r < n; ++r) sum = sum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), r));
  if (sum > 0.0f && lane < n) w = w / sum;
  *w_out = w;
}

}  // namespace nx
