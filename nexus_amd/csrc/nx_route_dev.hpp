// nx_route_dev.hpp — the one-token router as a device function, shared by the
// router kernels and by the gate/up GEMV (which routes a lone decode token
// itself instead of waiting on a router launch).
//
// InferenceEngine::route_moe_experts (src/engine/mod.rs:918-966): each finite
// logit becomes a 32-bit total-order-sortable key, a wave-wide max picks the
// largest logit and a ballot of its holders the lowest expert index among
// identical bit patterns; non-finite logits are never selected.
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
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

// maximum over the wave, in every lane: within each 16-lane row by DPP
// (swap neighbours, swap pairs, mirror halves of 8, mirror the row), then
// across the four rows from lanes 0, 16, 32, 48
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v));   // quad_perm [1, 0, 3, 2]
  v = max(v, dpp_u32<0x4E>(v));   // quad_perm [2, 3, 0, 1]
  v = max(v, dpp_u32<0x141>(v));  // row_half_mirror
  v = max(v, dpp_u32<0x140>(v));  // row_mirror
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
  const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
  const uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return max(max(a, b), max(c, d));
}

// The logits of one token as held by the router: lane holds expert
// lane + 64 i in l[i].  The loads are unconditional (indices clamped to the
// last expert, E >= 1), so they are in flight together and a caller can
// issue them before other loads it does not want the routing to wait for.
template <int EPL>
__device__ __forceinline__ void route_load(const float *__restrict__ row, int E, int lane,
                                           float (&l)[EPL]) {
#pragma unroll
  for (int i = 0; i < EPL; ++i) l[i] = row[min(lane + 64 * i, E - 1)];
}

// Routes one token with one wavefront from the logits route_load gave (the
// first EPL of them; 64 EPL >= E).  On return lane r < *n holds the r-th
// route (expert *e, weight *w); lanes >= *n hold e = -1, w = 0.  With
// weights false (wave-uniform) only the selection is made and *w is 0.
//
// Expert lane + 64 i keeps key[i] = the total-order-sortable bits of its
// logit (0 for a non-finite logit, a value no finite logit maps to).  Each
// selection takes the wave's largest key, then, among the experts holding
// exactly that key, the lowest index (the first set bit of the lowest
// non-empty ballot): the stable descending sort of the reference.
template <int EPL, int LN>
__device__ __forceinline__ void route_select(const float (&lv)[LN], int E, int k, int score_mode,
                                             int lane, int *e_out, float *w_out, int *n_out,
                                             bool weights = true) {
  static_assert(EPL <= LN, "the logits of every expert are loaded");
  uint32_t key[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i)
    key[i] = lane + 64 * i < E && isfinite(lv[i]) ? sortable(lv[i]) : 0u;
  const int kk = k < E ? k : E;
  uint32_t mine = 0;  // lane r keeps the r-th selection: its key and expert
  int mine_e = -1;
  int n = 0;
  for (int r = 0; r < kk; ++r) {
    uint32_t best = key[0];
#pragma unroll
    for (int i = 1; i < EPL; ++i) best = max(best, key[i]);
    best = wave_max_u32(best);
    if (best == 0) break;  // no finite logits left (uniform across the wave)
    int win = -1;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const unsigned long long m = __ballot(key[i] == best);
      if (win < 0 && m != 0ull) win = 64 * i + (int)__builtin_ctzll(m);
    }
#pragma unroll
    for (int i = 0; i < EPL; ++i)
      if (win == lane + 64 * i) key[i] = 0;
    if (lane == r) {
      mine = best;
      mine_e = win;
    }
    ++n;
  }
  float l = 0.f, w = 0.f;
  int e = -1;
  if (lane < n) {
    l = unsortable(mine);
    e = mine_e;
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

// route_load + route_select: routes the token whose logits are row[0 .. E)
template <int EPL>
__device__ __forceinline__ void route_one(const float *__restrict__ row, int E, int k,
                                          int score_mode, int lane, int *e_out, float *w_out,
                                          int *n_out, bool weights = true) {
  float l[EPL];
  route_load<EPL>(row, E, lane, l);
  route_select<EPL>(l, E, k, score_mode, lane, e_out, w_out, n_out, weights);
}

}  // namespace nx
