// nx_route.hip — top-k router, token->expert permutation and weighted combine
// on gfx950.
//
// Router (InferenceEngine::route_moe_experts, src/engine/mod.rs:918-966): one
// wavefront per token.  Each finite logit becomes a 64-bit key
// (total-order-sortable f32 bits << 32 | ~expert), so a wave-wide max picks
// the largest logit and, among identical bit patterns, the lowest expert
// index — exactly the order of the reference's stable descending sort by
// f32::total_cmp (+0.0 above -0.0).  Non-finite logits get key 0 and are never
// selected.  k rounds of arg-max give the top-k in order; the weights are
// exp(l - l_max) (evaluated in double and rounded once, which agrees with
// glibc expf to the last bit except where glibc's own error exceeds half an
// ulp), summed sequentially in route order and divided as in the reference.
//
// Permutation (no reference counterpart; it reorders the per-token loop of
// src/engine/mod.rs:994): a stable counting sort of the (token, slot) pairs by
// expert in one workgroup — LDS histogram, workgroup scan, then per chunk of
// tokens a bit matrix [expert][token] whose popcount prefix gives each pair
// its rank among earlier tokens of the same expert.
//
// Combine (src/engine/mod.rs:1018-1020): out[t] = sum over routes in route
// order of w * y, starting from 0, with no atomics (gather by inverse
// permutation), so the result is deterministic.
#include "nx_device.hpp"
#include "nx_internal.hpp"
#include "nx_route_dev.hpp"

namespace nx {

namespace {

template <int EPL>
__global__ __launch_bounds__(256) void k_route(const float *__restrict__ logits, int T, int E,
                                               int k, int score_mode,
                                               int32_t *__restrict__ rexp,
                                               float *__restrict__ rw,
                                               int32_t *__restrict__ rcnt) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;  // wave-uniform
  int e, n;
  float w;
  route_one<EPL>(logits + (size_t)t * E, E, k, score_mode, lane, &e, &w, &n);
  if (lane < k) {
    rexp[(size_t)t * k + lane] = e;
    rw[(size_t)t * k + lane] = w;
  }
  if (lane == 0) rcnt[t] = n;
}

// exclusive scan of one value per thread over a 1024-thread workgroup
__device__ int block_exclusive_scan(int v, int *wave_tot, int *total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) wave_tot[wave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) {
      const int s = wave_tot[w];
      wave_tot[w] = run;
      run += s;
    }
    *total = run;
  }
  __syncthreads();
  const int r = x - v + wave_tot[wave];
  __syncthreads();
  return r;
}

constexpr int PERM_THREADS = 1024;
constexpr int PERM_WORDS = 4096;  // LDS words per bit matrix
constexpr int PERM_KREG = 8;      // routes per token the permutation keeps in registers

__global__ __launch_bounds__(PERM_THREADS) void k_permute(
    const int32_t *__restrict__ rexp, const int32_t *__restrict__ rcnt, int T, int k, int E,
    int W, int tile_m, int32_t *__restrict__ ecount, int32_t *__restrict__ offsets,
    int32_t *__restrict__ ptok, int32_t *__restrict__ pslot, int32_t *__restrict__ inv,
    int32_t *__restrict__ active, int32_t *__restrict__ tiles, int shared_T, int tile_m2,
    int32_t *__restrict__ tiles2) {
  __shared__ int cnt[PERM_THREADS];
  __shared__ int base[PERM_THREADS];
  __shared__ int run[PERM_THREADS];
  __shared__ uint32_t bits[PERM_WORDS];
  __shared__ uint32_t pref[PERM_WORDS];
  __shared__ int wave_tot[PERM_THREADS / 64];
  __shared__ int total;
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += PERM_THREADS) cnt[e] = 0;
  __syncthreads();
  const int pairs = T * k;
  // PERM_HB pairs per thread at a time: their route and count loads all go
  // out before the first is used (no dependent round trip per pair)
  constexpr int PERM_HB = 8;
  for (int i0 = tid; i0 < pairs; i0 += PERM_HB * PERM_THREADS) {
    int ev[PERM_HB], nv[PERM_HB], rv[PERM_HB];
#pragma unroll
    for (int j = 0; j < PERM_HB; ++j) {
      const int i = i0 + j * PERM_THREADS;
      const int ic = i < pairs ? i : 0;
      const int t = ic / k;
      rv[j] = i < pairs ? ic - t * k : k;  // slot (k: no pair)
      ev[j] = rexp[ic];
      nv[j] = rcnt[t];
    }
#pragma unroll
    for (int j = 0; j < PERM_HB; ++j)
      if (rv[j] < nv[j]) atomicAdd(&cnt[ev[j]], 1);
  }
  __syncthreads();
  // E <= PERM_THREADS: one expert per thread
  const int c = tid < E ? cnt[tid] : 0;
  const int b = block_exclusive_scan(c, wave_tot, &total);
  const int npairs = total;
  if (tid < E) {
    base[tid] = b;
    run[tid] = 0;
    ecount[tid] = c;
    offsets[tid] = b;
  }
  if (tid == 0) offsets[E] = npairs;
  const int act = block_exclusive_scan(tid < E && c > 0 ? 1 : 0, wave_tot, &total);
  const int n_active = total;
  if (tid < E && c > 0) active[act] = tid;
  if (tid == 0) active[E] = n_active;
  // tile lists for the grouped GEMM: (expert, first row) per tm rows, the
  // shared expert's tiles last; a second list for a second tile height
  auto tile_list = [&](int tm, int32_t *out) {
    const int nt = tid < E ? (c + tm - 1) / tm : 0;
    const int tb = block_exclusive_scan(nt, wave_tot, &total);
    const int ntiles = total;
    for (int j = 0; j < nt; ++j) {
      out[2 + 2 * (tb + j)] = tid;
      out[2 + 2 * (tb + j) + 1] = j * tm;
    }
    const int nshared = (shared_T + tm - 1) / tm;
    for (int j = tid; j < nshared; j += PERM_THREADS) {
      out[2 + 2 * (ntiles + j)] = E;
      out[2 + 2 * (ntiles + j) + 1] = j * tm;
    }
    if (tid == 0) {
      out[0] = ntiles + nshared;
      out[1] = 0;
    }
  };
  if (tiles != nullptr) tile_list(tile_m, tiles);
  if (tiles2 != nullptr) tile_list(tile_m2, tiles2);
  __syncthreads();
  // ranks: chunks of CT = 32*W tokens, one token per thread
  const int CT = 32 * W;
  for (int t0 = 0; t0 < T; t0 += CT) {
    for (int i = tid; i < E * W; i += PERM_THREADS) bits[i] = 0;
    __syncthreads();
    const int tl = tid;
    const int t = t0 + tl;
    const bool mine = tl < CT && t < T;
    int nr = 0;
    // up to PERM_KREG routes per token are read once, all in flight together,
    // and kept for the rank pass
    int er[PERM_KREG];
    const bool kreg = k <= PERM_KREG;
    if (mine) {
      nr = rcnt[t];
      if (kreg) {
#pragma unroll
        for (int r = 0; r < PERM_KREG; ++r) er[r] = r < k ? rexp[(size_t)t * k + r] : 0;
#pragma unroll
        for (int r = 0; r < PERM_KREG; ++r)
          if (r < nr) atomicOr(&bits[er[r] * W + (tl >> 5)], 1u << (tl & 31));
      } else {
        for (int r = 0; r < nr; ++r) {
          const int e = rexp[(size_t)t * k + r];
          atomicOr(&bits[e * W + (tl >> 5)], 1u << (tl & 31));
        }
      }
    }
    __syncthreads();
    // pref[e W + w] = set bits of row e's words 0 .. w-1: W (a power of two
    // dividing 64) consecutive lanes hold one row, scanned with shuffles
    for (int i0 = 0; i0 < E * W; i0 += PERM_THREADS) {
      const int i = i0 + tid;  // every lane of a wave takes part in the shuffles
      const int v = i < E * W ? __popc(bits[i]) : 0;
      int x = v;
      for (int d = 1; d < W; d <<= 1) {
        const int y = __shfl_up(x, d, W);
        if ((tid & (W - 1)) >= d) x += y;
      }
      if (i < E * W) pref[i] = (uint32_t)(x - v);
    }
    __syncthreads();
    if (mine) {
      for (int r = 0; r < k; ++r) {
        if (r >= nr) {
          inv[(size_t)t * k + r] = -1;
          continue;
        }
        int e;
        if (kreg) {
          e = 0;
#pragma unroll
          for (int j = 0; j < PERM_KREG; ++j) e = j == r ? er[j] : e;  // stays in registers
        } else {
          e = rexp[(size_t)t * k + r];
        }
        const int wi = e * W + (tl >> 5);
        const int rank = (int)pref[wi] + __popc(bits[wi] & ((1u << (tl & 31)) - 1u));
        const int pos = base[e] + run[e] + rank;
        inv[(size_t)t * k + r] = pos;
        ptok[pos] = t;
        pslot[pos] = r;
      }
    }
    __syncthreads();
    for (int e = tid; e < E; e += PERM_THREADS)
      run[e] += (int)pref[e * W + W - 1] + __popc(bits[e * W + W - 1]);
    __syncthreads();
  }
}

// The permutation over many workgroups, for larger batches: chunk c (one
// workgroup) holds tokens [32 W c, 32 W c + 32 W).  k_perm_count marks the
// chunk's tokens in one bit row per expert (bit j of row e: token
// 32 W c + j routes to e) and writes the chunk's count per expert.
// k_perm_scatter rebuilds the rows, takes for each expert the sum over all
// chunks (the expert's count) and over the chunks before its own, scans the
// counts into the experts' bases, and places pair (t, r) of expert e at
// base(e) + pairs of e in earlier chunks + set bits of e's row below token
// t: the (token, slot) order of k_permute, so every output is the same.
// Workgroup 0 also writes the counts, offsets, active list and tile lists.
constexpr int PCH_THREADS = 256;
constexpr int PCH_WORDS = 8192;   // LDS words per bit matrix (E W)
constexpr int PCH_MAX_CHUNKS = 64;

// the chunk's bit rows in `bits` (E W words), zeroed first
__device__ __forceinline__ void chunk_bits(const int32_t *__restrict__ rexp,
                                           const int32_t *__restrict__ rcnt, int T, int k, int E,
                                           int W, int t0, uint32_t *bits) {
  const int tid = threadIdx.x;
  for (int i = tid; i < E * W; i += PCH_THREADS) bits[i] = 0;
  __syncthreads();
  const int np = 32 * W * k;
  // four pairs per thread at a time, their loads issued together
  for (int i0 = tid; i0 < np; i0 += 4 * PCH_THREADS) {
    int ev[4], ok[4], tl[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = i0 + j * PCH_THREADS;
      const int l = i / k, r = i - l * k, t = t0 + l;
      const bool in = i < np && t < T;
      tl[j] = l;
      ev[j] = in ? rexp[(size_t)t * k + r] : 0;
      ok[j] = in ? r < rcnt[t] : 0;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (ok[j]) atomicOr(&bits[ev[j] * W + (tl[j] >> 5)], 1u << (tl[j] & 31));
  }
  __syncthreads();
}

__global__ __launch_bounds__(PCH_THREADS) void k_perm_count(const int32_t *__restrict__ rexp,
                                                            const int32_t *__restrict__ rcnt,
                                                            int T, int k, int E, int W,
                                                            int32_t *__restrict__ chunk_cnt) {
  __shared__ uint32_t bits[PCH_WORDS];
  chunk_bits(rexp, rcnt, T, k, E, W, blockIdx.x * 32 * W, bits);
  for (int e = threadIdx.x; e < E; e += PCH_THREADS) {
    int c = 0;
    for (int w = 0; w < W; ++w) c += __popc(bits[e * W + w]);
    chunk_cnt[(size_t)blockIdx.x * E + e] = c;
  }
}

__global__ __launch_bounds__(PCH_THREADS) void k_perm_scatter(
    const int32_t *__restrict__ rexp, const int32_t *__restrict__ rcnt, int T, int k, int E,
    int W, int nch, const int32_t *__restrict__ chunk_cnt, int tile_m,
    int32_t *__restrict__ ecount, int32_t *__restrict__ offsets, int32_t *__restrict__ ptok,
    int32_t *__restrict__ pslot, int32_t *__restrict__ inv, int32_t *__restrict__ active,
    int32_t *__restrict__ tiles, int shared_T, int tile_m2, int32_t *__restrict__ tiles2) {
  __shared__ uint32_t bits[PCH_WORDS];
  __shared__ uint32_t pref[PCH_WORDS];
  __shared__ int base[PERM_THREADS];  // E <= 1024
  __shared__ int wave_tot[PCH_THREADS / 64];
  __shared__ int total;
  const int tid = threadIdx.x, ch = blockIdx.x, t0 = ch * 32 * W;
  // the chunk's pairs, four per thread at a time (pair i0 + 256 j): routes
  // and route counts.  A chunk of at most 1024 pairs is loaded once, before
  // anything else, and kept in registers for the bit rows and the ranks.
  const int np = 32 * W * k;
  const bool onepass = np <= 4 * PCH_THREADS;
  int ev[4], nr[4];
  auto load_pairs = [&](int i0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = i0 + j * PCH_THREADS;
      const int l = i / k, r = i - l * k, t = t0 + l;
      const bool in = i < np && t < T;
      ev[j] = in ? rexp[(size_t)t * k + r] : 0;
      nr[j] = in ? rcnt[t] : 0;
    }
  };
  if (onepass) load_pairs(tid);
  // experts 4 tid .. 4 tid + 3: their counts over all chunks and over the
  // chunks before this one, the loads of 16 chunks issued together (one
  // memory round trip per 16 chunks, not per chunk)
  int tot[4] = {0, 0, 0, 0}, bef[4] = {0, 0, 0, 0};
  constexpr int CB = 16;
  for (int c0 = 0; c0 < nch; c0 += CB) {
    int v[CB][4];
#pragma unroll
    for (int u = 0; u < CB; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int c = c0 + u, e = 4 * tid + j;
        v[u][j] = c < nch && e < E ? chunk_cnt[(size_t)c * E + e] : 0;
      }
#pragma unroll
    for (int u = 0; u < CB; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        tot[j] += v[u][j];
        bef[j] += c0 + u < ch ? v[u][j] : 0;
      }
  }
  const int sum4 = tot[0] + tot[1] + tot[2] + tot[3];
  const int b = block_exclusive_scan(sum4, wave_tot, &total);
  const int npairs = total;
  {
    int eb = b;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = 4 * tid + j;
      if (e < E) {
        base[e] = eb + bef[j];
        if (ch == 0) {
          ecount[e] = tot[j];
          offsets[e] = eb;
        }
      }
      eb += tot[j];
    }
  }
  if (ch == 0) {  // workgroup-uniform
    if (tid == 0) offsets[E] = npairs;
    int na = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) na += (4 * tid + j < E && tot[j] > 0) ? 1 : 0;
    int a = block_exclusive_scan(na, wave_tot, &total);
    const int n_active = total;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (4 * tid + j < E && tot[j] > 0) active[a++] = 4 * tid + j;
    if (tid == 0) active[E] = n_active;
    // tile lists: (expert, first row) per tm rows, the shared expert's last
    auto tile_list = [&](int tm, int32_t *out) {
      int nt4 = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) nt4 += 4 * tid + j < E ? (tot[j] + tm - 1) / tm : 0;
      int tb = block_exclusive_scan(nt4, wave_tot, &total);
      const int ntiles = total;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int e = 4 * tid + j;
        const int nt = e < E ? (tot[j] + tm - 1) / tm : 0;
        for (int q = 0; q < nt; ++q, ++tb) {
          out[2 + 2 * tb] = e;
          out[2 + 2 * tb + 1] = q * tm;
        }
      }
      const int nshared = (shared_T + tm - 1) / tm;
      for (int q = tid; q < nshared; q += PCH_THREADS) {
        out[2 + 2 * (ntiles + q)] = E;
        out[2 + 2 * (ntiles + q) + 1] = q * tm;
      }
      if (tid == 0) {
        out[0] = ntiles + nshared;
        out[1] = 0;
      }
    };
    if (tiles != nullptr) tile_list(tile_m, tiles);
    if (tiles2 != nullptr) tile_list(tile_m2, tiles2);
  }
  for (int i = tid; i < E * W; i += PCH_THREADS) bits[i] = 0;
  __syncthreads();  // (also orders base[] before the ranks)
  for (int i0 = tid; i0 < np; i0 += 4 * PCH_THREADS) {
    if (!onepass) load_pairs(i0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = i0 + j * PCH_THREADS;
      const int l = i / k, r = i - l * k;
      if (i < np && t0 + l < T && r < nr[j])
        atomicOr(&bits[ev[j] * W + (l >> 5)], 1u << (l & 31));
    }
  }
  __syncthreads();
  // pref[e W + w] = set bits of row e's words 0 .. w-1 (W consecutive lanes
  // hold a row, scanned with shuffles)
  for (int i0 = 0; i0 < E * W; i0 += PCH_THREADS) {
    const int i = i0 + tid;
    const int v = i < E * W ? __popc(bits[i]) : 0;
    int x = v;
    for (int d = 1; d < W; d <<= 1) {
      const int y = __shfl_up(x, d, W);
      if ((tid & (W - 1)) >= d) x += y;
    }
    if (i < E * W) pref[i] = (uint32_t)(x - v);
  }
  __syncthreads();
  for (int i0 = tid; i0 < np; i0 += 4 * PCH_THREADS) {
    if (!onepass) load_pairs(i0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = i0 + j * PCH_THREADS;
      const int l = i / k, r = i - l * k, t = t0 + l;
      if (i >= np || t >= T) continue;
      const size_t ix = (size_t)t * k + r;
      if (r >= nr[j]) {
        inv[ix] = -1;
        continue;
      }
      const int e = ev[j];
      const int wi = e * W + (l >> 5);
      const int pos = base[e] + (int)pref[wi] + __popc(bits[wi] & ((1u << (l & 31)) - 1u));
      inv[ix] = pos;
      ptok[pos] = t;
      pslot[pos] = r;
    }
  }
}

// Router and permutation in one workgroup for small batches (T <= 32,
// T*k <= 512, E <= 256): each of the 16 waves routes tokens wave,
// wave + 16; each valid pair (token t, slot r), i = t k + r, sets bit i of its expert's row
// of a bit matrix; thread e counts expert e's pairs, the workgroup scans the
// counts, and pair i's position within its expert is the number of bits
// below bit i in that row — the (token, slot) order of k_permute.
// tiles (optional): the tile list of k_permute, tile_m pairs per tile.
constexpr int RP_MAX_PAIRS = 512;
constexpr int RP_THREADS = 1024;
constexpr int RP_WORDS = RP_MAX_PAIRS / 32;  // bit-matrix words per expert

template <int EPL>
__global__ __launch_bounds__(RP_THREADS) void k_route_permute(
    const float *__restrict__ logits, int T, int E, int k, int score_mode,
    int32_t *__restrict__ rexp, float *__restrict__ rw, int32_t *__restrict__ rcnt,
    int32_t *__restrict__ ecount, int32_t *__restrict__ offsets, int32_t *__restrict__ ptok,
    int32_t *__restrict__ pslot, int32_t *__restrict__ inv, int32_t *__restrict__ active,
    int tile_m, int32_t *__restrict__ tiles, int *__restrict__ counters, int n_counters) {
  __shared__ int s_exp[RP_MAX_PAIRS];
  __shared__ int s_cnt[RP_MAX_PAIRS];
  __shared__ int s_base[256];
  __shared__ uint32_t s_bits[256 * RP_WORDS];
  __shared__ int wave_tot[RP_THREADS / 64];
  __shared__ int total;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < n_counters; i += RP_THREADS) counters[i] = 0;
  for (int i = tid; i < E * RP_WORDS; i += RP_THREADS) s_bits[i] = 0;
  for (int t = wave; t < T; t += RP_THREADS / 64) {
    int e, n;
    float w;
    route_one<EPL>(logits + (size_t)t * E, E, k, score_mode, lane, &e, &w, &n);
    if (lane < k) {
      rexp[(size_t)t * k + lane] = e;
      rw[(size_t)t * k + lane] = w;
      s_exp[t * k + lane] = e;
    }
    if (lane == 0) {
      rcnt[t] = n;
      s_cnt[t] = n;
    }
  }
  __syncthreads();
  const int pairs = T * k;
  const int pt = tid / k, pr = tid - pt * k;  // pair tid = (token, slot)
  const bool pvalid = tid < pairs && pr < s_cnt[pt];
  const int pe = pvalid ? s_exp[tid] : 0;
  if (pvalid) atomicOr(&s_bits[pe * RP_WORDS + (tid >> 5)], 1u << (tid & 31));
  __syncthreads();
  int c = 0;
  if (tid < E) {
#pragma unroll
    for (int w = 0; w < RP_WORDS; ++w) c += __popc(s_bits[tid * RP_WORDS + w]);
  }
  const int b = block_exclusive_scan(c, wave_tot, &total);
  const int npairs = total;
  const int act = block_exclusive_scan(tid < E && c > 0 ? 1 : 0, wave_tot, &total);
  const int n_active = total;
  if (tid < E) {
    ecount[tid] = c;
    offsets[tid] = b;
    s_base[tid] = b;
    if (c > 0) active[act] = tid;
  }
  if (tiles != nullptr) {
    const int nt = tid < E ? (c + tile_m - 1) / tile_m : 0;
    const int tb = block_exclusive_scan(nt, wave_tot, &total);
    for (int j = 0; j < nt; ++j) {
      tiles[2 + 2 * (tb + j)] = tid;
      tiles[2 + 2 * (tb + j) + 1] = j * tile_m;
    }
    if (tid == 0) {
      tiles[0] = total;
      tiles[1] = 0;
    }
  }
  if (tid == 0) {
    offsets[E] = npairs;
    active[E] = n_active;
  }
  __syncthreads();
  if (tid < pairs) {
    int pos = -1;
    if (pvalid) {
      const uint32_t *row = s_bits + pe * RP_WORDS;
      const int wi = tid >> 5;
      int rank = __popc(row[wi] & ((1u << (tid & 31)) - 1u));
      for (int w = 0; w < wi; ++w) rank += __popc(row[w]);
      pos = s_base[pe] + rank;
      ptok[pos] = pt;
      pslot[pos] = pr;
    }
    inv[tid] = pos;
  }
}

// per-pair row elements: f32, or bf16 (the upper half of an f32, exact)
__device__ __forceinline__ float yval(const float *__restrict__ y, size_t o) { return y[o]; }
__device__ __forceinline__ float yval(const uint16_t *__restrict__ y, size_t o) {
  return __uint_as_float((uint32_t)y[o] << 16);
}
__device__ __forceinline__ float4 yval4(const float *__restrict__ y, size_t o) {
  return *reinterpret_cast<const float4 *>(y + o);
}
__device__ __forceinline__ float4 yval4(const uint16_t *__restrict__ y, size_t o) {
  const uint2 u = *reinterpret_cast<const uint2 *>(y + o);
  return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                     __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u));
}

// y value at offset o: the sum of the ns partial buffers (K splits) in
// split order.  NS == 1: one buffer.  Otherwise the buffers are read 8 at a
// time (indices past the last clamped to it), so a run of loads is in flight
// together instead of one dependent load per buffer.
template <int NS, typename YT>
__device__ __forceinline__ float y_at(const YT *__restrict__ y, size_t stride, int ns, size_t o) {
  if constexpr (NS == 1) {
    return yval(y, o);
  } else {
    float v = 0.f;
    for (int s0 = 0; s0 < ns; s0 += 8) {
      float u[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) u[j] = yval(y, (size_t)min(s0 + j, ns - 1) * stride + o);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (s0 + j < ns) v = s0 + j == 0 ? u[j] : v + u[j];
    }
    return v;
  }
}

// out[t] = sum_r w[t,r] * y[pair(t,r)] (+ shared) in route order
// (src/engine/mod.rs:1017-1021).  The routes' pair indices and weights are
// read RB at a time (clamped to the last slot, k - 1) together with the
// route count, then their y values, so a token's loads take two dependent
// rounds and the routes' loads overlap.  inv == nullptr: the y rows are
// stored in route order (route r of token t at row t * k + r, as the
// one-token decode GEMV writes them), so every load of the token is issued
// at once and the rows of absent routes are read but not used.
template <int NS, int RB, typename YT>
__global__ __launch_bounds__(256) void k_combine(const YT *__restrict__ ypair,
                                                 const float *__restrict__ rw,
                                                 const int32_t *__restrict__ rcnt,
                                                 const int32_t *__restrict__ inv, int T, int k,
                                                 int H, int shared, float *out,
                                                 int ns, size_t stride, const float *residual) {
  const size_t total = (size_t)T * H;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const int t = (int)(i / H), h = (int)(i - (size_t)t * H);
    const float sh = shared ? y_at<NS>(ypair, stride, ns, ((size_t)T * k + t) * H + h) : 0.f;
    float acc = 0.0f;
    int n = k;  // the route count arrives with the first batch of routes
    for (int r0 = 0; r0 < n; r0 += RB) {
      int p[RB];
      float w[RB], yv[RB];
      if (r0 == 0) n = rcnt[t];
#pragma unroll
      for (int j = 0; j < RB; ++j) {
        const size_t r = (size_t)t * k + min(r0 + j, k - 1);
        p[j] = inv ? inv[r] : (int)r;
        w[j] = rw[r];
      }
#pragma unroll
      for (int j = 0; j < RB; ++j)
        yv[j] = (!inv || r0 + j < n) ? y_at<NS>(ypair, stride, ns, (size_t)p[j] * H + h) : 0.f;
#pragma unroll
      for (int j = 0; j < RB; ++j)
        if (r0 + j < n) acc = acc + __fmul_rn(w[j], yv[j]);
    }
    if (shared) acc = acc + sh;
    out[i] = residual ? residual[i] + acc : acc;
  }
}

// c ? a : b per component (a select of whole float4 values can become a
// select of their addresses, with the values in scratch memory)
__device__ __forceinline__ float4 sel4(bool c, const float4 &a, const float4 &b) {
  return make_float4(c ? a.x : b.x, c ? a.y : b.y, c ? a.z : b.z, c ? a.w : b.w);
}

// Slice sums of R rows of four consecutive columns at once (rows with
// use[r] false are not read and sum to zero): every used row's first SB
// slices are loaded (those past the last slice clamped to it: cache hits, no
// branches) before any is added, so with at most SB slices all the rows take
// one round of loads; the sums are selects, not branches, so nothing waits
// between the rows.  Per row the same additions in slice order as y_at.
template <int R, int SB, typename YT>
__device__ __forceinline__ void y4_rows(const YT *__restrict__ y, size_t stride, int ns,
                                        const size_t (&o)[R], const bool (&use)[R],
                                        float4 (&v)[R]) {
#pragma unroll
  for (int r = 0; r < R; ++r) v[r] = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s0 = 0; s0 < ns; s0 += SB) {
    float4 u[R][SB];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (use[r]) {
#pragma unroll
        for (int j = 0; j < SB; ++j)
          u[r][j] = yval4(y, (size_t)min(s0 + j, ns - 1) * stride + o[r]);
      } else {
#pragma unroll
        for (int j = 0; j < SB; ++j) u[r][j] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int j = 0; j < SB; ++j) {
        const float4 a = v[r], b = u[r][j];
        const float4 sum = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
        if (j == 0)  // slice s0 < ns always
          v[r] = sel4(s0 == 0, b, sum);
        else
          v[r] = sel4(s0 + j < ns, sum, a);
      }
  }
}

// k_combine with the token's routes read once per workgroup: workgroup
// blockIdx.x covers 4 * blockDim.x columns (four per thread, float4 stores)
// of token blockIdx.x / nchunk, so the token's count, pair indices and
// weights are workgroup-uniform loads and no thread divides its index by H.
// (Whole rows per workgroup, with the route loads paid once per token,
// measured slower at 2048-4096 tokens: the chunks' parallelism matters
// more.)  The residual is loaded with the routes' indices; with K slices
// (NS == 0) a batch's routes and the shared row load their slices together
// (up to SB slices in one round: two rounds of dependent loads in all, where
// a row at a time took one per route and batch of slices).  Per element the
// same operations in the same order as k_combine.  Requires H % 4 == 0,
// 16-byte aligned out and residual, and ypair aligned to four of its
// elements.
template <int NS, int RB, int SB, typename YT>
__global__ __launch_bounds__(256) void k_combine4(const YT *__restrict__ ypair,
                                                  const float *__restrict__ rw,
                                                  const int32_t *__restrict__ rcnt,
                                                  const int32_t *__restrict__ inv, int T, int k,
                                                  int H, int shared, float *out, int ns,
                                                  size_t stride, const float *residual,
                                                  int nchunk) {
  static_assert(NS == 1 || (RB + 1) * SB <= 40, "slice batch too large for registers");
  const int t = (int)(blockIdx.x / (unsigned)nchunk);
  const int c4 = (int)(blockIdx.x - (unsigned)t * (unsigned)nchunk) * (int)blockDim.x +
                 (int)threadIdx.x;
  if (4 * c4 >= H) return;
  const size_t col = 4 * (size_t)c4;
  const size_t i = (size_t)t * H + col;
  const size_t sh_off = ((size_t)T * k + t) * H + col;
  const float4 rv = residual ? *reinterpret_cast<const float4 *>(residual + i)
                             : make_float4(0.f, 0.f, 0.f, 0.f);
  float4 sh = (NS == 1 && shared) ? yval4(ypair, sh_off) : make_float4(0.f, 0.f, 0.f, 0.f);
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  int n = k;  // the route count arrives with the first batch of routes
  for (int r0 = 0; r0 < n; r0 += RB) {
    int p[RB];
    float w[RB];
    float4 yv[RB];
    if (r0 == 0) n = rcnt[t];
#pragma unroll
    for (int j = 0; j < RB; ++j) {
      const size_t r = (size_t)t * k + min(r0 + j, k - 1);
      p[j] = inv ? inv[r] : (int)r;
      w[j] = rw[r];
    }
    if constexpr (NS == 0) {
      size_t o[RB + 1];  // the routes, then the shared row
      bool use[RB + 1];
      float4 v[RB + 1];
#pragma unroll
      for (int j = 0; j < RB; ++j) {
        o[j] = (size_t)p[j] * H + col;
        use[j] = !inv || r0 + j < n;
      }
      o[RB] = sh_off;
      use[RB] = shared && r0 == 0;
      y4_rows<RB + 1, SB>(ypair, stride, ns, o, use, v);
#pragma unroll
      for (int j = 0; j < RB; ++j) yv[j] = v[j];
      if (r0 == 0) sh = v[RB];
    } else {
#pragma unroll
      for (int j = 0; j < RB; ++j)
        yv[j] = (!inv || r0 + j < n) ? yval4(ypair, (size_t)p[j] * H + col)
                                     : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int j = 0; j < RB; ++j)
      if (r0 + j < n) {
        acc.x = acc.x + __fmul_rn(w[j], yv[j].x);
        acc.y = acc.y + __fmul_rn(w[j], yv[j].y);
        acc.z = acc.z + __fmul_rn(w[j], yv[j].z);
        acc.w = acc.w + __fmul_rn(w[j], yv[j].w);
      }
  }
  if (shared) {
    acc.x = acc.x + sh.x;
    acc.y = acc.y + sh.y;
    acc.z = acc.z + sh.z;
    acc.w = acc.w + sh.w;
  }
  if (residual) {
    acc.x = rv.x + acc.x;
    acc.y = rv.y + acc.y;
    acc.z = rv.z + acc.z;
    acc.w = rv.w + acc.w;
  }
  *reinterpret_cast<float4 *>(out + i) = acc;
}

// k_combine4 for bf16 rows without K splits, eight columns per thread: one
// 16-byte load per route (eight bf16, widened exactly) and two float4
// stores, so a wave moves 1 KB per route load instead of 512 bytes.  Per
// element the same operations in the same order as k_combine.  Requires
// H % 8 == 0, 16-byte aligned out, residual and ypair.
__device__ __forceinline__ void bf16x8(const uint16_t *__restrict__ y, size_t o, float4 &a,
                                       float4 &b) {
  const uint4 u = *reinterpret_cast<const uint4 *>(y + o);
  a = make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                  __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u));
  b = make_float4(__uint_as_float(u.z << 16), __uint_as_float(u.z & 0xffff0000u),
                  __uint_as_float(u.w << 16), __uint_as_float(u.w & 0xffff0000u));
}
__device__ __forceinline__ void fma_add4(float4 &acc, float w, const float4 &y) {
  acc.x = acc.x + __fmul_rn(w, y.x);
  acc.y = acc.y + __fmul_rn(w, y.y);
  acc.z = acc.z + __fmul_rn(w, y.z);
  acc.w = acc.w + __fmul_rn(w, y.w);
}
__device__ __forceinline__ void add4(float4 &acc, const float4 &y) {
  acc.x = acc.x + y.x;
  acc.y = acc.y + y.y;
  acc.z = acc.z + y.z;
  acc.w = acc.w + y.w;
}
__device__ __forceinline__ void radd4(float4 &acc, const float4 &r) {  // residual first
  acc.x = r.x + acc.x;
  acc.y = r.y + acc.y;
  acc.z = r.z + acc.z;
  acc.w = r.w + acc.w;
}
// Slice sums of R bf16 rows of eight consecutive columns, as y4_rows (every
// used row's first SB slices loaded before any is added, slices past the
// last clamped to it, the sums in slice order): v0 the first four columns,
// v1 the last four.
template <int R, int SB>
__device__ __forceinline__ void y8_rows(const uint16_t *__restrict__ y, size_t stride, int ns,
                                        const size_t (&o)[R], const bool (&use)[R],
                                        float4 (&v0)[R], float4 (&v1)[R]) {
  const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int r = 0; r < R; ++r) v0[r] = v1[r] = z;
  for (int s0 = 0; s0 < ns; s0 += SB) {
    // raw words, widened only when added (values, not references: the
    // arrays stay in registers)
    uint4 u[R][SB];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (use[r]) {
#pragma unroll
        for (int j = 0; j < SB; ++j)
          u[r][j] = *reinterpret_cast<const uint4 *>(y + (size_t)min(s0 + j, ns - 1) * stride + o[r]);
      } else {
#pragma unroll
        for (int j = 0; j < SB; ++j) u[r][j] = make_uint4(0u, 0u, 0u, 0u);
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int j = 0; j < SB; ++j) {
        const uint4 w = u[r][j];
        const float4 b0 = make_float4(__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u),
                                      __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xffff0000u));
        const float4 b1 = make_float4(__uint_as_float(w.z << 16), __uint_as_float(w.z & 0xffff0000u),
                                      __uint_as_float(w.w << 16), __uint_as_float(w.w & 0xffff0000u));
        float4 a0 = v0[r], a1 = v1[r];
        add4(a0, b0);
        add4(a1, b1);
        if (j == 0) {  // slice s0 < ns always
          v0[r] = sel4(s0 == 0, b0, a0);
          v1[r] = sel4(s0 == 0, b1, a1);
        } else {
          v0[r] = sel4(s0 + j < ns, a0, v0[r]);
          v1[r] = sel4(s0 + j < ns, a1, v1[r]);
        }
      }
  }
}

// k_combine4 for bf16 rows, eight columns per thread: one 16-byte load per
// route row (and K slice) and two float4 stores, so a wave moves 1 KB per
// load instead of 512 bytes.  With K slices (NS == 0) a batch's routes and
// the shared row load their first SB slices together, as in k_combine4.
// Per element the same operations in the same order as k_combine.
// Requires H % 8 == 0, 16-byte aligned out, residual and ypair.
template <int NS, int RB, int SB>
__global__ __launch_bounds__(256) void k_combine8(const uint16_t *__restrict__ ypair,
                                                  const float *__restrict__ rw,
                                                  const int32_t *__restrict__ rcnt,
                                                  const int32_t *__restrict__ inv, int T, int k,
                                                  int H, int shared, float *out, int ns,
                                                  size_t stride, const float *residual,
                                                  int nchunk) {
  static_assert(NS == 1 || (RB + 1) * SB <= 20, "slice batch too large for registers");
  const int t = (int)(blockIdx.x / (unsigned)nchunk);
  const int c8 = (int)(blockIdx.x - (unsigned)t * (unsigned)nchunk) * (int)blockDim.x +
                 (int)threadIdx.x;
  if (8 * c8 >= H) return;
  const size_t col = 8 * (size_t)c8;
  const size_t i = (size_t)t * H + col;
  const size_t sh_off = ((size_t)T * k + t) * H + col;
  const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
  float4 r0v = z, r1v = z, sh0 = z, sh1 = z;
  if (residual) {
    r0v = *reinterpret_cast<const float4 *>(residual + i);
    r1v = *reinterpret_cast<const float4 *>(residual + i + 4);
  }
  if (NS == 1 && shared) bf16x8(ypair, sh_off, sh0, sh1);
  float4 acc0 = z, acc1 = z;
  int n = k;  // the route count arrives with the first batch of routes
  for (int r0 = 0; r0 < n; r0 += RB) {
    int p[RB];
    float w[RB];
    float4 y0[RB], y1[RB];
    if (r0 == 0) n = rcnt[t];
#pragma unroll
    for (int j = 0; j < RB; ++j) {
      const size_t r = (size_t)t * k + min(r0 + j, k - 1);
      p[j] = inv ? inv[r] : (int)r;
      w[j] = rw[r];
    }
    if constexpr (NS == 0) {
      size_t o[RB + 1];  // the routes, then the shared row
      bool use[RB + 1];
      float4 v0[RB + 1], v1[RB + 1];
#pragma unroll
      for (int j = 0; j < RB; ++j) {
        o[j] = (size_t)p[j] * H + col;
        use[j] = !inv || r0 + j < n;
      }
      o[RB] = sh_off;
      use[RB] = shared && r0 == 0;
      y8_rows<RB + 1, SB>(ypair, stride, ns, o, use, v0, v1);
#pragma unroll
      for (int j = 0; j < RB; ++j) {
        y0[j] = v0[j];
        y1[j] = v1[j];
      }
      if (r0 == 0) {
        sh0 = v0[RB];
        sh1 = v1[RB];
      }
    } else {
#pragma unroll
      for (int j = 0; j < RB; ++j) {
        y0[j] = z;
        y1[j] = z;
        if (!inv || r0 + j < n) bf16x8(ypair, (size_t)p[j] * H + col, y0[j], y1[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < RB; ++j)
      if (r0 + j < n) {
        fma_add4(acc0, w[j], y0[j]);
        fma_add4(acc1, w[j], y1[j]);
      }
  }
  if (shared) {
    add4(acc0, sh0);
    add4(acc1, sh1);
  }
  if (residual) {
    radd4(acc0, r0v);
    radd4(acc1, r1v);
  }
  *reinterpret_cast<float4 *>(out + i) = acc0;
  *reinterpret_cast<float4 *>(out + i + 4) = acc1;
}

}  // namespace

int launch_route(nx_ctx *c, const float *d_logits, int T, int E, int k, int score_mode,
                 int32_t *d_expert, float *d_weight, int32_t *d_count) {
  if (T <= 0) return NX_OK;
  if (E > 1024) return fail(NX_ERR_UNSUPPORTED, "router supports at most 1024 experts");
  if (k > 64) return fail(NX_ERR_UNSUPPORTED, "router supports top_k <= 64");
  const unsigned g = (unsigned)((T + 3) / 4);
  const int epl = (E + 63) / 64;
#define NX_ROUTE(N)                                                                        \
  return launch(c, "route_topk", [&] {                                                     \
    go(c, k_route<N>, dim3(g), dim3(256), 0, d_logits, T, E, k, score_mode, d_expert, d_weight, \
                                         d_count);                                          \
  })
  if (epl <= 1) NX_ROUTE(1);
  if (epl <= 2) NX_ROUTE(2);
  if (epl <= 4) NX_ROUTE(4);
  if (epl <= 8) NX_ROUTE(8);
  NX_ROUTE(16);
#undef NX_ROUTE
}

int launch_permute(nx_ctx *c, const int32_t *d_expert, const int32_t *d_count, int T, int k,
                   int E, int tile_m, int32_t *d_ecount, int32_t *d_offsets, int32_t *d_ptok,
                   int32_t *d_pslot, int32_t *d_inv, int32_t *d_active, int32_t *d_tiles,
                   int shared_T, int tile_m2, int32_t *d_tiles2) {
  if (E > PERM_THREADS) return fail(NX_ERR_UNSUPPORTED, "permutation supports at most 1024 experts");
  int W = PERM_WORDS / (E > 0 ? E : 1);
  if (W > PERM_THREADS / 32) W = PERM_THREADS / 32;
  if (W < 1) W = 1;
  while (W & (W - 1)) W &= W - 1;  // a power of two: rows are scanned within a wave
  // Large batches: one workgroup per chunk of 32 Wc tokens (Wc the smallest
  // power of two from 2 that gives at most 64 chunks), two launches.  Below
  // 4096 pairs, and with few experts up to two of the single workgroup's
  // chunks, the one launch is as fast or faster (measured, us: Mixtral
  // 256 / 2048 tokens 7.6 / 14.3 against 13.0 / 16.6; Qwen3 128 tokens 11.8
  // against 13.8; Qwen3 512 tokens 16.2 against 13.7; DeepSeek 4096 tokens
  // 82.8 against 20.0).
  const int one_wg_chunks = (T + 32 * W - 1) / (32 * W);
  if ((long)T * k >= 4096 && E > 0 && (E >= 64 || one_wg_chunks >= 3)) {
    int Wc = 2;
    while (Wc < 32 && (T + 32 * Wc - 1) / (32 * Wc) > PCH_MAX_CHUNKS && E * 2 * Wc <= PCH_WORDS)
      Wc *= 2;
    const int nch = (T + 32 * Wc - 1) / (32 * Wc);
    if (E * Wc <= PCH_WORDS && nch <= PCH_MAX_CHUNKS) {
      void *vcc;
      NX_TRY(ws_get(c, WS_PERM_CHUNK, (size_t)nch * E * sizeof(int32_t), &vcc));
      int32_t *d_cc = static_cast<int32_t *>(vcc);
      NX_TRY(launch(c, "permute_count", [&] {
        go(c, k_perm_count, dim3(nch), dim3(PCH_THREADS), 0, d_expert, d_count, T, k, E, Wc, d_cc);
      }));
      return launch(c, "permute", [&] {
        go(c, k_perm_scatter, dim3(nch), dim3(PCH_THREADS), 0, d_expert, d_count, T, k, E, Wc,
           nch, (const int32_t *)d_cc, tile_m > 0 ? tile_m : 1, d_ecount, d_offsets, d_ptok,
           d_pslot, d_inv, d_active, d_tiles, shared_T, tile_m2 > 0 ? tile_m2 : 1, d_tiles2);
      });
    }
  }
  return launch(c, "permute", [&] {
    go(c, k_permute, dim3(1), dim3(PERM_THREADS), 0, d_expert, d_count, T, k, E, W,
                                                 tile_m > 0 ? tile_m : 1, d_ecount, d_offsets,
                                                 d_ptok, d_pslot, d_inv, d_active, d_tiles,
                                                 shared_T, tile_m2 > 0 ? tile_m2 : 1, d_tiles2);
  });
}

#ifndef NX_RP_TOKENS_PER_WAVE
#define NX_RP_TOKENS_PER_WAVE 2
#endif
bool route_permute_fusable(int T, int E, int k) {
  // each wave routes its tokens one after another: beyond a few per wave the
  // router kernel, spread over the chip, is faster
  return T >= 1 && T <= NX_RP_TOKENS_PER_WAVE * (RP_THREADS / 64) &&
         (long)T * k <= RP_MAX_PAIRS && E <= 256 && k <= 64;
}

int launch_route_permute(nx_ctx *c, const float *d_logits, int T, int E, int k, int score_mode,
                         int32_t *d_expert, float *d_weight, int32_t *d_count, int32_t *d_ecount,
                         int32_t *d_offsets, int32_t *d_ptok, int32_t *d_pslot, int32_t *d_inv,
                         int32_t *d_active, int tile_m, int32_t *d_tiles, int *d_counters,
                         int n_counters) {
  if (!route_permute_fusable(T, E, k)) return fail(NX_ERR_UNSUPPORTED, "batch too large for the fused router");
  const int epl = (E + 63) / 64;
  const int nc = d_counters ? n_counters : 0;
  const int tm = tile_m > 0 ? tile_m : 1;
#define NX_RP(N)                                                                              \
  return launch(c, "route_permute", [&] {                                                     \
    go(c, k_route_permute<N>, dim3(1), dim3(RP_THREADS), 0, d_logits, T, E, k, score_mode, d_expert, \
                                                        d_weight, d_count, d_ecount, d_offsets,  \
                                                        d_ptok, d_pslot, d_inv, d_active, tm,    \
                                                        d_tiles, d_counters, nc);                \
  })
  if (epl <= 1) NX_RP(1);
  if (epl <= 2) NX_RP(2);
  NX_RP(4);
#undef NX_RP
}

namespace {
template <typename YT>
int combine_rows(nx_ctx *c, const YT *d_ypair, const float *d_weight, const int32_t *d_count,
                 const int32_t *d_inv, int T, int k, int H, bool shared, float *d_out, int nsplit,
                 size_t split_stride, const float *d_residual) {
  const size_t total = (size_t)T * H;
  if (total == 0) return NX_OK;
  const int ns = nsplit > 1 ? nsplit : 1;
  const int sh = shared ? 1 : 0;
  auto al16 = [](const void *q) { return ((uintptr_t)q & 15u) == 0; };
  const bool y_al = ((uintptr_t)d_ypair & (4 * sizeof(YT) - 1)) == 0;
  // Workgroups of 256 threads (1024 columns).  With K slices (a thread's
  // loads are the slices of every route) and fewer than two such workgroups
  // per CU: 128 or 64 threads, so a few tokens' rows spread over more CUs
  // (measured, Mixtral 32 tokens 19 slices: 7.1 -> 6.9 us; not with one
  // slice, where a token's 2048 columns on 8 workgroups took longer than on 2).
  int tpb = 256;
  while (ns > 1 && tpb > 64 && (long)T * ((H / 4 + tpb - 1) / tpb) < 2L * c->num_cu) tpb /= 2;
  if constexpr (std::is_same<YT, uint16_t>::value) {
    // bf16 rows (the grouped GEMM's down pass, up to 4 K splits): eight
    // columns per thread; workgroups of 128 threads when a row's eighths
    // fill those and not 256 (DeepSeek's 7168 columns: 7 of 128, not 4 of
    // 256 with one half idle)
    if (ns <= 4 && H % 8 == 0 && al16(d_ypair) && al16(d_out) && al16(d_residual)) {
      const int t8 = (H / 8) % 256 && (H / 8) % 128 == 0 ? 128 : 256;
      const int nch8 = (H / 8 + t8 - 1) / t8;
      if ((size_t)T * nch8 < (1u << 31)) {
        auto run8 = [&](auto kern) {
          return launch(c, "combine", [&] {
            go(c, kern, dim3((unsigned)(T * nch8)), dim3((unsigned)t8), 0, d_ypair, d_weight,
               d_count, d_inv, T, k, H, sh, d_out, ns, split_stride, d_residual, nch8);
          });
        };
        if (ns == 1) {
          if (k <= 2) return run8(k_combine8<1, 2, 1>);
          if (k <= 4) return run8(k_combine8<1, 4, 1>);
          return run8(k_combine8<1, 8, 1>);
        }
        if (k <= 2) return ns <= 2 ? run8(k_combine8<0, 2, 2>) : run8(k_combine8<0, 2, 4>);
        if (k <= 4) return ns <= 2 ? run8(k_combine8<0, 4, 2>) : run8(k_combine8<0, 4, 4>);
        return run8(k_combine8<0, 8, 2>);  // two slices per round
      }
    }
  }
  const int nchunk = (H / 4 + tpb - 1) / tpb;
  if (H % 4 == 0 && y_al && al16(d_out) && al16(d_residual) &&
      (size_t)T * nchunk < (1u << 31)) {
    auto run4 = [&](auto kern) {
      return launch(c, "combine", [&] {
        go(c, kern, dim3((unsigned)(T * nchunk)), dim3((unsigned)tpb), 0, d_ypair, d_weight,
           d_count, d_inv, T, k, H, sh, d_out, ns, split_stride, d_residual, nchunk);
      });
    };
    if (ns == 1) {
      if (k <= 2) return run4(k_combine4<1, 2, 8, YT>);
      if (k <= 4) return run4(k_combine4<1, 4, 8, YT>);
      return run4(k_combine4<1, 8, 8, YT>);
    }
    // slices loaded 2, 4 or 8 at a time, the fewest that cover the slice
    // count (at most 4 for more than 4 routes): a wider batch than the
    // slices only repeats the last slice's loads and costs registers
    // (Mixtral prefill, 2 K splits of bf16 rows, 8 at a time: 29 -> 46 us).
    // 24 at a time for Mixtral's 19 slices measured slower (7.5 against
    // 7.1 us: the registers halve the waves per SIMD).
    if (k <= 2) {
      if (ns <= 2) return run4(k_combine4<0, 2, 2, YT>);
      if (ns <= 4) return run4(k_combine4<0, 2, 4, YT>);
      return run4(k_combine4<0, 2, 8, YT>);
    }
    if (k <= 4) {
      if (ns <= 2) return run4(k_combine4<0, 4, 2, YT>);
      if (ns <= 4) return run4(k_combine4<0, 4, 4, YT>);
      return run4(k_combine4<0, 4, 8, YT>);
    }
    if (ns <= 2) return run4(k_combine4<0, 8, 2, YT>);
    return run4(k_combine4<0, 8, 4, YT>);
  }
  size_t g = (total + 255) / 256;
  if (g > 65536) g = 65536;
  auto run1 = [&](auto kern) {
    return launch(c, "combine", [&] {
      go(c, kern, dim3((unsigned)g), dim3(256), 0, d_ypair, d_weight, d_count, d_inv, T, k, H, sh,
                                               d_out, ns, split_stride, d_residual);
    });
  };
  // routes read together: top-k up to 2, 4, else 8 at a time
  if (ns == 1) {
    if (k <= 2) return run1(k_combine<1, 2, YT>);
    if (k <= 4) return run1(k_combine<1, 4, YT>);
    return run1(k_combine<1, 8, YT>);
  }
  if (k <= 2) return run1(k_combine<0, 2, YT>);
  if (k <= 4) return run1(k_combine<0, 4, YT>);
  return run1(k_combine<0, 8, YT>);
}

}  // namespace

int launch_combine(nx_ctx *c, const float *d_ypair, const float *d_weight, const int32_t *d_count,
                   const int32_t *d_inv, int T, int k, int H, bool shared, float *d_out,
                   int nsplit, size_t split_stride, const float *d_residual) {
  return combine_rows(c, d_ypair, d_weight, d_count, d_inv, T, k, H, shared, d_out, nsplit,
                      split_stride, d_residual);
}

int launch_combine_bf16(nx_ctx *c, const uint16_t *d_ypair, const float *d_weight,
                        const int32_t *d_count, const int32_t *d_inv, int T, int k, int H,
                        bool shared, float *d_out, int nsplit, size_t split_stride,
                        const float *d_residual) {
  return combine_rows(c, d_ypair, d_weight, d_count, d_inv, T, k, H, shared, d_out, nsplit,
                      split_stride, d_residual);
}

}  // namespace nx
