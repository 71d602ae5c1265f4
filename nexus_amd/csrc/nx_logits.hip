// nx_logits.hip — router logits on gfx950: logits[t][e] = sum_c W[e][c] * x[t][c].
//
// The reference computes router logits with its host matvec
// (InferenceEngine::matvec, src/engine/mod.rs:775-801): per output, sum starts
// at 0.0f and for col in 0..cols adds weight * input, the product rounded to
// f32 and then the sum rounded to f32 (Rust never fuses a*b+c into an fma).
// Top-k routing compares those logits exactly, ties going to the lower
// expert, so a device router that must pick the same experts as the reference
// has to reproduce that order to the last bit.
//
// Exact mode does: every (token, expert) pair is one sequential chain over
// the columns, with separately rounded products and sums (contraction is off
// in every kernel here; fast mode asks for fma explicitly).  A sum that
// starts at +0.0 is never -0.0, so adding +0.0 products for columns past the
// row end (loads out of range return zeros) leaves it unchanged.
//
// Fast mode sums in a parallel order with fma: the result differs from the
// exact one by at most 2 (H+1) 2^-24 sum_c |W[e][c] x[t][c]| (both lie within
// (H+1) 2^-24 sum |w x| of the real dot product).
//
// Kernels:
//   k_logits_chain8  exact, few chains (decode).  Eight chains per wavefront,
//                    eight lanes per chain: in each group of 32 columns lane
//                    8c+j loads columns 4j..4j+3 of chain c's weight and input
//                    rows (each chain reads one 128-byte line of each, by DMA
//                    into an LDS ring) and forms the four products; the
//                    chain's 32 products go through LDS and are added in
//                    column order.  Products cost
//                    4 instructions per 32 columns instead of 32, so a chain
//                    advances one dependent add per instruction slot (about
//                    4.4 clocks: a chain's latency is ~H * 1.9 ns).
//   k_logits_tile    exact, many chains (prefill).  A workgroup owns a tile
//                    of tokens x experts, each lane a register block of
//                    chains, with both operands staged through an LDS ring.
//   k_logits_dot     fast, few tokens.  A workgroup per (expert, block of
//                    tokens) strides over the row in 16-byte loads and reduces
//                    with DPP and LDS.
//   k_logits_rows8   fast, more tokens, at most 8 experts: W in registers,
//                    the token rows streamed once.
//   k_logits_mfma    fast, more tokens: f32 MFMA tiles of tokens x experts.
#include "nx_device.hpp"
#include "nx_internal.hpp"
#include "nx_rows.hpp"

namespace nx {

namespace {

struct F4 {
  float v[4];
};

__device__ __forceinline__ F4 load_f4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const auto q = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  F4 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o.v[i] = __uint_as_float(q[i]);
  return o;
}

// four columns c..c+3 of a row starting at byte `row`; columns at or past H
// (and every column of an invalid row) read as zero
template <bool VEC>
__device__ __forceinline__ F4 load_cols(__amdgpu_buffer_rsrc_t r, uint32_t row, int c, int H,
                                        bool valid) {
  if constexpr (VEC) {  // H % 4 == 0: the four columns are all in or all out
    return load_f4(r, valid && c < H ? row + 4u * (uint32_t)c : OOB);
  } else {
    F4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      o.v[i] = __uint_as_float(bload4(r, valid && c + i < H ? row + 4u * (uint32_t)(c + i) : OOB));
    return o;
  }
}

typedef __attribute__((address_space(3))) void lds_void;

// s_waitcnt vmcnt(n) with the other counters unconstrained
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00);
}

template <int V>
using IC = std::integral_constant<int, V>;

// Workgroup barrier for LDS hand-offs between waves: waits for this wave's
// LDS operations only (DMA loads in flight stay in flight).  The wavefront
// fences keep the compiler from moving memory accesses across the barrier.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt unconstrained
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
}

constexpr int C8_G = 4;     // 32-column groups per ring stage
constexpr int C8_NS = 4;    // ring stages (loads run C8_NS - 1 stages ahead)
constexpr int C8_ROW = 36;  // floats per chain in the LDS product tile (32 + 4 pad)

// Operands go global -> LDS by DMA (buffer_load ... lds) into a ring of
// stages, with explicit vmcnt waits, so nothing is carried in registers from
// one loop trip to the next.  A stage holds, per group, the 64 lanes' four
// weight and four input columns (lane l's 16 bytes at 16 l with 16-byte
// loads; with 4-byte loads column i of lane l at 256 i + 4 l).
// DIAG: chain t pairs row t of W with row t of X (E = 1), so W = X gives
// the sequential sum of squares of each row (rms_norm's variance sum).
// chain8_run: the engine, for a 128-thread workgroup, chains chain0 ..
// chain0 + 7 (chain = t E + e); returns chain chain0 + lane / 8 % 8's sum in
// the lanes of the second wave (the first wave's return value is
// meaningless).  Every wave's DMA has drained when it returns.
template <bool VEC>
__device__ __forceinline__ float chain8_run(const float *__restrict__ W,
                                            const float *__restrict__ X, int T, int E, int H,
                                            int chain0, bool DIAG) {
#pragma clang fp contract(off)
  // one array per ring stage and operand (eight, as many DMA targets as the
  // compiler tracks): it then knows which DMA a read depends on and waits for
  // that one only
  __shared__ __attribute__((aligned(16))) float ringw0[C8_G][256], ringx0[C8_G][256];
  __shared__ __attribute__((aligned(16))) float ringw1[C8_G][256], ringx1[C8_G][256];
  __shared__ __attribute__((aligned(16))) float ringw2[C8_G][256], ringx2[C8_G][256];
  __shared__ __attribute__((aligned(16))) float ringw3[C8_G][256], ringx3[C8_G][256];
  __shared__ __attribute__((aligned(16))) float prod0[C8_G][8 * C8_ROW];
  __shared__ __attribute__((aligned(16))) float prod1[C8_G][8 * C8_ROW];
  static_assert(C8_NS == 4, "four ring arrays");
  const bool producer = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) == 0;
  const int lane = threadIdx.x & 63;
  const int j = lane & 7;
  const int cw = lane >> 3;  // chain within the wave
  const int chain = chain0 + cw;
  const bool valid = chain < T * E;
  const int t = valid ? chain / E : 0;
  const int e = valid ? chain - t * E : 0;
  const auto rw = make_rsrc(W, (uint32_t)((size_t)(DIAG ? T : E) * H * 4));
  const auto rx = make_rsrc(X, (uint32_t)((size_t)T * H * 4));
  // lane's first column of every group (invalid chains read past the buffers)
  const uint32_t wbase = valid ? (uint32_t)(DIAG ? t : e) * (uint32_t)H * 4u + 16u * j : OOB;
  const uint32_t xbase = valid ? (uint32_t)t * (uint32_t)H * 4u + 16u * j : OOB;
  const int nk = (H + 32 * C8_G - 1) / (32 * C8_G);  // stages
  // ring slot S: weight (P = 0) or input (P = 1) columns
  auto slot_of = [&](auto st, auto pt) -> float(*)[256] {
    constexpr int S = decltype(st)::value, P = decltype(pt)::value;
    if constexpr (S == 0) return P ? ringx0 : ringw0;
    else if constexpr (S == 1) return P ? ringx1 : ringw1;
    else if constexpr (S == 2) return P ? ringx2 : ringw2;
    else return P ? ringx3 : ringw3;
  };
  auto prod_of = [&](auto pb) -> float(*)[8 * C8_ROW] {
    if constexpr (decltype(pb)::value == 0) return prod0;
    else return prod1;
  };

  // DMA of stage k into ring slot S = k % C8_NS.  Columns at or past H read
  // as zero: whole groups past the end through a uniform offset past the
  // buffers, the lanes of a group that straddles H through a per-lane test.
  auto issue = [&](auto st, int k) {
    float(*sw)[256] = slot_of(st, IC<0>{});
    float(*sx)[256] = slot_of(st, IC<1>{});
#pragma unroll
    for (int g = 0; g < C8_G; ++g) {
      const int g0 = (k * C8_G + g) * 32;  // first column of the group (uniform)
      if constexpr (VEC) {
        const uint32_t uo = g0 < H ? 4u * (uint32_t)g0 : OOB;
        uint32_t ow = wbase + uo, ox = xbase + uo;
        if (g0 + 32 > H && g0 < H) {  // the group straddles the row end
          const bool in = 4 * j < H - g0;
          ow = in ? ow : OOB;
          ox = in ? ox : OOB;
        }
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_void *)sw[g], 16, ow, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void *)sx[g], 16, ox, 0, 0, 0);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool in = g0 + 4 * j + i < H;
          const uint32_t o = 4u * (uint32_t)(g0 + i);
          const uint32_t ow = in ? wbase + o : OOB;
          const uint32_t ox = in ? xbase + o : OOB;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_void *)(sw[g] + 64 * i), 4, ow, 0, 0, 0);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void *)(sx[g] + 64 * i), 4, ox, 0, 0, 0);
        }
      }
    }
  };
  constexpr int LOADS = VEC ? 2 * C8_G : 8 * C8_G;  // loads per stage
  // stages issued ahead of the one whose products are formed (vmcnt < 64)
  constexpr int AHEAD = VEC ? C8_NS - 2 : 1;

  // lane (cw, j): the four products of its columns of stage slot S into
  // product buffer PB
  auto products = [&](auto st, auto pb) {
    float(*sw)[256] = slot_of(st, IC<0>{});
    float(*sx)[256] = slot_of(st, IC<1>{});
    float(*prod)[8 * C8_ROW] = prod_of(pb);
#pragma unroll
    for (int g = 0; g < C8_G; ++g) {
      float w4[4], x4[4];
      if constexpr (VEC) {
        const float4 a = *reinterpret_cast<const float4 *>(&sw[g][4 * lane]);
        const float4 b = *reinterpret_cast<const float4 *>(&sx[g][4 * lane]);
        w4[0] = a.x, w4[1] = a.y, w4[2] = a.z, w4[3] = a.w;
        x4[0] = b.x, x4[1] = b.y, x4[2] = b.z, x4[3] = b.w;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) w4[i] = sw[g][64 * i + lane], x4[i] = sx[g][64 * i + lane];
      }
      float4 p;
      p.x = w4[0] * x4[0];
      p.y = w4[1] * x4[1];
      p.z = w4[2] * x4[2];
      p.w = w4[3] * x4[3];
      *reinterpret_cast<float4 *>(&prod[g][cw * C8_ROW + 4 * j]) = p;
    }
  };
  float s = 0.f;
  // every lane of chain cw adds the chain's products of buffer PB in column
  // order (broadcast reads, one group ahead of the adds)
  auto adds = [&](auto pb) {
    float(*prod)[8 * C8_ROW] = prod_of(pb);
    float4 q[2][8];
    auto read = [&](int g) {
#pragma unroll
      for (int m = 0; m < 8; ++m)
        q[g & 1][m] = *reinterpret_cast<const float4 *>(&prod[g][cw * C8_ROW + 4 * m]);
    };
    read(0);
#pragma unroll
    for (int g = 0; g < C8_G; ++g) {
      if (g + 1 < C8_G) read(g + 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        s = s + q[g & 1][m].x;
        s = s + q[g & 1][m].y;
        s = s + q[g & 1][m].z;
        s = s + q[g & 1][m].w;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Two waves.  Wave 0 produces: at step k it issues the DMA of stage
  // k+1+AHEAD and forms the products of stage k+1.  Wave 1 consumes: at step k
  // it adds the products of stage k, so its instruction stream is the chain's
  // adds and the LDS reads that feed them.  A workgroup barrier ends each
  // step: the products of stage k+1 are then complete, and the consumer's
  // reads of the other buffer are done before the producer rewrites it.
  if (producer) {
    issue(IC<0>{}, 0);
    if constexpr (AHEAD >= 1) issue(IC<1>{}, 1);
    if constexpr (AHEAD >= 2) issue(IC<2>{}, 2);
    wait_vm<LOADS * AHEAD>();  // stage 0 has landed
    __builtin_amdgcn_sched_barrier(0);
    products(IC<0>{}, IC<0>{});
  }
  lds_barrier();
  auto step = [&](auto st, int k) {
    constexpr int S = decltype(st)::value;
    if (producer) {
      issue(IC<(S + 1 + AHEAD) % C8_NS>{}, k + 1 + AHEAD);  // past the row end: zeros
      wait_vm<LOADS * AHEAD>();                               // stage k+1 has landed
      __builtin_amdgcn_sched_barrier(0);
      products(IC<(S + 1) % C8_NS>{}, IC<(S + 1) % 2>{});
    } else {
      adds(IC<S % 2>{});
    }
    lds_barrier();
  };
  for (int k = 0; k < nk; k += C8_NS) {
    step(IC<0>{}, k);
    if (k + 1 >= nk) break;
    step(IC<1>{}, k + 1);
    if (k + 2 >= nk) break;
    step(IC<2>{}, k + 2);
    if (k + 3 >= nk) break;
    step(IC<3>{}, k + 3);
  }
  wait_vm<0>();  // the DMA of stages past the end has drained
  return s;
}

template <bool VEC, bool DIAG = false>
__global__ __launch_bounds__(128) void k_logits_chain8(const float *__restrict__ W,
                                                      const float *__restrict__ X, int T, int E,
                                                      int H, float *__restrict__ out) {
  const int chain = blockIdx.x * 8 + ((threadIdx.x >> 3) & 7);
  const float s = chain8_run<VEC>(W, X, T, E, H, blockIdx.x * 8, DIAG);
  if ((threadIdx.x >> 6) == 1 && chain < T * E && (threadIdx.x & 7) == 0) out[chain] = s;
}

// The exact prologue of one MoE block (RMSNorm, then the router logits of
// the normalised row) in one launch, or (NORM false) exact router logits of
// few tokens by themselves: workgroup (g, t) takes token t and CPG experts,
// four waves with one router chain per LPC lanes (LPC = 32: two chains per
// wave, 8 per workgroup, rows up to 4096; LPC = 64: one per wave, 4 per
// workgroup, rows up to 7168); every wave also runs the sum of squares
// itself.  Requires H % 4 == 0, 0 < H <= LPC RUN and 16-byte aligned rows.
//
// A sequential f32 sum is bound by its dependent adds, and it reaches that
// bound only when every operand is already in a register: reading operands
// from LDS or memory while the chain runs roughly doubles its time.  So each
// chain is cut into LPC runs of RUN consecutive columns, run r held in the
// registers of lane r of the chain's lanes, loaded and formed before the
// chain starts.  Every lane adds its run to the chain's value on entry (one
// instruction advances all lanes); the value lane r ends with is the chain's
// value after run r, read out with readlane and handed to run r + 1.  The
// adds are those of a left-to-right sum, so the result is bit-identical to
// the column-order chain.
//
// Rows reach the runs through LDS: coalesced 16-byte loads, stored run by
// run with one float4 of padding per run (RUN / 4 + 1 float4 apart), so the
// lanes reading their runs' k-th float4 hit different banks.
//  1. Each wave stages its router rows in its own LDS buffers; the row (x)
//     goes to a shared buffer, zero-padded to LPC runs, and each thread
//     keeps its share of the row and of the norm weight in registers.
//  2. The sum of squares: 64 runs of RUN LPC / 64 columns, run r in lane r
//     (runs past the row end are skipped; a partial last run adds +0 to a
//     sum that started at +0, which leaves it unchanged).
//     rstd = 1 / sqrt(sum / H + eps).
//  3. Each thread forms its share of the normalised row, (x_i rstd) w_i,
//     into the shared buffer (workgroup 0 also writes it to xn); each lane
//     then forms the products W[e][i] xn_i of its run.
//  4. The router chains, run r of the chain on lanes LPC h .. in lane
//     LPC h + r.
// The arithmetic is that of the RMSNorm kernel and the chain kernel, so the
// row and the logits are bit-identical to theirs.
template <int LPC>
struct PrologueShape {
  static_assert(LPC == 32 || LPC == 64, "lanes per chain");
  static constexpr int RUN = LPC == 32 ? 128 : 112;   // columns per run
  static constexpr int RUN4 = RUN / 4;                // float4 per run
  static constexpr int MAXH = LPC * RUN;              // 4096 / 7168
  static constexpr int PAD4 = LPC * (RUN4 + 1);       // padded row, in float4
  static constexpr int CPW = 64 / LPC;                // chains per wave
  static constexpr int CPG = 4 * CPW;                 // chains (experts) per workgroup
  static constexpr int S4 = RUN4 * LPC / 64;          // float4 per lane, sum of squares
  static constexpr int RJ = LPC * RUN4 / 64;          // float4 per lane of a staged router row
  static constexpr int XJ = LPC * RUN4 / 256;         // float4 per thread of the row
  static_assert(LPC * RUN4 % 256 == 0, "whole float4 of the row per thread");
};
constexpr int BP_MAXH = PrologueShape<64>::MAXH;      // 7168
static_assert(BP_MAXH == kPrologueMaxH, "the register-run chains' widest row");

template <bool NORM, int LPC>
__global__ __launch_bounds__(256) void k_block_prologue(const float *__restrict__ x,
                                                        const float *__restrict__ nw, float eps,
                                                        const float *__restrict__ W, int E, int H,
                                                        float *__restrict__ xn,
                                                        float *__restrict__ logits) {
#pragma clang fp contract(off)
  using PS = PrologueShape<LPC>;
  constexpr int RUN4 = PS::RUN4, CPW = PS::CPW, S4 = PS::S4, RJ = PS::RJ, XJ = PS::XJ;
  __shared__ float4 xs[PS::PAD4], ws[4][CPW][PS::PAD4];  // 152 KB / 148.5 KB
  const int t = blockIdx.y, tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, hl = lane % LPC, ch = lane / LPC;
  const int e0 = blockIdx.x * PS::CPG + wave * CPW;  // the wave's experts: e0 .. e0 + CPW - 1
  const int H4 = H >> 2;
  const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
  auto pad = [](int i) { return i + i / RUN4; };  // float4 i of the row -> LDS slot
  // 1. loads with indices clamped into the rows and values selected
  // afterwards: no branches, so every load is issued before the first wait
  float4 xv[XJ], nv[XJ];
  {
    const float4 *xr4 = reinterpret_cast<const float4 *>(x + (size_t)t * H);
    const float4 *nw4 = reinterpret_cast<const float4 *>(nw);
#pragma unroll
    for (int j = 0; j < XJ; ++j) {
      const int i = min(j * 256 + tid, H4 - 1);
      xv[j] = xr4[i];
      if constexpr (NORM) nv[j] = nw4[i];
    }
  }
#pragma unroll
  for (int h = 0; h < CPW; ++h) {
    const int e = e0 + h;
    const float4 *r4 = reinterpret_cast<const float4 *>(W + (size_t)(e < E ? e : 0) * H);
    float4 wr[RJ];
#pragma unroll
    for (int j = 0; j < RJ; ++j) wr[j] = r4[min(j * 64 + lane, H4 - 1)];
#pragma unroll
    for (int j = 0; j < RJ; ++j) {
      const int i = j * 64 + lane;
      float4 v = wr[j];
      if (e >= E || i >= H4) v = z4;
      ws[wave][h][pad(i)] = v;
    }
  }
#pragma unroll
  for (int j = 0; j < XJ; ++j) {
    const int i = j * 256 + tid;
    if (i >= H4) xv[j] = z4;  // (the padding: zero squares and products)
    xs[pad(i)] = xv[j];
  }
  __syncthreads();  // the row is in LDS
  if constexpr (NORM) {
    // 2. the sum of squares, run r (float4 S4 r .. of the row) in lane r
    float ss = 0.f;
    {
      float4 q[S4];
#pragma unroll
      for (int k = 0; k < S4; ++k) {
        const float4 v = xs[pad(lane * S4 + k)];
        q[k] = make_float4(v.x * v.x, v.y * v.y, v.z * v.z, v.w * v.w);
      }
      const int nsq = (H4 + S4 - 1) / S4;
      for (int r = 0; r < nsq; ++r) {
        float a = ss;
#pragma unroll
        for (int k = 0; k < S4; ++k) {
          a = a + q[k].x;
          a = a + q[k].y;
          a = a + q[k].z;
          a = a + q[k].w;
        }
        ss = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), r));
      }
    }
    const float rs = 1.0f / __builtin_sqrtf(ss / (float)H + eps);
    // 3. the normalised row, into the shared buffer once every wave has
    // read its squares
    __syncthreads();
    float4 *xo4 = reinterpret_cast<float4 *>(xn + (size_t)t * H);
#pragma unroll
    for (int j = 0; j < XJ; ++j) {
      const int i = j * 256 + tid;
      const float4 v = xv[j], w = nv[j];
      const float4 o = make_float4((v.x * rs) * w.x, (v.y * rs) * w.y, (v.z * rs) * w.z,
                                   (v.w * rs) * w.w);
      xs[pad(i)] = o;
      if (blockIdx.x == 0 && i < H4) xo4[i] = o;
    }
    __syncthreads();
  }
  // the products of each lane's run
  float4 p[RUN4];
  {
    const float4 *my = ws[wave][ch];
#pragma unroll
    for (int k = 0; k < RUN4; ++k) {
      const int c = hl * (RUN4 + 1) + k;
      const float4 w = my[c], o = xs[c];
      p[k] = make_float4(w.x * o.x, w.y * o.y, w.z * o.z, w.w * o.w);
    }
  }
  // 4. the router chains, run r of chain h in lane LPC h + r
  const int nrt = (H4 + RUN4 - 1) / RUN4;
  float s0 = 0.f, s1 = 0.f;
  for (int r = 0; r < nrt; ++r) {
    float a = (CPW == 2 && ch) ? s1 : s0;
#pragma unroll
    for (int k = 0; k < RUN4; ++k) {
      a = a + p[k].x;
      a = a + p[k].y;
      a = a + p[k].z;
      a = a + p[k].w;
    }
    s0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), r));
    if constexpr (CPW == 2) s1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 32 + r));
  }
  if (hl == 0 && e0 + ch < E) logits[(size_t)t * E + e0 + ch] = (CPW == 2 && ch) ? s1 : s0;
}

constexpr int TL_NS = 3;  // ring stages of the tiled kernel

// Tile of (16 RB tokens) x (16 RB experts) per 256-thread workgroup: lane l
// holds the RB x RB chains of tokens t0 + RB (l / 16) + i and experts
// e0 + RB (l % 16) + j.  Columns are staged KC = 128 / RB at a time (512
// 16-byte units per operand and stage) in an LDS ring filled by DMA; unit u
// of row r sits at r * (KC / 4) + (u ^ (r & 7)), so the rows a wave reads at
// one column spread over the banks.  Each chain is summed in column order
// with separately rounded products and sums (exact mode).
// Requires H % 4 == 0 and 16-byte aligned rows.
template <int RB>
__global__ __launch_bounds__(256) void k_logits_tile(const float *__restrict__ W,
                                                     const float *__restrict__ X, int T, int E,
                                                     int H, float *__restrict__ out) {
#pragma clang fp contract(off)
  constexpr int ROWS = 16 * RB;   // rows per operand tile
  constexpr int KC = 128 / RB;    // columns per stage
  constexpr int U = KC / 4;       // 16-byte units per row
  constexpr int UNITS = ROWS * U; // = 512
  // 1 KB DMAs per operand and stage: UNITS / 64 = 8, two per wave
  constexpr int PW = UNITS / 64 / 4;
  static_assert(UNITS == 512 && PW == 2, "tile shape");
  __shared__ __attribute__((aligned(16))) float w0[UNITS * 4], x0[UNITS * 4];
  __shared__ __attribute__((aligned(16))) float w1[UNITS * 4], x1[UNITS * 4];
  __shared__ __attribute__((aligned(16))) float w2[UNITS * 4], x2[UNITS * 4];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int e0 = blockIdx.x * ROWS, t0 = blockIdx.y * ROWS;
  const auto rw = make_rsrc(W, (uint32_t)((size_t)E * H * 4));
  const auto rx = make_rsrc(X, (uint32_t)((size_t)T * H * 4));

  // DMA d of a wave (d < 2 PW: weight units for d < PW, input units after)
  // writes LDS units b*64 .. b*64+63 of its operand, b = wave * PW + d % PW
  // < UNITS / 64; lane L fetches the 16 bytes that belong at unit b*64 + L
  uint32_t doff[2 * PW];
  int dcol[2 * PW];
#pragma unroll
  for (int d = 0; d < 2 * PW; ++d) {
    const int p = (wave * PW + d % PW) * 64 + lane;
    const int r = p / U, u = (p % U) ^ (r & 7);
    const int row = (d < PW ? e0 : t0) + r;
    const bool ok = row < (d < PW ? E : T);
    doff[d] = ok ? (uint32_t)row * (uint32_t)H * 4u + 16u * (uint32_t)u : OOB;
    dcol[d] = 4 * u;
  }
  auto wbuf = [&](auto st) -> float * {
    constexpr int S = decltype(st)::value;
    if constexpr (S == 0) return w0;
    else if constexpr (S == 1) return w1;
    else return w2;
  };
  auto xbuf = [&](auto st) -> float * {
    constexpr int S = decltype(st)::value;
    if constexpr (S == 0) return x0;
    else if constexpr (S == 1) return x1;
    else return x2;
  };
  auto issue = [&](auto st, int c) {
    const int k0 = c * KC;
    float *wb = wbuf(st), *xb = xbuf(st);
#pragma unroll
    for (int d = 0; d < 2 * PW; ++d) {
      const uint32_t off = k0 + dcol[d] < H ? doff[d] + 4u * (uint32_t)k0 : OOB;
      float *dst = (d < PW ? wb : xb) + (wave * PW + d % PW) * 256;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(d < PW ? rw : rx, (lds_void *)dst, 16, off, 0, 0,
                                               0);
    }
  };

  const int tg = tid >> 4, eg = tid & 15;
  float s[RB][RB];
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int j = 0; j < RB; ++j) s[i][j] = 0.f;
  auto compute = [&](auto st) {
    const float *wb = wbuf(st), *xb = xbuf(st);
#pragma unroll
    for (int k4 = 0; k4 < U; ++k4) {
      float4 xv[RB], wv[RB];
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const int r = RB * tg + i;
        xv[i] = *reinterpret_cast<const float4 *>(xb + 4 * (r * U + (k4 ^ (r & 7))));
      }
#pragma unroll
      for (int j = 0; j < RB; ++j) {
        const int r = RB * eg + j;
        wv[j] = *reinterpret_cast<const float4 *>(wb + 4 * (r * U + (k4 ^ (r & 7))));
      }
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
          for (int j = 0; j < RB; ++j) {
            const float xk = kk == 0 ? xv[i].x : kk == 1 ? xv[i].y : kk == 2 ? xv[i].z : xv[i].w;
            const float wk = kk == 0 ? wv[j].x : kk == 1 ? wv[j].y : kk == 2 ? wv[j].z : wv[j].w;
            s[i][j] = s[i][j] + wk * xk;
          }
    }
  };
  // stage c: wait for its DMA (stage c+1 may stay in flight), barrier (all
  // waves' DMA of stage c landed; all reads of stage c-1's slot done), DMA of
  // stage c+2 into that slot, then the chains advance KC columns
  auto step = [&](auto st, int c) {
    constexpr int S = decltype(st)::value;
    wait_vm<2 * PW>();
    lds_barrier();
    issue(IC<(S + 2) % TL_NS>{}, c + 2);
    compute(st);
  };
  const int nst = (H + KC - 1) / KC;
  issue(IC<0>{}, 0);
  issue(IC<1>{}, 1);
  for (int c = 0; c < nst; c += TL_NS) {
    step(IC<0>{}, c);
    if (c + 1 >= nst) break;
    step(IC<1>{}, c + 1);
    if (c + 2 >= nst) break;
    step(IC<2>{}, c + 2);
  }
  wait_vm<0>();  // the DMA of stages past the end has drained
#pragma unroll
  for (int i = 0; i < RB; ++i) {
    const int t = t0 + RB * tg + i;
#pragma unroll
    for (int j = 0; j < RB; ++j) {
      const int e = e0 + RB * eg + j;
      if (t < T && e < E) out[(size_t)t * E + e] = s[i][j];
    }
  }
}

// fast mode, few tokens: workgroup (expert, token block of BT)
template <int BT, bool VEC>
__global__ __launch_bounds__(256) void k_logits_dot(const float *__restrict__ W,
                                                    const float *__restrict__ X, int T, int E,
                                                    int H, float *__restrict__ out) {
  __shared__ float part[4][BT];
  const int e = blockIdx.x;
  const int t0 = blockIdx.y * BT;
  const auto rw = make_rsrc(W, (uint32_t)((size_t)E * H * 4));
  const auto rx = make_rsrc(X, (uint32_t)((size_t)T * H * 4));
  const uint32_t wrow = (uint32_t)e * (uint32_t)H * 4u;
  float s[BT];
#pragma unroll
  for (int b = 0; b < BT; ++b) s[b] = 0.f;
  for (int c = 4 * threadIdx.x; c < H; c += 4 * 256) {
    const F4 w = load_cols<VEC>(rw, wrow, c, H, true);
#pragma unroll
    for (int b = 0; b < BT; ++b) {
      const bool ok = t0 + b < T;
      const F4 x = load_cols<VEC>(rx, (uint32_t)(ok ? t0 + b : 0) * (uint32_t)H * 4u, c, H, ok);
#pragma unroll
      for (int i = 0; i < 4; ++i) s[b] = __builtin_fmaf(w.v[i], x.v[i], s[b]);
    }
  }
  group_sum_n<64, BT>(s);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 63) {
#pragma unroll
    for (int b = 0; b < BT; ++b) part[wave][b] = s[b];
  }
  __syncthreads();
  if (threadIdx.x < BT && t0 + (int)threadIdx.x < T) {
    const int b = threadIdx.x;
    out[(size_t)(t0 + b) * E + e] = (part[0][b] + part[1][b]) + (part[2][b] + part[3][b]);
  }
}

// Fast mode, many tokens, at most 8 experts and rows of at most 4 NJ x 256
// columns: a workgroup holds W in registers (thread t: columns 4 (t + 256 j)
// .. + 3 of every expert row, j < NJ; absent experts and columns as zeros)
// and streams the rows of its tokens t0 .. t0 + tpw - 1, the next token's row
// loaded while the current one is multiplied.  Per token each thread forms
// 8 partial dots; the wave reduces them by halving exchanges (lane bit 5,
// then 4, then 3: each step sends the half of its values it drops and adds
// the partner's half of those it keeps), leaving lane l with expert
// 4 b5 + 2 b4 + b3 summed over the lanes that share those bits, which three
// more exchanges complete; the four waves add through LDS at the end.
template <int NJ>
__global__ __launch_bounds__(256) void k_logits_rows8(const float *__restrict__ W,
                                                      const float *__restrict__ X, int T, int E,
                                                      int H, int tpw, float *__restrict__ out) {
  constexpr int MAXT = 16;  // tokens per workgroup at most
  __shared__ float part[MAXT][4][8];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const auto rw = make_rsrc(W, (uint32_t)((size_t)E * H * 4));
  const auto rx = make_rsrc(X, (uint32_t)((size_t)T * H * 4));
  float w[8][NJ][4];
#pragma unroll
  for (int e = 0; e < 8; ++e)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const F4 v = load_cols<true>(rw, (uint32_t)(e < E ? e : 0) * (uint32_t)H * 4u,
                                   4 * (tid + 256 * j), H, e < E);
#pragma unroll
      for (int i = 0; i < 4; ++i) w[e][j][i] = v.v[i];
    }
  const int t0 = (int)blockIdx.x * tpw;
  const int nt = min(tpw, T - t0);
  auto load_row = [&](int t, F4 (&xr)[NJ]) {
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      xr[j] = load_cols<true>(rx, (uint32_t)(t < T ? t : 0) * (uint32_t)H * 4u,
                              4 * (tid + 256 * j), H, t < T);
  };
  F4 xa[NJ], xb[NJ];
  load_row(t0, xa);
  for (int b = 0; b < nt; ++b) {
    load_row(t0 + b + 1 < t0 + nt ? t0 + b + 1 : T, xb);  // the next row (past the end: zeros)
    float s[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc = __builtin_fmaf(w[e][j][i], xa[j].v[i], acc);
      s[e] = acc;
    }
    // halving exchanges over lane bits 5, 4, 3: 8 -> 4 -> 2 -> 1 values
    const bool b5 = lane & 32, b4 = lane & 16, b3 = lane & 8;
    float s4[4], s2[2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      s4[i] = (b5 ? s[4 + i] : s[i]) + __shfl_xor(b5 ? s[i] : s[4 + i], 32, 64);
#pragma unroll
    for (int i = 0; i < 2; ++i)
      s2[i] = (b4 ? s4[2 + i] : s4[i]) + __shfl_xor(b4 ? s4[i] : s4[2 + i], 16, 64);
    float v = (b3 ? s2[1] : s2[0]) + __shfl_xor(b3 ? s2[0] : s2[1], 8, 64);
    v += __shfl_xor(v, 4, 64);
    v += __shfl_xor(v, 2, 64);
    v += __shfl_xor(v, 1, 64);
    if ((lane & 7) == 0) part[b][wave][lane >> 3] = v;  // expert 4 b5 + 2 b4 + b3
#pragma unroll
    for (int j = 0; j < NJ; ++j) xa[j] = xb[j];
  }
  __syncthreads();
  if (tid < nt * 8) {
    const int b = tid >> 3, e = tid & 7;
    if (e < E)
      out[(size_t)(t0 + b) * E + e] = (part[b][0][e] + part[b][1][e]) + (part[b][2][e] + part[b][3][e]);
  }
}

typedef float f32x4_t __attribute__((ext_vector_type(4)));

// Fast mode, many tokens, on the matrix cores (v_mfma_f32_16x16x4_f32, f32
// operands and sums): logits = X . W^T.  A wave owns MT x NT tiles of 16
// tokens x 16 experts over a range of 16-column steps.  Lane l feeds row
// l % 16 of each operand tile (token t0 + 16 m + l % 16 of X, expert e0 + 16
// n + l % 16 of W) with one 16-byte load per step, columns k + 4 (l / 16) ..
// + 3, one per MFMA: the four MFMAs of a step cover the step's 16 columns in
// a permuted order, the same for both operands, which fast mode allows.
// KS waves of a workgroup split the steps and add their tiles through LDS in
// wave order; with KS = 1 the four waves own four neighbouring token tiles.
// Lane l holds output rows 4 (l / 16) .. + 3 of column l % 16 of a tile.
// Rows of X and W past the matrices, and columns past the row (whole float4s:
// H % 4 == 0), read as zeros.  D steps are in flight while one is multiplied.
template <int MT, int NT, int KS>
__global__ __launch_bounds__(256) void k_logits_mfma(const float *__restrict__ W,
                                                     const float *__restrict__ X, int T, int E,
                                                     int H, float *__restrict__ out) {
  constexpr int WT = 4 / KS;  // a workgroup's output tiles, along the tokens
  constexpr int D = 3;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int kpart = wave % KS, tw = wave / KS;
  const int t0 = ((int)blockIdx.x * WT + tw) * 16 * MT, e0 = (int)blockIdx.y * 16 * NT;
  const int r = lane & 15, g = lane >> 4;
  const auto rx = make_rsrc(X, (uint32_t)((size_t)T * H * 4));
  const auto rw = make_rsrc(W, (uint32_t)((size_t)E * H * 4));
  uint32_t xo[MT], wo[NT];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const int t = t0 + 16 * m + r;
    xo[m] = t < T ? (uint32_t)t * (uint32_t)H * 4u : OOB;
  }
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int e = e0 + 16 * n + r;
    wo[n] = e < E ? (uint32_t)e * (uint32_t)H * 4u : OOB;
  }
  const int nsteps = (H + 15) / 16;
  const int sb = kpart * nsteps / KS, se = (kpart + 1) * nsteps / KS;
  f32x4_t acc[MT][NT];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[m][n] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  uint4 a[D][MT], b[D][NT];
  // loads of step s into ring slot j (steps past the range read zeros)
  auto issue = [&](int j, int s) {
    const int k = 16 * s + 4 * g;
    const uint32_t ko = s < se && k < H ? 4u * (uint32_t)k : OOB;
#pragma unroll
    for (int m = 0; m < MT; ++m) a[j][m] = bload16(rx, xo[m] + ko);
#pragma unroll
    for (int n = 0; n < NT; ++n) b[j][n] = bload16(rw, wo[n] + ko);
  };
  auto lane_f = [](const uint4 &v, int i) {
    return __uint_as_float(i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w);
  };
#pragma unroll
  for (int j = 0; j < D - 1; ++j) issue(j, sb + j);
  for (int s = sb; s < se; s += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      if (s + j >= se) break;  // wave-uniform
      issue((j + D - 1) % D, s + j + D - 1);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
          for (int n = 0; n < NT; ++n)
            acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(lane_f(a[j][m], i), lane_f(b[j][n], i),
                                                             acc[m][n], 0, 0, 0);
    }
  }
  if constexpr (KS > 1) {
    __shared__ f32x4_t red[4 * MT * NT * 64];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int n = 0; n < NT; ++n) red[((wave * MT + m) * NT + n) * 64 + lane] = acc[m][n];
    __syncthreads();
    if (kpart != 0) return;  // wave-uniform
#pragma unroll
    for (int q = 1; q < KS; ++q)
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int n = 0; n < NT; ++n) acc[m][n] += red[(((tw * KS + q) * MT + m) * NT + n) * 64 + lane];
  }
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      const int e = e0 + 16 * n + r;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t0 + 16 * m + 4 * g + i;
        if (t < T && e < E) out[(size_t)t * E + e] = acc[m][n][i];
      }
    }
}

void launch_tile(nx_ctx *c, int rb, const float *W, const float *X, int T, int E, int H,
                 float *out) {
  const int rows = 16 * rb;
  const dim3 grid((E + rows - 1) / rows, (T + rows - 1) / rows);
  if (rb == 4) go(c, k_logits_tile<4>, dim3(grid), dim3(256), 0, W, X, T, E, H, out);
  else if (rb == 2) go(c, k_logits_tile<2>, dim3(grid), dim3(256), 0, W, X, T, E, H, out);
  else go(c, k_logits_tile<1>, dim3(grid), dim3(256), 0, W, X, T, E, H, out);
}

}  // namespace

// chains (token, expert pairs) up to which the exact path uses k_logits_chain8
constexpr long LOGITS_CHAIN8_MAX = 16384;
constexpr long LOGITS_RUNS_MAX_WG = 256;  // workgroups of the register-run chains
// fast path: tokens up to which k_logits_dot is used (eight tokens per
// workgroup beyond 4; the MFMA tiles have too few workgroups below ~32 tokens:
// Mixtral at 32 tokens 12.5 us on two of them)
constexpr int LOGITS_DOT_MAX_T = 32;

int launch_router_logits(nx_ctx *c, const float *d_w, const float *d_x, int T, int E, int H,
                         bool exact, float *d_out) {
  if (T <= 0 || E <= 0) return NX_OK;
  const bool vec = H % 4 == 0 && ((uintptr_t)d_w & 15) == 0 && ((uintptr_t)d_x & 15) == 0;
  const long chains = (long)T * E;
  // fast mode: few tokens on k_logits_dot, more on the GEMM below; the exact
  // order is also a valid fast order, so the chain kernel serves rows it
  // cannot load whole (unaligned, H % 4 != 0) in both modes
  const bool dot = !exact && vec && T <= LOGITS_DOT_MAX_T;
  const bool chain8 = !vec || (exact && chains <= LOGITS_CHAIN8_MAX);
  // exact, rows up to 7168, up to one round of workgroups (each holds a CU's
  // LDS): the register-run chains of the block prologue without its RMSNorm
  // (its loads clamp their indices into the row: register_row_fits)
  const bool narrow = H <= PrologueShape<32>::MAXH;
  const int cpg = narrow ? PrologueShape<32>::CPG : PrologueShape<64>::CPG;
  if (exact && vec && register_row_fits(H, kPrologueMaxH) &&
      (long)T * ((E + cpg - 1) / cpg) <= LOGITS_RUNS_MAX_WG) {
    const dim3 grid((unsigned)((E + cpg - 1) / cpg), (unsigned)T);
    return launch(c, "router_logits_runs", [&] {
      if (narrow)
        go(c, k_block_prologue<false, 32>, grid, dim3(256), 0, d_x, nullptr, 0.f, d_w, E, H,
           nullptr, d_out);
      else
        go(c, k_block_prologue<false, 64>, grid, dim3(256), 0, d_x, nullptr, 0.f, d_w, E, H,
           nullptr, d_out);
    });
  }
  if (chain8) {
    const unsigned grid = (unsigned)((chains + 7) / 8);
    return launch(c, "router_logits_chain8", [&] {
      if (vec)
        go(c, k_logits_chain8<true>, dim3(grid), dim3(128), 0, d_w, d_x, T, E, H, d_out);
      else
        go(c, k_logits_chain8<false>, dim3(grid), dim3(128), 0, d_w, d_x, T, E, H, d_out);
    });
  }
  if (dot) {
    const int bt = T == 1 ? 1 : (T <= 4 ? 4 : 8);
    const dim3 grid(E, (T + bt - 1) / bt);
    return launch(c, "router_logits_dot", [&] {
      if (bt == 1) go(c, k_logits_dot<1, true>, dim3(grid), dim3(256), 0, d_w, d_x, T, E, H, d_out);
      else if (bt == 4) go(c, k_logits_dot<4, true>, dim3(grid), dim3(256), 0, d_w, d_x, T, E, H, d_out);
      else go(c, k_logits_dot<8, true>, dim3(grid), dim3(256), 0, d_w, d_x, T, E, H, d_out);
    });
  }
  if (!exact && vec && E <= 8 && H <= 4096 && (size_t)T * H * 4 < (1u << 31)) {
    // fast mode, more than a few tokens, at most 8 experts: W in registers,
    // the token rows streamed once (Mixtral at 2048 tokens on the MFMA tiles
    // below: 14.4 us, 128 workgroups of 16-token tiles half empty)
    const int tpw = (int)std::min<long>(16, std::max<long>(1, (T + c->num_cu - 1) / c->num_cu));
    const dim3 grid((unsigned)((T + tpw - 1) / tpw));
    return launch(c, "router_logits_rows8", [&] {
      if (H <= 1024) go(c, k_logits_rows8<1>, grid, dim3(256), 0, d_w, d_x, T, E, H, tpw, d_out);
      else if (H <= 2048) go(c, k_logits_rows8<2>, grid, dim3(256), 0, d_w, d_x, T, E, H, tpw, d_out);
      else go(c, k_logits_rows8<4>, grid, dim3(256), 0, d_w, d_x, T, E, H, tpw, d_out);
    });
  }
  if (!exact && (size_t)T * H * 4 < (1u << 31) && (size_t)E * H * 4 < (1u << 31)) {
    // Fast mode, more than a few tokens: logits = X . W^T on the matrix
    // cores in f32 (any summation order is within fast mode's bound).  Tiles
    // of 16 x 16 for up to 16 experts, else of 32 x 32 per wave; the four
    // waves of a workgroup split K unless the output tiles alone fill two
    // workgroups per CU.
    const int nt = E <= 16 ? 1 : 2;
    const long tiles_n = (E + 16 * nt - 1) / (16 * nt);
    // tokens per workgroup: 16 (16 x 16 tiles, K split), 128 (four 32 x 32
    // tiles) or 32 (one 32 x 32 tile, K split)
    const bool ks1 = nt == 2 && (long)((T + 127) / 128) * tiles_n >= 2L * c->num_cu;
    const int tm = nt == 1 ? 16 : (ks1 ? 128 : 32);
    const dim3 grid((unsigned)((T + tm - 1) / tm), (unsigned)tiles_n);
    return launch(c, "router_logits_mfma", [&] {
      if (nt == 1) go(c, k_logits_mfma<1, 1, 4>, grid, dim3(256), 0, d_w, d_x, T, E, H, d_out);
      else if (ks1) go(c, k_logits_mfma<2, 2, 1>, grid, dim3(256), 0, d_w, d_x, T, E, H, d_out);
      else go(c, k_logits_mfma<2, 2, 4>, grid, dim3(256), 0, d_w, d_x, T, E, H, d_out);
    });
  }
  // chains per lane: as many as keep at least 1024 waves in the grid
  const int rb = chains >= 1024L * 64 * 16 ? 4 : (chains >= 1024L * 64 * 4 ? 2 : 1);
  return launch(c, "router_logits_tile",
                [&] { launch_tile(c, rb, d_w, d_x, T, E, H, d_out); });
}

int launch_block_prologue(nx_ctx *c, const float *d_x, const float *d_nw, float eps,
                          const float *d_w, int T, int E, int H, float *d_xn, float *d_logits) {
  if (T <= 0 || E <= 0) return NX_OK;
  if (!block_prologue_fits(H, d_x, d_nw, d_w, d_xn))
    return fail(NX_ERR_UNSUPPORTED, "block prologue: row shape or alignment not supported");
  // runs of 128 columns on 32 lanes (rows up to 4096), else of 112 on 64
  if (H <= PrologueShape<32>::MAXH) {
    const dim3 grid((unsigned)((E + PrologueShape<32>::CPG - 1) / PrologueShape<32>::CPG),
                    (unsigned)T);
    return launch(c, "block_prologue", [&] {
      go(c, k_block_prologue<true, 32>, grid, dim3(256), 0, d_x, d_nw, eps, d_w, E, H, d_xn,
         d_logits);
    });
  }
  const dim3 grid((unsigned)((E + PrologueShape<64>::CPG - 1) / PrologueShape<64>::CPG),
                  (unsigned)T);
  return launch(c, "block_prologue", [&] {
    go(c, k_block_prologue<true, 64>, grid, dim3(256), 0, d_x, d_nw, eps, d_w, E, H, d_xn,
       d_logits);
  });
}

bool block_prologue_fits(int H, const void *x, const void *nw, const void *w, const void *xn) {
  auto al = [](const void *q) { return ((uintptr_t)q & 15) == 0; };
  return register_row_fits(H, kPrologueMaxH) && al(x) && al(nw) && al(w) && al(xn);
}

int launch_sumsq_exact(nx_ctx *c, const float *d_x, int T, int H, float *d_out) {
  if (T <= 0) return NX_OK;
  const bool vec = H % 4 == 0 && ((uintptr_t)d_x & 15) == 0;
  const unsigned grid = (unsigned)((T + 7) / 8);
  return launch(c, "rms_sumsq_chain8", [&] {
    if (vec)
      go(c, k_logits_chain8<true, true>, dim3(grid), dim3(128), 0, d_x, d_x, T, 1, H, d_out);
    else
      go(c, k_logits_chain8<false, true>, dim3(grid), dim3(128), 0, d_x, d_x, T, 1, H, d_out);
  });
}

}  // namespace nx
