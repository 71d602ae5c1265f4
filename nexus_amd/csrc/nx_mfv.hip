// nx_mfv.hip — few-token grouped matvec on MFMA for Q4_K, Q4_0, Q8_0 and Q2_K experts: decode
// batches whose experts see a handful of tokens each (2 to ~128 tokens),
// with or without a shared expert (as wide as the routed ones) that sees
// every token.
//
// The decode GEMV's exact integer dot costs about one instruction per
// weight per token, so its time grows with the tokens an expert sees; the
// prefill GEMM dequantizes every weight into its operands, which costs the
// same at 8 tokens as at 128.  Here the weights are never dequantized:
//
//   sum_i w_i x_i over a 32-weight sub-block s of a Q4_K block
//     = (d sc_s) sum_i q_i x_i  -  (dmin m_s) sum_i x_i
//
// (src/quant/mod.rs:820-849: w_i = d sc_s q_i - dmin m_s).  The operand of
// weight i is the integer q_i sc_s (at most 15 x 63 = 945) written as the
// bits of an fp16 subnormal, i.e. the exact value q_i sc_s 2^-24: a byte
// permute and a packed 16-bit multiply per two weights, no float
// conversion.  With the 6-bit scale inside the operands, one
// v_mfma_f32_16x16x32_f16 may span several sub-blocks, so the 8 MFMAs of a
// block accumulate together; d 2^24 and the dmin term apply once per block.
// sum_s m_s X_s is one more MFMA per block, on the pairs' staged sub-block
// sums X_s and the row's 6-bit mins.
//
// Activations keep close to fp32 precision: per pair and 256-element chunk
// they are scaled by a power of two so the chunk maximum lies in
// [2^13, 2^14), split into x' = hi + lo with hi = fp16(x') and lo =
// fp16(x' - hi), and both halves go through the MFMA (two MFMAs per
// sub-block, chained).  hi + lo carries 22 bits of x', so the dot products
// match an fp32 evaluation to a few units of 2^-22 of the chunk maximum.
//
// Work: a workgroup of 4 waves owns one tile of up to 16 pairs of one
// expert (the permutation's tile list with tile_m = 16), 256 weight rows
// (of both matrices for gate/up) and one K slice of 4 (gate/up) or 3 (down)
// chunks (a chunk is 256 positions: one Q4_K or Q2_K block, 8 Q4_0 or
// Q8_0 blocks); wave w streams 64 of the rows as 4 row tiles of 16.  The
// slice's activations of the tile's pairs are staged once into LDS in MFMA
// operand layout, with each pair's unscale factor and block or sub-block
// sums; the codes and scales of the next 3 (row tile, chunk) steps (Q8_0:
// 2) are in flight while a step is computed.  Slices write partial sums,
// which the SwiGLU kernel (gate/up) and the weighted combine (down) add in
// slice order.
//
// Q4_0 (w_i = d (q_i - 8) per 32-weight block, src/quant/mod.rs:723-745)
// runs the same kernel on chunks of 8 blocks: one MFMA pair per block, the
// codes unsigned (q_i 2^-24) and the 8 taken off through each block's
// staged activation sum, the f16 block scale d applied to that MFMA's
// result.  The loads give a lane group two whole blocks; a 4 x 4 dword
// transpose across the lane groups hands every lane group its 8 weights of
// each block.  Q8_0 (w_i = d q_i, q_i a signed byte, src/quant/mod.rs:
// 689-703) likewise, with the operand q_i + 128 (one byte permute per two
// weights), 128 X taken off, and dword pairs transposed (a lane group loads
// two whole blocks of 32 bytes).
//
// Q2_K (w_i = d sc q_i - dmin m per 16-weight sub-block, 4-bit sc and m,
// src/quant/mod.rs:913-937): a chunk is one block, its 4 resident segments
// (64 weights in 16 bytes) one per lane group; MFMA u takes dword u % 4 of
// half u / 4, 8 weights of sub-block 4 g + u / 2, whose scale goes into the
// operands (q sc <= 45); the min term is one MFMA per chunk on the 16
// sub-block sums, as for Q4_K.
#include "nx_device.hpp"
#include "nx_internal.hpp"

namespace nx {

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int MV_M = 16;   // pairs per tile
constexpr int MV_K = 256;  // K positions per chunk

struct MfvArgs {
  const uint8_t *qs0, *qs1, *meta0, *meta1;  // role planes (gate, up) or (down, -)
  size_t qs_stride, meta_stride;             // per expert
  uint32_t row_qs, row_meta;
  int rows, nseg, nchunk;                    // nchunk = cols / 256
  const float *x;
  int x_stride;
  const int32_t *perm_token;  // gate/up: pair -> token row of x; down: null (pair row)
  const int32_t *offsets;     // [E + 1]
  const int32_t *tiles;       // [0] = tile count, [1] unused, then (expert, first pair within it)
  // the shared expert (tiles of expert E; pairs T k + t, t the token), with
  // the routed experts' row layout
  const uint8_t *sqs0, *sqs1, *smeta0, *smeta1;
  int E, T, k;
  float *out;                 // partial sums: [slice][pair][out_stride]
  int out_stride;             // gate/up: 2 F (gate rows, then up rows); down: H
  size_t out_split;           // floats between slices
  int nrb, ntiles_g, nks;     // grid: row blocks, tile bound, K slices
  int xcd_pairs;              // 1: the 1-D slice-pair grid below, 0: (row block, tile, slice)
};

// LDS area of one chunk: the A operands (hi, lo) of the 8 MFMAs in lane
// order and the per-pair unscale factors; Q4_0 also keeps each block's
// activation sum (times 8) per pair, Q4_K and Q2_K the A operand of the
// min-term MFMA (each sub-block's activation sum, hi and lo)
struct MfvStageBase {
  uint4 a[8][2][64];  // [MFMA][hi, lo][lane]
  float sx[MV_M];
};
template <int FMT>
struct MfvStage : MfvStageBase {
  // Q4_K: lane L holds pair L % 16's sums of sub-blocks 2 (L / 16) and
  // 2 (L / 16) + 1, each as (hi, lo) fp16
  uint2 xm[64];
};
template <>
struct MfvStage<NX_FMT_Q2_K> : MfvStageBase {
  // Q2_K: lane L holds pair L % 16's sums of sub-blocks 4 (L / 16) ..
  // 4 (L / 16) + 3, each as (hi, lo) fp16
  uint4 xm[64];
};
template <>
struct MfvStage<NX_FMT_Q4_0> : MfvStageBase {
  float xs[8][MV_M];  // [block][pair]: 8 times the block's sum of the operand values
};
template <>
struct MfvStage<NX_FMT_Q8_0> : MfvStageBase {
  float xs[8][MV_M];  // [block][pair]: 128 times the block's sum of the operand values
};

// 4 x 4 transpose of dwords across the four 16-lane groups: on return
// c[k] of lane group g holds what c[g] of lane group k held (register
// swaps between lane halves, then between neighbouring lane groups)
__device__ __forceinline__ void transpose_groups(uint32_t (&c)[4]) {
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const auto v = __builtin_amdgcn_permlane32_swap(c[k], c[k + 2], false, false);
    c[k] = v[0];
    c[k + 2] = v[1];
  }
#pragma unroll
  for (int k = 0; k < 4; k += 2) {
    const auto v = __builtin_amdgcn_permlane16_swap(c[k], c[k + 1], false, false);
    c[k] = v[0];
    c[k + 1] = v[1];
  }
}

// element of sub-block group g held in operand position p: the nibble order
// of a code dword (positions 2i, 2i+1 = elements i, 4+i)
__device__ __forceinline__ constexpr int opos_elem(int p) { return (p & 1) * 4 + (p >> 1); }

// one (row tile, chunk) step of a lane: Q4_K dword (lane / 16) of each
// sub-block's code half, and the block's scales (d, dmin, scales12); Q4_0
// blocks 2 g and 2 g + 1 and the chunk's 8 block scales
template <int NMAT, int FMT>
struct MfvStep {
  uint4 q[NMAT][2];  // sub-block g's code half, then sub-block g + 4's
  uint4 m[NMAT];
};
// Q8_0: blocks 2 g and 2 g + 1 of the chunk (halves 0 and 1 each) and the
// chunk's 8 block scales
template <int NMAT>
struct MfvStep<NMAT, NX_FMT_Q8_0> {
  uint4 q[NMAT][4];  // [2 t + h]: half h of block 2 g + t
  uint4 m[NMAT];
};
// Q2_K: segment g of the chunk (64 weights in 16 bytes) and its scale-plane
// entry {f16 d, f16 dmin, the segment's four scale/min bytes}
template <int NMAT>
struct MfvStep<NMAT, NX_FMT_Q2_K> {
  uint4 q[NMAT][1];
  uint2 m[NMAT];
};

// Workgroup = (row block of 256 rows, tile of <= 16 pairs, K slice of
// MV_KS chunks).  Prologue: the slice's activations of the tile's pairs are
// staged once into LDS (one barrier).  Then wave w streams rows
// 64 w .. 64 w + 63 of the block as 4 row tiles x MV_KS chunks (16 or 12 steps),
// with the codes of the next MV_D - 1 steps in flight.  Each workgroup writes
// its slice's partial sums: gate/up to part[slice][pair][2][F] (gate, then
// up), down to part[slice][pair][H].
// chunks per K slice: four for gate/up; three for down, whose 48-50 KB stage
// and at most 155 VGPRs then fit three workgroups on a CU (Mixtral 32 tokens: down
// 83 -> 80 us; 64 tokens 116 -> 109 us; two chunks, four workgroups per
// CU, gained no more and added combine work)
constexpr int MV_KS_GATEUP = 4, MV_KS_DOWN = 3;
// steps in flight + 1: gate/up one per chunk of the slice, but Q8_0,
// whose steps carry twice the code bytes (two steps in flight, for the
// registers); down one more than its slice's chunks (three steps in flight
// at 134-150 VGPRs, still three workgroups per CU: Mixtral 32 tokens down
// 78.4 -> 76.9 us, 64 tokens 94.9 -> 93.1 us; gate/up with four in flight
// was slower, 144 -> 146 us), Q8_0 as many (four slots spill)
template <bool GATEUP, int FMT>
constexpr int mv_ring() {
  if constexpr (GATEUP) return FMT == NX_FMT_Q8_0 ? 3 : MV_KS_GATEUP;
  return FMT == NX_FMT_Q8_0 ? MV_KS_DOWN : MV_KS_DOWN + 1;
}
constexpr int MV_RTW = 4;  // row tiles per wave
constexpr int MV_WG_ROWS = 4 * 16 * MV_RTW;

template <bool GATEUP, int MV_KS, int FMT, int MV_D>
__global__ __launch_bounds__(256, MV_KS == 3 ? 3 : 2) void k_mfv(const MfvArgs a) {
  static_assert(FMT == NX_FMT_Q4_K || FMT == NX_FMT_Q4_0 || FMT == NX_FMT_Q2_K ||
                    FMT == NX_FMT_Q8_0,
                "Q4_K, Q4_0, Q2_K and Q8_0 codes");
  // Q4_0 and Q8_0: one MFMA per 32-weight block, scaled per block
  constexpr bool Q40 = FMT == NX_FMT_Q4_0, Q2K = FMT == NX_FMT_Q2_K, Q80 = FMT == NX_FMT_Q8_0;
  constexpr bool BLK = Q40 || Q80;
  // MV_D ring slots: MV_D - 1 steps in flight while one is computed
  constexpr int NMAT = GATEUP ? 2 : 1;
  constexpr int NSTEP = MV_RTW * MV_KS;
  __shared__ MfvStage<FMT> stage[MV_KS];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int tile, rb, slice;
  if (a.xcd_pairs) {
    // 1-D grid: workgroup L runs on XCD L % 8, and an XCD's consecutive
    // workgroups take the two K slices of one (row block, tile) item, so the
    // 128-byte scale lines the two slices share are read through one L2 at
    // about the same time
    const int L = (int)blockIdx.x, xcd = L & 7, j = L >> 3;
    const long it = (long)(j >> 1) * 8 + xcd;
    rb = (int)(it % a.nrb);
    const long r2 = it / a.nrb;
    tile = (int)(r2 % a.ntiles_g);
    slice = 2 * (int)(r2 / a.ntiles_g) + (j & 1);
    if (slice >= a.nks) return;  // workgroup-uniform (items past the last)
  } else {
    tile = blockIdx.y;
    rb = blockIdx.x;
    slice = blockIdx.z;
  }
  if (tile >= a.tiles[0]) return;  // workgroup-uniform
  // tile t: expert tiles[2 + 2t] (E: the shared expert), first pair
  // tiles[3 + 2t] within the expert.  These and the expert's offsets are
  // scalar loads, which do not queue behind the weight stream's vector loads
  // (loading every expert's offset with vector loads ahead of the expert id
  // was slower: Mixtral 32 tokens 266 -> 274 us)
  const int e = __builtin_amdgcn_readfirstlane(a.tiles[2 + 2 * tile]);
  const int m0 = __builtin_amdgcn_readfirstlane(a.tiles[3 + 2 * tile]);
  const bool routed = e < a.E;
  const int pair0 = __builtin_amdgcn_readfirstlane(routed ? a.offsets[e] + m0 : a.T * a.k + m0);
  const int cnt = __builtin_amdgcn_readfirstlane(
      min(MV_M, routed ? a.offsets[e + 1] - pair0 : a.T - m0));
  const int c0 = slice * MV_KS;  // first chunk of the slice
  const int row_base = rb * MV_WG_ROWS + wave * 16 * MV_RTW;

  // ---- weights: lane holds row (lane % 16) of each row tile and K group
  // (lane / 16) of every sub-block
  const int l16 = lane & 15, g = lane >> 4;
  __amdgpu_buffer_rsrc_t rq[NMAT], rm[NMAT];
  {
    const uint32_t nq = (uint32_t)a.rows * a.row_qs, nm = (uint32_t)a.rows * a.row_meta;
    rq[0] = make_rsrc(routed ? a.qs0 + (size_t)e * a.qs_stride : a.sqs0, nq);
    rm[0] = make_rsrc(routed ? a.meta0 + (size_t)e * a.meta_stride : a.smeta0, nm);
    if constexpr (NMAT == 2) {
      rq[1] = make_rsrc(routed ? a.qs1 + (size_t)e * a.qs_stride : a.sqs1, nq);
      rm[1] = make_rsrc(routed ? a.meta1 + (size_t)e * a.meta_stride : a.smeta1, nm);
    }
  }
  // step i: row tile i / MV_KS, chunk c0 + i % MV_KS
  // The planes are in panels of 64 segments (nx_device.hpp): the chunk's
  // panel grp starts at grp * rows * prq (codes) and grp * rows * prm
  // (scales), prq and prm a row's bytes in a panel, and holds gsz segments
  // of each row.  Rows past the matrix and chunks past the row (wave-uniform)
  // read at OOB.  Per-lane parts
  // of the offsets stay in one register per step; the rest goes in the scalar
  // offset.
  auto issue = [&](MfvStep<NMAT, FMT> &w, int i) {
    const int row = row_base + 16 * (i / MV_KS) + l16;
    const int c = c0 + i % MV_KS;
    if constexpr (Q2K) {
      // 16 bytes of codes and 8 of scales per segment: segment 4c + g at
      // 16 (j % 64) and 8 (j % 64) of the row's part of its panel; the 4
      // lanes of a row read 64 contiguous code bytes
      const int j0 = 4 * c;
      const int grp = j0 >> 6;
      const uint32_t prq = panel_row_bytes(a.nseg, 16), prm = panel_row_bytes(a.nseg, 8);
      const uint32_t base = (uint32_t)grp * (uint32_t)a.rows * prq + (uint32_t)((j0 & 63) * 16);
      const uint32_t mbase = (uint32_t)grp * (uint32_t)a.rows * prm + (uint32_t)((j0 & 63) * 8);
      const bool cv = i < NSTEP && c < a.nchunk && row < a.rows;
      const uint32_t vq = cv ? (uint32_t)row * prq + 16u * g : OOB;
      const uint32_t vm = cv ? (uint32_t)row * prm + 8u * g : OOB;
#pragma unroll
      for (int mt = 0; mt < NMAT; ++mt) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(rq[mt], (int)vq, (int)base, 0);
        w.q[mt][0] = make_uint4(v[0], v[1], v[2], v[3]);
        const auto u = __builtin_amdgcn_raw_buffer_load_b64(rm[mt], (int)vm, (int)mbase, 0);
        w.m[mt] = make_uint2(u[0], u[1]);
      }
    } else if constexpr (Q80) {
      // 8 segments (blocks) per chunk, in one group of 64: half h of
      // segment 8c + 2g + t sits at base + h 16 gsz + 32 g + 16 t; the
      // chunk's 8 f16 scales are 16 bytes of the scale plane's panel row
      const int j0 = 8 * c;
      const int grp = j0 >> 6;
      const int gsz = min(64, a.nseg - (grp << 6));
      const uint32_t prq = panel_row_bytes(a.nseg, 32), prm = panel_row_bytes(a.nseg, 2);
      const uint32_t base = (uint32_t)grp * (uint32_t)a.rows * prq + (uint32_t)((j0 & 63) * 16);
      const bool cv = i < NSTEP && c < a.nchunk && row < a.rows;
      const uint32_t vq = cv ? (uint32_t)row * prq + 32u * g : OOB;
      const uint32_t vm = cv ? ((uint32_t)grp * (uint32_t)a.rows + (uint32_t)row) * prm + 2u * (uint32_t)(j0 & 63)
                             : OOB;
#pragma unroll
      for (int mt = 0; mt < NMAT; ++mt) {
#pragma unroll
        for (int th = 0; th < 4; ++th) {
          const int t = th >> 1, h = th & 1;
          const auto v = __builtin_amdgcn_raw_buffer_load_b128(
              rq[mt], (int)vq, (int)(base + h * 16u * gsz + 16u * t), 0);
          w.q[mt][th] = make_uint4(v[0], v[1], v[2], v[3]);
        }
        w.m[mt] = bload16(rm[mt], vm);
      }
    } else {
      // the chunk's 4 segments share one group of 64: half h of segment
      // 4c + g sits at base + h 16 gsz + 16 g; the 4 lanes of a row read 64
      // contiguous bytes per half
      const int j0 = 4 * c;
      const int grp = j0 >> 6;
      const int gsz = min(64, a.nseg - (grp << 6));
      const uint32_t prq = panel_row_bytes(a.nseg, 32), prm = panel_row_bytes(a.nseg, 4);
      const uint32_t base = (uint32_t)grp * (uint32_t)a.rows * prq + (uint32_t)((j0 & 63) * 16);
      // steps past the last (issued by the pipeline's tail), chunks past the
      // row (wave-uniform) and rows past the matrix read at OOB
      const bool cv = i < NSTEP && c < a.nchunk && row < a.rows;
      const uint32_t vq = cv ? (uint32_t)row * prq + 16u * g : OOB;
      const uint32_t vm = cv ? ((uint32_t)grp * (uint32_t)a.rows + (uint32_t)row) * prm + 16u * (uint32_t)(c - 16 * grp)
                             : OOB;
#pragma unroll
      for (int mt = 0; mt < NMAT; ++mt) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const auto v = __builtin_amdgcn_raw_buffer_load_b128(rq[mt], (int)vq,
                                                               (int)(base + h * 16u * gsz), 0);
          w.q[mt][h] = make_uint4(v[0], v[1], v[2], v[3]);
        }
        w.m[mt] = bload16(rm[mt], vm);
      }
    }
  };

  // ---- stage the slice: thread t owns positions 16j .. 16j+15 of every
  // chunk of pair m = t / 16; chunks past the row read as zeros.  The token
  // lookup and the activation loads go out before the first weight steps:
  // vector loads complete in issue order, so activation loads issued after
  // the weights would wait for them (at 32 tokens the staging then took
  // ~12 of a ~38 us workgroup), while the weights are needed only after the
  // staging's barrier anyway.
  const int sm = tid >> 4, sj = tid & 15;
  const float *xrow = nullptr;
  if (sm < cnt) {
    // gate/up: the pair's token (a shared pair's is its index in the
    // tile's run); down: the pair's row of act
    const int r = a.perm_token ? (routed ? a.perm_token[pair0 + sm] : m0 + sm) : pair0 + sm;
    xrow = a.x + (size_t)r * a.x_stride;
  }
  // every lane loads (absent pairs and chunks from row 0 of x, zeroed when
  // converted), so the loads are not branched around
  const bool pv = xrow != nullptr;
  if (!pv) xrow = a.x;
  float4 xr[MV_KS][4];
#pragma unroll
  for (int kc = 0; kc < MV_KS; ++kc) {
    const bool v = pv && c0 + kc < a.nchunk;
    const float *src = xrow + (size_t)(v ? c0 + kc : 0) * MV_K + 16 * sj;
#pragma unroll
    for (int q = 0; q < 4; ++q) xr[kc][q] = *reinterpret_cast<const float4 *>(src + 4 * q);
  }
  __builtin_amdgcn_sched_barrier(0);

  // the first weight steps, in flight during the staging
  MfvStep<NMAT, FMT> ring[MV_D];
#pragma unroll
  for (int i = 0; i < MV_D - 1; ++i) issue(ring[i], i);
  __builtin_amdgcn_sched_barrier(0);

  {
    float xv[MV_KS][16];
#pragma unroll
    for (int kc = 0; kc < MV_KS; ++kc) {
      const bool v = pv && c0 + kc < a.nchunk;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        xv[kc][4 * q] = v ? xr[kc][q].x : 0.f;
        xv[kc][4 * q + 1] = v ? xr[kc][q].y : 0.f;
        xv[kc][4 * q + 2] = v ? xr[kc][q].z : 0.f;
        xv[kc][4 * q + 3] = v ? xr[kc][q].w : 0.f;
      }
    }
#pragma unroll
    for (int kc = 0; kc < MV_KS; ++kc) {
      MfvStage<FMT> &st = stage[kc];
      float mx = 0.f;
#pragma unroll
      for (int v = 0; v < 16; ++v) mx = fmaxf(mx, fabsf(xv[kc][v]));
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
      // max|x| < 2^E; scale the chunk maximum into [2^13, 2^14)
      int E = 0;
      if (mx > 0.f && mx <= 3.4e38f) {
        (void)frexpf(mx, &E);
        E = max(E, -100);
      }
      const float up = __builtin_amdgcn_ldexpf(1.0f, 14 - E);
      // x' = x 2^(14-E) = hi + lo; the sub-block sums are of hi + lo, the
      // values the operands carry
      _Float16 hv[16], lv[16];
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float sv = xv[kc][v] * up;
        hv[v] = (_Float16)sv;
        lv[v] = (_Float16)(sv - (float)hv[v]);
      }
      // Operands, Q4_K: MFMA u (0..7), lane group g takes elements
      // 32 g + 8 u (u < 4) or 128 + 32 g + 8 (u - 4) (u >= 4), position p
      // holding element + opos_elem(p).  This thread's 16 positions
      // 16 sj .. 16 sj + 15 are those of group g = (sj % 8) / 2, MFMAs
      // u0, u0 + 1 with u0 = 4 (sj / 8) + 2 (sj % 2).  Q4_0: MFMA b is
      // block b (elements 32 b ..), lane group g taking its elements
      // 32 b + 8 g + opos_elem(p); this thread's positions are block sj / 2,
      // groups 2 (sj % 2) and 2 (sj % 2) + 1.  Q2_K: lane group g takes
      // segment g (elements 64 g ..), MFMA u its elements 32 (u / 4) +
      // 8 (u % 4) + opos_elem(p) (dword u % 4 of half u / 4); this thread's
      // positions are segment sj / 4, half (sj / 2) % 2, dwords 2 (sj % 2)
      // and 2 (sj % 2) + 1.
#pragma unroll
      for (int uu = 0; uu < 2; ++uu) {
        _Float16 ho[8], lo[8];
#pragma unroll
        for (int p = 0; p < 8; ++p) {
          // Q8_0 operands hold their 8 codes in element order
          const int e = Q80 ? p : opos_elem(p);
          ho[p] = hv[8 * uu + e];
          lo[p] = lv[8 * uu + e];
        }
        const int gq = BLK ? 2 * (sj & 1) + uu : Q2K ? sj >> 2 : (sj & 7) >> 1;
        const int u = BLK   ? sj >> 1
                      : Q2K ? 4 * ((sj >> 1) & 1) + 2 * (sj & 1) + uu
                            : 4 * (sj >> 3) + 2 * (sj & 1) + uu;
        const int L = sm + 16 * gq;
        st.a[u][0][L] = __builtin_bit_cast(uint4, ho);
        st.a[u][1][L] = __builtin_bit_cast(uint4, lo);
      }
      // the sums of the values the operands carry (hi + lo) over this
      // thread's 16 positions: Q2_K sub-block sj; with the neighbour's, Q4_0
      // block sj / 2 and Q4_K sub-block sj / 2
      float bs = 0.f;
#pragma unroll
      for (int v = 0; v < 16; ++v) bs += (float)hv[v] + (float)lv[v];
      if constexpr (!Q2K) bs += __shfl_xor(bs, 1, 64);
      if constexpr (BLK) {
        // the codes' offset times the block sum: Q4_0 8, Q8_0 128
        if ((sj & 1) == 0) st.xs[sj >> 1][sm] = (Q80 ? 128.0f : 8.0f) * bs;
      } else {
        // the min-term operand: X 2^-6 (|X| <= 32 x 2^14) as hi + lo fp16
        const float xq = bs * 0.015625f;
        const _Float16 xh = (_Float16)xq, xl = (_Float16)(xq - (float)xh);
        const uint32_t hl = (uint32_t)__builtin_bit_cast(uint16_t, xh) |
                            ((uint32_t)__builtin_bit_cast(uint16_t, xl) << 16);
        if constexpr (Q2K) {
          (&st.xm[sm + 16 * (sj >> 2)].x)[sj & 3] = hl;
        } else {
          const int sb = sj >> 1;  // sub-block
          if ((sj & 1) == 0) (&st.xm[sm + 16 * (sb >> 1)].x)[sb & 1] = hl;
        }
      }
      if (sj == 0) st.sx[sm] = __builtin_amdgcn_ldexpf(1.0f, E - 14);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  __syncthreads();

  // q 2^-24 sc as fp16 bits (q sc <= 945 < 1024: an exact subnormal) for
  // the 8 unsigned codes of a dword, in nibble order (the 4-bit planes hold
  // q ^ 8: their callers flip it back)
  auto operand = [](uint32_t cw, uint32_t sc2) {
    const uint32_t lo = cw & 0x0F0F0F0Fu, hi = (cw >> 4) & 0x0F0F0F0Fu;
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    const u16x2 sv = __builtin_bit_cast(u16x2, sc2);
    uint32_t d[4];
    d[0] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(hi, lo, 0x0C040C00u)) * sv);
    d[1] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(hi, lo, 0x0C050C01u)) * sv);
    d[2] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(hi, lo, 0x0C060C02u)) * sv);
    d[3] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(hi, lo, 0x0C070C03u)) * sv);
    return __builtin_bit_cast(f16x8, d);
  };

  // step (row tile rt, chunk kc) into accr, the row tile's accumulators:
  //   sum_i w_i x_i = d sum_s sc_s sum_{i in s} q_i x_i - dmin sum_s m_s X_s
  // with sc_s inside the operands, so the 8 MFMAs of the block accumulate
  // together and d, dmin apply once per block
  auto compute = [&](const MfvStep<NMAT, FMT> &w, const MfvStage<FMT> &st, f32x4 (&accr)[NMAT]) {
    if constexpr (BLK) {
      // Q4_0 (src/quant/mod.rs:723-745: w = d (q - 8) per 32-weight block)
      // and Q8_0 (src/quant/mod.rs:689-703: w = d q, q a signed byte).  One
      // MFMA per block: lane group g holds the block's elements 8 g ..
      // 8 g + 7, so the block scale d applies to the MFMA's result; the
      // codes go in unsigned, q + o as an fp16 subnormal ((q + o) 2^-24,
      // Q4_0 o = -8 + 8 from the stored q ^ 8, Q8_0 o = 128), and the staged
      // block sums X take off the offset:
      //   sum_i w_i x_i = d (2^24 sum_i ((q_i + o) 2^-24) x_i - o X).
      // Q4_0: the loads give lane group g the 16 bytes of blocks 2 g and
      // 2 g + 1 (halves 0 and 1 of segment g); transposed across the lane
      // groups, dword s of half h is then dword g of block 2 s + h.  Q8_0:
      // lane group g loads blocks 2 g + t (t = 0, 1) whole; the dword pairs
      // (2 k, 2 k + 1) transposed across the lane groups, pair s of parity t
      // is then dwords 2 g, 2 g + 1 of block 2 s + t.
      constexpr int NW = Q80 ? 2 : 1;  // code dwords per lane and MFMA
      uint32_t cq[NMAT][2][NW][4];
#pragma unroll
      for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if constexpr (Q80) {
            const uint4 q0 = w.q[mt][2 * h], q1 = w.q[mt][2 * h + 1];  // block 2 g + h
            const uint32_t lo[4] = {q0.x, q0.z, q1.x, q1.z}, hi[4] = {q0.y, q0.w, q1.y, q1.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              cq[mt][h][0][k] = lo[k];
              cq[mt][h][NW - 1][k] = hi[k];
            }
          } else {
            cq[mt][h][0][0] = w.q[mt][h].x;
            cq[mt][h][0][1] = w.q[mt][h].y;
            cq[mt][h][0][2] = w.q[mt][h].z;
            cq[mt][h][0][3] = w.q[mt][h].w;
          }
#pragma unroll
          for (int v = 0; v < NW; ++v) transpose_groups(cq[mt][h][v]);
        }
      // Q8_0: (q ^ 0x80) = q + 128 per byte, each byte widened to 16 bits
      // in element order: the bits of the fp16 subnormal (q + 128) 2^-24
      auto operand8 = [](uint32_t lo, uint32_t hi) {
        lo ^= 0x80808080u;
        hi ^= 0x80808080u;
        uint32_t d[4];
        d[0] = __builtin_amdgcn_perm(lo, lo, 0x0C010C00u);
        d[1] = __builtin_amdgcn_perm(lo, lo, 0x0C030C02u);
        d[2] = __builtin_amdgcn_perm(hi, hi, 0x0C010C00u);
        d[3] = __builtin_amdgcn_perm(hi, hi, 0x0C030C02u);
        return __builtin_bit_cast(f16x8, d);
      };
      float sx[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) sx[k] = st.sx[4 * g + k];
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const f16x8 ahi = __builtin_bit_cast(f16x8, st.a[b][0][lane]);
        const f16x8 alo = __builtin_bit_cast(f16x8, st.a[b][1][lane]);
        const float4 xs = *reinterpret_cast<const float4 *>(&st.xs[b][4 * g]);
#pragma unroll
        for (int mt = 0; mt < NMAT; ++mt) {
          const f16x8 bq = Q80 ? operand8(cq[mt][b & 1][0][b >> 1], cq[mt][b & 1][NW - 1][b >> 1])
                               : operand(cq[mt][b & 1][0][b >> 1] ^ 0x88888888u, 0x00010001u);
          f32x4 y = f32x4{0.f, 0.f, 0.f, 0.f};
          y = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bq, y, 0, 0, 0);
          y = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bq, y, 0, 0, 0);
          asm volatile("" : "+v"(y));
          // block b's scale: the f16 at half (b % 2) of scale dword b / 2
          const uint32_t dw = (&w.m[mt].x)[b >> 1];
          const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(b & 1 ? dw >> 16 : dw & 0xFFFFu));
          accr[mt][0] = fmaf(sx[0] * d, fmaf(16777216.0f, y[0], -xs.x), accr[mt][0]);
          accr[mt][1] = fmaf(sx[1] * d, fmaf(16777216.0f, y[1], -xs.y), accr[mt][1]);
          accr[mt][2] = fmaf(sx[2] * d, fmaf(16777216.0f, y[2], -xs.z), accr[mt][2]);
          accr[mt][3] = fmaf(sx[3] * d, fmaf(16777216.0f, y[3], -xs.w), accr[mt][3]);
          // the block's scaling happens here: left free, the compiler sinks
          // every block's scaling to the step's end and holds all 8 blocks'
          // results meanwhile (1480 bytes of spills per lane)
          asm volatile("" : "+v"(accr[mt]));
        }
      }
    } else {
      // Q4_K: this lane's sub-blocks g and g + 4 (get_scale_min_k4,
      // src/quant/mod.rs:1163-1170, on scales12), MFMAs u < 4 and u >= 4.
      // Q2_K (src/quant/mod.rs:913-937: w = d sc q - dmin m per 16-weight
      // sub-block, sc and m the low and high nibble of its scale byte): this
      // lane's sub-blocks 4 g + v, v = u / 2, from the segment's four scale
      // bytes.  The scales go into the code operands.  sum_s m_s X_s is one
      // more MFMA per chunk, on the staged sub-block sums X_s (hi, lo) and
      // the row's mins (each twice, for hi and lo): Q4_K K = 16 (lane group g
      // takes sub-blocks 2 g, 2 g + 1), Q2_K K = 32 (sub-blocks 4 g ..
      // 4 g + 3).  (Mins in operands of their own under every code MFMA
      // cost 16 MFMAs per chunk instead of one: Mixtral 32 tokens 262 ->
      // 247 us, Q2_K 64 tokens 285 -> 248 us.)
      constexpr int NV = Q2K ? 4 : 2;
      uint32_t sc2[NMAT][NV], bm[NMAT][NV];
#pragma unroll
      for (int mt = 0; mt < NMAT; ++mt) {
        uint32_t scv[NV], mnv[NV];
        if constexpr (Q2K) {
#pragma unroll
          for (int v = 0; v < NV; ++v) {
            scv[v] = (w.m[mt].y >> (8 * v)) & 15;
            mnv[v] = (w.m[mt].y >> (8 * v + 4)) & 15;
          }
        } else {
          const uint32_t p03 = w.m[mt].y, p47 = w.m[mt].z, p8b = w.m[mt].w;
          scv[0] = (p03 >> (8 * g)) & 63;
          scv[1] = ((p8b >> (8 * g)) & 15) | (((p03 >> (8 * g + 6)) & 3) << 4);
          // mins of sub-blocks j = 2 g + v: j < 4 from p47 alone, j >= 4
          // from p8b's high nibble and p47's top bits
#pragma unroll
          for (int v = 0; v < 2; ++v) {
            const int jb = 8 * ((2 * g + v) & 3);
            const uint32_t lo6 = (p47 >> jb) & 63;
            const uint32_t hi6 = ((p8b >> (jb + 4)) & 15) | (((p47 >> (jb + 6)) & 3) << 4);
            mnv[v] = g < 2 ? lo6 : hi6;
          }
        }
#pragma unroll
        for (int v = 0; v < NV; ++v) {
          sc2[mt][v] = scv[v] | (scv[v] << 16);
          bm[mt][v] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)mnv[v]) * 0x10001u;
        }
      }
      f32x4 y[NMAT], ym[NMAT];
#pragma unroll
      for (int mt = 0; mt < NMAT; ++mt) {
        y[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
        if constexpr (Q2K) {
          const uint4 xa = st.xm[lane];
          const uint32_t av[4] = {xa.x, xa.y, xa.z, xa.w};
          ym[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, av),
                                                          __builtin_bit_cast(f16x8, bm[mt]),
                                                          f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        } else {
          const uint2 xa = st.xm[lane];
          const uint32_t av[2] = {xa.x, xa.y};
          ym[mt] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, av),
                                                         __builtin_bit_cast(f16x4, bm[mt]),
                                                         f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        }
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const f16x8 ahi = __builtin_bit_cast(f16x8, st.a[u][0][lane]);
        const f16x8 alo = __builtin_bit_cast(f16x8, st.a[u][1][lane]);
#pragma unroll
        for (int mt = 0; mt < NMAT; ++mt) {
          uint32_t cw;
          if constexpr (Q2K)  // the 2-bit codes of half u / 4 widened to nibbles (no offset)
            cw = ((&w.q[mt][0].x)[u & 3] >> (2 * (u >> 2))) & 0x33333333u;
          else
            cw = (u < 4 ? (&w.q[mt][0].x)[u] : (&w.q[mt][1].x)[u - 4]) ^ 0x88888888u;
          constexpr int vsh = Q2K ? 1 : 2;
          const f16x8 b = operand(cw, sc2[mt][u >> vsh]);
          y[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, b, y[mt], 0, 0, 0);
          y[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, b, y[mt], 0, 0, 0);
        }
        // one MFMA step's operands live at a time: make the accumulators
        // exist here, or the compiler gathers every step's operands first.
        // Each is pinned as one register tuple (pinning its four elements
        // separately made the compiler move them between registers: ~64
        // extra moves per step)
#pragma unroll
        for (int mt = 0; mt < NMAT; ++mt) asm volatile("" : "+v"(y[mt]));
      }
      float sx[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) sx[k] = st.sx[4 * g + k];
#pragma unroll
      for (int mt = 0; mt < NMAT; ++mt) {
        const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(w.m[mt].x & 0xFFFF));
        const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(w.m[mt].x >> 16));
        const float dd = d * 16777216.0f;  // code operands carry 2^-24
        const float dm = dmin * 64.0f;     // the min-term operands carry X 2^-6
#pragma unroll
        for (int k = 0; k < 4; ++k)
          accr[mt][k] = fmaf(sx[k], fmaf(dd, y[mt][k], -dm * ym[mt][k]), accr[mt][k]);
      }
    }
  };

  // steps i = MV_KS rt + kc: stage kc, ring slot i % MV_D
  float *out = a.out + (size_t)slice * a.out_split;
  // fully unrolled: ring registers carried around a loop back edge get
  // copied there, and copying a register with a load in flight waits for it
#pragma unroll
  for (int rt = 0; rt < MV_RTW; ++rt) {
    f32x4 accr[NMAT];
#pragma unroll
    for (int mt = 0; mt < NMAT; ++mt) accr[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < MV_KS; ++kc) {
      const int i = MV_KS * rt + kc;
      // issued unconditionally: a branch around the loads would leave the
      // compiler unsure how many are outstanding, and it would then wait
      // for all of them
      issue(ring[(i + MV_D - 1) % MV_D], i + MV_D - 1);
      compute(ring[i % MV_D], stage[kc], accr);
      __builtin_amdgcn_sched_barrier(0);
    }
    // partial sums of the slice: lane holds row (lane % 16), pairs 4g .. 4g+3
    const int row = row_base + 16 * rt + l16;
    if (row < a.rows) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int m = 4 * g + k;
        if (m >= cnt) continue;
        const size_t o = (size_t)(pair0 + m) * a.out_stride + row;
        out[o] = accr[0][k];
        if constexpr (GATEUP) out[o + a.rows] = accr[1][k];
      }
    }
  }
}

// act[p][f] = silu(sum_s gate_s[p][f]) * sum_s up_s[p][f] over the K slices
// of the gate/up pass, summed in slice order.  Four consecutive columns per
// thread (F % 4 == 0, 16-byte aligned buffers); the slices are loaded SB at
// a time (past the last slice clamped to it) before any is added, so up to
// SB slices take one round of loads, and added by per-component selects.
template <int SB>
__global__ __launch_bounds__(256) void k_mfv_swiglu(const float *__restrict__ part, int nslice,
                                                    size_t slice_stride, int pairs, int F,
                                                    float *__restrict__ act) {
  const int F4 = F >> 2;
  const size_t n4 = (size_t)pairs * F4;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n4;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t p = i / F4;
    const size_t f = 4 * (i - p * F4);
    const size_t o = p * 2 * F + f;
    float4 g = make_float4(0.f, 0.f, 0.f, 0.f), u = g;
    for (int s0 = 0; s0 < nslice; s0 += SB) {
      float4 gv[SB], uv[SB];
#pragma unroll
      for (int j = 0; j < SB; ++j) {
        const size_t so = (size_t)min(s0 + j, nslice - 1) * slice_stride + o;
        gv[j] = *reinterpret_cast<const float4 *>(part + so);
        uv[j] = *reinterpret_cast<const float4 *>(part + so + F);
      }
#pragma unroll
      for (int j = 0; j < SB; ++j) {
        const bool first = s0 + j == 0, in = s0 + j < nslice;
        const float a[4] = {g.x, g.y, g.z, g.w}, b[4] = {u.x, u.y, u.z, u.w};
        const float ga[4] = {gv[j].x, gv[j].y, gv[j].z, gv[j].w};
        const float ua[4] = {uv[j].x, uv[j].y, uv[j].z, uv[j].w};
        float rg[4], ru[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          rg[c] = first ? ga[c] : (in ? a[c] + ga[c] : a[c]);
          ru[c] = first ? ua[c] : (in ? b[c] + ua[c] : b[c]);
        }
        g = make_float4(rg[0], rg[1], rg[2], rg[3]);
        u = make_float4(ru[0], ru[1], ru[2], ru[3]);
      }
    }
    *reinterpret_cast<float4 *>(act + p * F + f) =
        make_float4(silu_mul(g.x, u.x), silu_mul(g.y, u.y), silu_mul(g.z, u.z), silu_mul(g.w, u.w));
  }
}

// the kernel of a pass for the experts' format
template <bool GATEUP, int KS>
void (*mfv_kernel(int fmt))(MfvArgs) {
  switch (fmt) {
  case NX_FMT_Q4_0: return k_mfv<GATEUP, KS, NX_FMT_Q4_0, mv_ring<GATEUP, NX_FMT_Q4_0>()>;
  case NX_FMT_Q8_0: return k_mfv<GATEUP, KS, NX_FMT_Q8_0, mv_ring<GATEUP, NX_FMT_Q8_0>()>;
  case NX_FMT_Q2_K: return k_mfv<GATEUP, KS, NX_FMT_Q2_K, mv_ring<GATEUP, NX_FMT_Q2_K>()>;
  default: return k_mfv<GATEUP, KS, NX_FMT_Q4_K, mv_ring<GATEUP, NX_FMT_Q4_K>()>;
  }
}

}  // namespace

int mfv_max_tiles(int T, int k, int E, bool shared) {
  const long pairs = (long)T * k;
  return (int)((pairs + MV_M - 1) / MV_M + std::min<long>(E, pairs) +
               (shared ? (T + MV_M - 1) / MV_M : 0));
}

bool mfv_supports(const nx_experts *ex) {
  // whole 256-weight chunks in both products: Q4_K and Q2_K always, Q4_0
  // and Q8_0 when H and F are multiples of 256
  if (ex->fmt == NX_FMT_Q4_K || ex->fmt == NX_FMT_Q2_K) return true;
  return (ex->fmt == NX_FMT_Q4_0 || ex->fmt == NX_FMT_Q8_0) && ex->H % MV_K == 0 &&
         ex->F % MV_K == 0;
}

int launch_mfv(nx_ctx *c, const MfvPlan &p) {
  const nx_experts *ex = p.ex;
  if (!mfv_supports(ex))
    return fail(NX_ERR_UNSUPPORTED,
                "the split-activation MFMA path takes Q4_K and Q2_K experts, or Q4_0 and Q8_0 "
                "experts whose hidden and FFN widths are multiples of 256");
  // activation rows are read as float4 runs of whole chunks
  if (reinterpret_cast<uintptr_t>(p.x) & 15)
    return fail(NX_ERR_UNSUPPORTED, "the split-activation MFMA path needs 16-byte aligned inputs");
  const bool shared = ex->Fs > 0;
  if (shared && ex->Fs != ex->F)
    return fail(NX_ERR_UNSUPPORTED,
                "the split-activation MFMA path takes a shared expert as wide as the routed ones");
  const int H = ex->H, F = ex->F;
  // routed pairs, then one pair per token for the shared expert
  const size_t pairs = (size_t)p.T * p.k + (shared ? (size_t)p.T : 0);
  const int nks_g = (H / MV_K + MV_KS_GATEUP - 1) / MV_KS_GATEUP;
  const int nks_d = (F / MV_K + MV_KS_DOWN - 1) / MV_KS_DOWN;
  void *vg, *va, *vy;
  NX_TRY(ws_get(c, WS_MFV_PART, (size_t)nks_g * pairs * 2 * F * sizeof(float), &vg));
  NX_TRY(ws_get(c, WS_ACT, pairs * F * sizeof(float), &va));
  NX_TRY(ws_get(c, WS_YPAIR, (size_t)nks_d * pairs * H * sizeof(float), &vy));
  float *gpart = static_cast<float *>(vg), *act = static_cast<float *>(va),
        *ypart = static_cast<float *>(vy);
  for (int pass = 0; pass < 2; ++pass) {
    const bool gateup = pass == 0;
    const RolePlane &R0 = ex->role[gateup ? NX_ROLE_GATE : NX_ROLE_DOWN];
    const RolePlane &R1 = ex->role[gateup ? NX_ROLE_UP : NX_ROLE_DOWN];
    MfvArgs a{};
    a.qs0 = R0.qs;
    a.qs1 = R1.qs;
    a.meta0 = R0.meta;
    a.meta1 = R1.meta;
    a.qs_stride = R0.qs_stride;
    a.meta_stride = R0.meta_stride;
    a.row_qs = R0.row_qs;
    a.row_meta = R0.row_meta;
    a.rows = R0.rows;
    a.nseg = R0.nseg;
    a.nchunk = R0.cols / MV_K;
    a.offsets = p.offsets;
    a.tiles = p.tiles;
    a.E = ex->E;
    a.T = p.T;
    a.k = p.k;
    if (shared) {
      const RolePlane &S0 = ex->shared[gateup ? NX_ROLE_GATE : NX_ROLE_DOWN];
      const RolePlane &S1 = ex->shared[gateup ? NX_ROLE_UP : NX_ROLE_DOWN];
      a.sqs0 = S0.qs;
      a.sqs1 = S1.qs;
      a.smeta0 = S0.meta;
      a.smeta1 = S1.meta;
    }
    if (gateup) {
      a.x = p.x;
      a.x_stride = H;
      a.perm_token = p.perm_token;
      a.out = gpart;
      a.out_stride = 2 * F;
      a.out_split = pairs * 2 * F;
    } else {
      a.x = act;
      a.x_stride = F;
      a.perm_token = nullptr;
      a.out = ypart;
      a.out_stride = H;
      a.out_split = pairs * H;
    }
    const int nks = gateup ? nks_g : nks_d;
    a.nrb = (a.rows + MV_WG_ROWS - 1) / MV_WG_ROWS;
    a.ntiles_g = p.max_tiles;
    a.nks = nks;
    // slice pairs on one XCD where a 128-byte scale line spans two slices
    // (16 scale bytes per chunk: Q4_K, Q4_0, Q8_0) and the slices pair up
    // (Qwen3 64 tokens 125 -> 120 us, Mixtral 32 tokens 245.5 -> 243.3 us;
    // with an odd count the unpaired slices' idle workgroups cost more than
    // the sharing gains: DeepSeek's 7 gate/up slices 459 -> 488 us)
    a.xcd_pairs = gateup && nks % 2 == 0 && ex->fmt != NX_FMT_Q2_K ? 1 : 0;
    const long items = (long)a.nrb * a.ntiles_g * (nks / 2);
    const dim3 grid = a.xcd_pairs ? dim3((unsigned)(16 * ((items + 7) / 8)))
                                  : dim3((unsigned)a.nrb, (unsigned)p.max_tiles, (unsigned)nks);
    if (gateup) {
      const auto kern = mfv_kernel<true, MV_KS_GATEUP>(ex->fmt);
      NX_TRY(launch(c, "mfv_gateup", [&] { go(c, kern, grid, dim3(256), 0, a); }));
      // (measured against one column per thread and a slice per round of
      // loads: Mixtral 32 tokens 6.8 -> 6.6 us, DeepSeek 32 tokens with its
      // 7 slices 9.6 -> 7.9 us)
      const size_t n4 = pairs * F / 4;
      const unsigned gs = (unsigned)std::min<size_t>((n4 + 255) / 256, 65536);
      auto swiglu = [&](auto kern) {
        return launch(c, "mfv_swiglu", [&] {
          go(c, kern, dim3(gs), dim3(256), 0, gpart, nks_g, pairs * 2 * F, (int)pairs, F, act);
        });
      };
      NX_TRY(nks_g <= 2 ? swiglu(k_mfv_swiglu<2>)
                        : nks_g <= 4 ? swiglu(k_mfv_swiglu<4>) : swiglu(k_mfv_swiglu<8>));
    } else {
      const auto kern = mfv_kernel<false, MV_KS_DOWN>(ex->fmt);
      NX_TRY(launch(c, "mfv_down", [&] { go(c, kern, grid, dim3(256), 0, a); }));
    }
  }
  return launch_combine(c, ypart, p.rw, p.rcnt, p.inv, p.T, p.k, H, shared, p.out, nks_d,
                        pairs * (size_t)H, p.residual);
}

}  // namespace nx
