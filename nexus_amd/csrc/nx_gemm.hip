// nx_gemm.hip — prefill path: grouped GEMM over the resident quantized
// experts on CDNA4 MFMA (fp16 or bf16 operands, fp32 accumulate).
//
// Replaces, for many tokens per expert, the matvec/SwiGLU/matvec sequence of
// dispatch_moe_ffn (src/engine/mod.rs:994-1017) applied token by token:
//   gate/up: act[p] = silu(W_gate . x[tok(p)]) * (W_up . x[tok(p)])  for the
//            pairs p of each expert, written as fp16/bf16;
//   down:    y[p] = W_down . act[p]  (fp32), then the route-weighted combine.
//
// Work decomposition.  The permutation kernel lists M-tiles (expert, first
// pair) of 128 pairs; the 1-D grid covers (M-tile, 128-row N-tile) pairs in
// an XCD-aware order (see k_gemm; extra workgroups exit).  A workgroup of 4 waves owns
// a 128x128 output tile (gate/up: two of them, for the gate and the up rows);
// wave w owns weight rows 32w .. 32w+31 of the tile for all 128 pairs, as
// 4 v_mfma_f32_32x32x16 tiles per matrix.
//
// K loop, 64 elements per step (one Q4_K segment = sub-blocks s and s+4 of a
// block, two Q8_0 / Q4_0 blocks, or 64 F32 values).  The activation tile is
// gathered row by row through the permutation into LDS, shared by the four
// waves.  The weights never pass through LDS: lane l of wave w dequantizes
// half l/32 of the step for weight row 32w + l%32 (32 values, bit-exact f32,
// rounded once to the operand type) straight into its MFMA B operands.  Within
// a step, MFMA sub-step kk uses, for lane half h, the K positions
// 32h + 8kk .. 32h + 8kk + 7; the A operands read the same positions from LDS.
// The codes and scales of the next step are fetched while the MFMAs of the
// current step run.
#include <type_traits>

#include "nx_device.hpp"
#include "nx_internal.hpp"

namespace nx {

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128;   // pairs per tile
constexpr int BN = 128;   // weight rows per tile
constexpr int BK = 64;    // K elements per step

template <bool BF16>
struct OpT;
template <>
struct OpT<false> {
  using T = _Float16;
  using V8 = f16x8;
  __device__ __forceinline__ static uint16_t bits(float v) {
    return __builtin_bit_cast(uint16_t, (_Float16)v);
  }
  __device__ __forceinline__ static f32x16 mfma(const V8 &a, const V8 &b, const f32x16 &c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct OpT<true> {
  using T = __bf16;
  using V8 = bf16x8;
  __device__ __forceinline__ static uint16_t bits(float v) {
    return __builtin_bit_cast(uint16_t, (__bf16)v);
  }
  __device__ __forceinline__ static f32x16 mfma(const V8 &a, const V8 &b, const f32x16 &c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

struct GemmArgs {
  // weights: role bases (gate, up) or (down, -), per-expert strides, row bytes
  const uint8_t *qs0, *qs1, *meta0, *meta1;
  size_t qs_stride, meta_stride;
  uint32_t row_qs, row_meta;
  int rows, cols, nseg;
  const uint8_t *sqs0, *sqs1, *smeta0, *smeta1;
  uint32_t srow_qs, srow_meta;
  int srows, scols, snseg;
  // activations (operand type), [rows][a_stride]; a_bytes = size of the buffer
  const uint16_t *a;
  int a_stride;
  uint32_t a_bytes;
  const int32_t *perm_token;  // gate/up: pair -> token row of `a`; down: null (a is per pair)
  const int32_t *offsets;
  const int32_t *tiles;  // [0] = count, then (expert, first pair) pairs; expert E = shared
  int E, T, k, has_shared;
  // outputs
  uint16_t *act;  // gate/up: [pairs][act_stride] operand type
  int act_stride;
  float *y;       // down: [pairs][H]
  int y_stride;
  // grid decomposition (see k_gemm): N-tiles and the tile order
  int n_tiles, xcd_split;
};

// One thread's share of a weight tile: row = tid / 2, half h = tid % 2 of the
// 64-element K step, dequantized to 32 floats in K order.
template <int FMT>
struct WLoad {
  uint4 q[2];  // codes (Q4_K / Q4_0: q[0] only; F32: 8 floats in q[0..1]x... see below)
  uint4 f[6];  // F32 only: 32 floats = 8 x uint4 with q[0..1]
  uint4 m;     // scales
};

template <int FMT>
__device__ __forceinline__ void w_fetch(WLoad<FMT> &w, __amdgpu_buffer_rsrc_t rq,
                                        __amdgpu_buffer_rsrc_t rm, uint32_t row_off_q,
                                        uint32_t row_off_m, int ks, int h, int nseg, bool valid) {
  if constexpr (FMT == NX_FMT_Q4_K) {
    // segment ks, half h: the 32 codes of sub-block s (h = 0) or s+4 (h = 1)
    const uint32_t o = valid ? row_off_q + seg_off(ks, h, nseg) : OOB;
    w.q[0] = bload16(rq, o);
    w.m = bload16(rm, valid ? row_off_m + (uint32_t)(ks >> 2) * 16u : OOB);
  } else if constexpr (FMT == NX_FMT_Q8_0) {
    // blocks 2ks + h (segment = block): 32 codes
    const int j = 2 * ks + h;
    const bool v = valid && j < nseg;
    w.q[0] = bload16(rq, v ? row_off_q + seg_off(j, 0, nseg) : OOB);
    w.q[1] = bload16(rq, v ? row_off_q + seg_off(j, 1, nseg) : OOB);
    // the scale's dword, and where in it the scale sits: the selection is
    // left to the decode, so that nothing waits for the load here
    const uint32_t mo = row_off_m + (uint32_t)j * 2u;
    w.m.x = bload4(rm, v ? (mo & ~3u) : OOB);
    w.m.y = (mo & 2u) * 8u;
  } else if constexpr (FMT == NX_FMT_Q4_0) {
    // segment ks holds blocks 2ks (half 0) and 2ks+1 (half 1)
    w.q[0] = bload16(rq, valid ? row_off_q + seg_off(ks, h, nseg) : OOB);
    // both blocks' scales; half h takes its own at decode time
    w.m.x = bload4(rm, valid ? row_off_m + (uint32_t)ks * 4u : OOB);
  } else {  // F32: segments 8ks + 4h .. +3 (8 floats each)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = 8 * ks + 4 * h + i;
      const bool v = valid && j < nseg;
      const uint4 a = bload16(rq, v ? row_off_q + seg_off(j, 0, nseg) : OOB);
      const uint4 b = bload16(rq, v ? row_off_q + seg_off(j, 1, nseg) : OOB);
      if (i == 0) {
        w.q[0] = a;
        w.q[1] = b;
      } else {
        w.f[2 * (i - 1)] = a;
        w.f[2 * (i - 1) + 1] = b;
      }
    }
  }
}

// dequantize this thread's 32 weights (half h of the 64-element step) to
// floats in K order: positions 32h .. 32h+31 of the step
template <int FMT>
__device__ __forceinline__ void w_decode(const WLoad<FMT> &w, int ks, int h, float *v) {
  if constexpr (FMT == NX_FMT_Q4_K) {
    // half 0: sub-block s = ks%4, half 1: sub-block s+4
    const float d = h2f(w.m.x & 0xFFFFu), dmin = h2f(w.m.x >> 16);
    const int s = ks & 3;
    const uint32_t b0 = (w.m.y >> (8 * s)) & 0xFFu;
    const uint32_t b4 = (w.m.z >> (8 * s)) & 0xFFu;
    const uint32_t b8 = (w.m.w >> (8 * s)) & 0xFFu;
    const float sc = h ? (float)((b8 & 15u) | ((b0 >> 6) << 4)) : (float)(b0 & 63u);
    const float mn = h ? (float)((b8 >> 4) | ((b4 >> 6) << 4)) : (float)(b4 & 63u);
    const uint32_t ws[4] = {w.q[0].x, w.q[0].y, w.q[0].z, w.q[0].w};
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // stored nibbles are q ^ 8
        const uint32_t byte = ((ws[k] >> (8 * i)) & 0xFFu) ^ 0x88u;
        // src/quant/mod.rs:841: d * sc * q - dmin * m (exact products)
        v[8 * k + i] = d * sc * (float)(byte & 15u) - dmin * mn;
        v[8 * k + 4 + i] = d * sc * (float)(byte >> 4) - dmin * mn;
      }
  } else if constexpr (FMT == NX_FMT_Q8_0) {
    const float d = h2f((w.m.x >> w.m.y) & 0xFFFFu);
    const uint32_t ws[8] = {w.q[0].x, w.q[0].y, w.q[0].z, w.q[0].w,
                            w.q[1].x, w.q[1].y, w.q[1].z, w.q[1].w};
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        v[4 * j + i] = (float)(int32_t)(int8_t)((ws[j] >> (8 * i)) & 0xFFu) * d;
  } else if constexpr (FMT == NX_FMT_Q4_0) {
    const float d = h2f((w.m.x >> (16 * h)) & 0xFFFFu);
    const uint32_t ws[4] = {w.q[0].x, w.q[0].y, w.q[0].z, w.q[0].w};
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t byte = ((ws[k] >> (8 * i)) & 0xFFu) ^ 0x88u;  // stored nibbles are q ^ 8
        v[8 * k + i] = (float)((int)(byte & 15u) - 8) * d;
        v[8 * k + 4 + i] = (float)((int)(byte >> 4) - 8) * d;
      }
  } else {
    const uint4 all[8] = {w.q[0], w.q[1], w.f[0], w.f[1], w.f[2], w.f[3], w.f[4], w.f[5]};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      v[4 * j] = __uint_as_float(all[j].x);
      v[4 * j + 1] = __uint_as_float(all[j].y);
      v[4 * j + 2] = __uint_as_float(all[j].z);
      v[4 * j + 3] = __uint_as_float(all[j].w);
    }
  }
}

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// The 32 weights of this lane's half step as MFMA B operands b[kk] (values
// 8kk .. 8kk+7 of the half).
template <int FMT, bool BF16>
__device__ __forceinline__ void w_operands(const WLoad<FMT> &w, int ks, int h,
                                           typename OpT<BF16>::V8 (&b)[4]) {
  if constexpr (FMT == NX_FMT_Q8_0 && !BF16) {
    // fp16 without a float detour: byte u = q ^ 0x80 becomes the f16 1024 + u
    // (exponent byte 0x64 above it), minus 1152 gives q exactly, and the f16
    // product with the f16 scale is q * d rounded once, as from the exact value
#pragma clang fp contract(off)
    const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)(w.m.x >> w.m.y));
    const h2 dd = {d, d}, off = {(_Float16)1152.0f, (_Float16)1152.0f};
    const uint32_t ws[8] = {w.q[0].x, w.q[0].y, w.q[0].z, w.q[0].w,
                            w.q[1].x, w.q[1].y, w.q[1].z, w.q[1].w};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      h2 r[4];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint32_t u = ws[2 * kk + j] ^ 0x80808080u;
        const h2 lo = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u));
        const h2 hi = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u));
        r[2 * j] = (lo - off) * dd;
        r[2 * j + 1] = (hi - off) * dd;
      }
      b[kk] = typename OpT<BF16>::V8{r[0][0], r[0][1], r[1][0], r[1][1],
                                     r[2][0], r[2][1], r[3][0], r[3][1]};
    }
  } else {
    float v[32];
    w_decode<FMT>(w, ks, h, v);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int i = 0; i < 8; ++i) b[kk][i] = (typename OpT<BF16>::T)v[8 * kk + i];
  }
}

// element index (within the activation row) of K position p of step ks
template <int FMT>
__device__ __forceinline__ int a_elem(int ks, int p) {
  if constexpr (FMT == NX_FMT_Q4_K)
    return (ks >> 2) * 256 + (ks & 3) * 32 + (p & 31) + ((p >> 5) << 7);
  return ks * 64 + p;
}

// LDS ring of activation stages: stage = the 128 x 64 activation tile of one
// K step as 128 rows of eight 16-byte chunks; chunk c of row r is stored at
// slot c ^ (r & 7), so the MFMA reads of eight consecutive rows hit eight
// different bank groups.  Distinct arrays per stage let the compiler track
// each stage's direct-to-LDS loads separately.
constexpr int RING = 4;
typedef __attribute__((address_space(3))) void lds_void;

template <int S>
__device__ __forceinline__ uint4 *ring_stage(uint4 *r0, uint4 *r1, uint4 *r2, uint4 *r3) {
  if constexpr (S == 0) return r0;
  else if constexpr (S == 1) return r1;
  else if constexpr (S == 2) return r2;
  else return r3;
}

// s_waitcnt vmcnt(n) (other counters unconstrained), n a compile-time constant
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00);
}

// F32 weights keep 64 floats of codes per stage per lane: one workgroup per CU
template <int FMT, bool BF16, bool GATEUP>
__global__ __launch_bounds__(256, FMT == NX_FMT_F32 ? 1 : 2) void k_gemm(const GemmArgs g) {
  using Op = OpT<BF16>;
  using V8 = typename Op::V8;
  constexpr int NMAT = GATEUP ? 2 : 1;
  // vector-memory instructions per K step: 4 activation chunks, and per
  // matrix the weight codes and scales
  constexpr int NWM = FMT == NX_FMT_F32 ? 8 : (FMT == NX_FMT_Q8_0 ? 3 : 2);
  constexpr int NA = 4, NW = NMAT * NWM;
  __shared__ __attribute__((aligned(16))) uint4 ring0[BM * 8];
  __shared__ __attribute__((aligned(16))) uint4 ring1[BM * 8];
  __shared__ __attribute__((aligned(16))) uint4 ring2[BM * 8];
  __shared__ __attribute__((aligned(16))) uint4 ring3[BM * 8];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Tile order.  xcd_split (gate/up): workgroup L runs on XCD L % 8; XCD x
  // owns N-tiles [x * npx, (x+1) * npx) and walks them with the M-tile list
  // fastest, so the M-tiles of one expert take each weight tile from the same
  // L2 back to back.  Otherwise (down, whose activation tiles span K = the
  // expert width and are the larger operand): N-tiles fastest, so the N-tiles
  // of one activation tile run together.
  const int L = blockIdx.x;
  const int mcount = g.tiles[0];
  if (mcount <= 0) return;
  int tile, ntile;
  if (g.xcd_split) {
    const int xcd = L & 7, j = L >> 3, npx = (g.n_tiles + 7) >> 3;
    tile = j % mcount;
    ntile = xcd * npx + j / mcount;
    if (ntile >= min(g.n_tiles, (xcd + 1) * npx)) return;  // workgroup-uniform
  } else {
    tile = L / g.n_tiles;
    ntile = L - tile * g.n_tiles;
    if (tile >= mcount) return;  // workgroup-uniform
  }
  const int e = g.tiles[2 + 2 * tile], m0 = g.tiles[3 + 2 * tile];
  const bool routed = e < g.E;
  const int pair0 = routed ? g.offsets[e] : g.T * g.k;
  const int count = routed ? g.offsets[e + 1] - pair0 : g.T;
  const int rows = routed ? g.rows : g.srows;
  const int cols = routed ? g.cols : g.scols;
  const int nseg = routed ? g.nseg : g.snseg;
  const uint32_t rq = routed ? g.row_qs : g.srow_qs;
  const uint32_t rm = routed ? g.row_meta : g.srow_meta;
  const int n0 = ntile * BN;
  if (n0 >= rows) return;
  const int mrows = min(BM, count - m0);

  const uint8_t *q0p = routed ? g.qs0 + (size_t)e * g.qs_stride : g.sqs0;
  const uint8_t *q1p = routed ? g.qs1 + (size_t)e * g.qs_stride : g.sqs1;
  const uint8_t *m0p = routed ? g.meta0 + (size_t)e * g.meta_stride : g.smeta0;
  const uint8_t *m1p = routed ? g.meta1 + (size_t)e * g.meta_stride : g.smeta1;
  const __amdgpu_buffer_rsrc_t rq0 = make_rsrc(q0p, (uint32_t)rows * rq);
  const __amdgpu_buffer_rsrc_t rq1 = make_rsrc(q1p, (uint32_t)rows * rq);
  const __amdgpu_buffer_rsrc_t rm0 = make_rsrc(m0p, (uint32_t)rows * rm);
  const __amdgpu_buffer_rsrc_t rm1 = make_rsrc(m1p, (uint32_t)rows * rm);

  // ---- activation chunks: instruction q of this wave fills stage chunks
  // (4 * wave + q) * 64 + lane, i.e. row r_q = (4 * wave + q) * 8 + lane / 8,
  // slot lane % 8, which holds K chunk (lane % 8) ^ (r_q & 7) of that row
  // (gathered through the permutation for gate/up).  One wave-uniform
  // resource spans the activation buffer; absent rows read zero.
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(g.a, g.a_bytes);
  uint32_t aoff[NA];
  int achunk[NA];
  int arow[NA];
#pragma unroll
  for (int q = 0; q < NA; ++q) {
    const int r = (4 * wave + q) * 8 + (lane >> 3);
    achunk[q] = (lane & 7) ^ (r & 7);
    // absent rows look up the tile's first pair (always present) and are
    // masked below, so the four lookups go out together
    const int p = pair0 + m0 + (r < mrows ? r : 0);
    arow[q] = GATEUP ? (routed ? g.perm_token[p] : p - pair0) : p;
  }
#pragma unroll
  for (int q = 0; q < NA; ++q) {
    const int r = (4 * wave + q) * 8 + (lane >> 3);
    aoff[q] = r < mrows ? (uint32_t)arow[q] * (uint32_t)g.a_stride * 2u : OOB;
  }

  // ---- weights: row n0 + 32 * wave + lane % 32, half lane / 32 of the step
  const int l32 = lane & 31, kh = lane >> 5;
  const int wrow = n0 + 32 * wave + l32;
  const bool wrow_ok = wrow < rows;
  const uint32_t wq_off = (uint32_t)wrow * rq, wm_off = (uint32_t)wrow * rm;

  // number of 64-element K steps
  const int nks = FMT == NX_FMT_Q4_K ? nseg : (FMT == NX_FMT_F32 ? (nseg + 7) / 8 : (FMT == NX_FMT_Q8_0 ? (nseg + 1) / 2 : nseg));

  auto issue_a = [&](auto stage, int ks) {
    constexpr int S = decltype(stage)::value;
    uint4 *dst = ring_stage<S>(ring0, ring1, ring2, ring3);
#pragma unroll
    for (int q = 0; q < NA; ++q) {
      const int el = a_elem<FMT>(ks, 8 * achunk[q]);
      const uint32_t off = (aoff[q] != OOB && el < cols) ? aoff[q] + (uint32_t)el * 2u : OOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void *)(dst + (4 * wave + q) * 64), 16, off,
                                               0, 0, 0);
    }
  };
  WLoad<FMT> wbuf[2][NMAT];
  auto issue_w = [&](WLoad<FMT>(&wb)[NMAT], int ks) {
    // steps past the end read zeros (their activations are zero too)
#pragma unroll
    for (int mt = 0; mt < NMAT; ++mt)
      w_fetch<FMT>(wb[mt], mt == 0 ? rq0 : rq1, mt == 0 ? rm0 : rm1, wq_off, wm_off, ks, kh, nseg,
                   wrow_ok && ks < nks);
  };

  // ---- accumulators: acc[mt][mi] = pairs 32mi .. 32mi+31 x this wave's 32 rows
  f32x16 acc[NMAT][4];
#pragma unroll
  for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mt][i][r] = 0.f;

  // Software pipeline over a whole number of ring rounds (steps past nks load
  // zeros and add nothing).  Step ks: wait until this wave's loads of
  // activation stage ks and weights ks have landed, barrier (every wave's
  // share of the stage is in LDS, and every wave is done reading stage ks-1's
  // slot), issue activation stage ks+3 into that slot and weights ks+2, decode
  // weights ks into B operands, run the step's MFMAs.  Every step issues the
  // same loads, unconditionally (a conditional load would make the compiler
  // copy its registers, waiting for all loads in flight): A(ks) at step ks-3,
  // W(ks) at step ks-2 after A(ks+1), so after W(ks) come exactly A(ks+2) and
  // W(ks+1), and vmcnt <= NA + NW completes both.
  auto wait_step = [&]() {
    wait_vm<NA + NW>();
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  };
  auto compute = [&](auto stage, const V8 (&bf)[NMAT][4]) {
    constexpr int S = decltype(stage)::value;
    const uint4 *src = ring_stage<S>(ring0, ring1, ring2, ring3);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int c = 4 * kh + kk;
      V8 af[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 32 * i + l32;
        af[i] = __builtin_bit_cast(V8, src[r * 8 + (c ^ (r & 7))]);
      }
#pragma unroll
      for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[mt][i] = Op::mfma(af[i], bf[mt][kk], acc[mt][i]);
    }
  };
  auto step = [&](auto stage, auto buf, int ks) {
    constexpr int S = decltype(stage)::value, B = decltype(buf)::value;
    wait_step();
    issue_a(std::integral_constant<int, (S + 3) % RING>{}, ks + 3);
    V8 bf[NMAT][4];
#pragma unroll
    for (int mt = 0; mt < NMAT; ++mt) w_operands<FMT, BF16>(wbuf[B][mt], ks, kh, bf[mt]);
    issue_w(wbuf[B], ks + 2);
    compute(stage, bf);
    // keep each step's work in its step (register pressure)
    __builtin_amdgcn_sched_barrier(0);
  };

  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  issue_a(I0{}, 0);
  issue_a(I1{}, 1);
  issue_w(wbuf[0], 0);
  issue_a(I2{}, 2);
  issue_w(wbuf[1], 1);
  for (int ks = 0; ks < nks; ks += RING) {
    step(I0{}, I0{}, ks);
    step(I1{}, I1{}, ks + 1);
    step(I2{}, I0{}, ks + 2);
    step(I3{}, I1{}, ks + 3);
  }
  // no direct-to-LDS write may land after the workgroup has ended
  wait_vm<0>();

  // ---- epilogue.  32x32 accumulator layout: lane holds column (lane % 32),
  // register r holds row (r / 4) * 8 + (lane / 32) * 4 + r % 4.
  const int col = n0 + 32 * wave + l32, rq4 = kh * 4;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = i * 32 + (r >> 2) * 8 + rq4 + (r & 3);
      if (row < mrows && col < rows) {
        const size_t p = (size_t)(pair0 + m0 + row);
        if constexpr (GATEUP) {
          const float v = silu_mul(acc[0][i][r], acc[1][i][r]);
          g.act[p * g.act_stride + col] = Op::bits(v);
        } else {
          g.y[p * g.y_stride + col] = acc[0][i][r];
        }
      }
    }
}

// f32 activations -> operand type (one row per token)
template <bool BF16>
__global__ __launch_bounds__(256) void k_to_half(const float *__restrict__ x, size_t n,
                                                 uint16_t *__restrict__ out) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    out[i] = OpT<BF16>::bits(x[i]);
}

using GemmFn = void (*)(GemmArgs);

template <bool BF16, bool GATEUP>
GemmFn pick_fmt(int fmt) {
  switch (fmt) {
  case NX_FMT_Q4_K: return k_gemm<NX_FMT_Q4_K, BF16, GATEUP>;
  case NX_FMT_Q8_0: return k_gemm<NX_FMT_Q8_0, BF16, GATEUP>;
  case NX_FMT_Q4_0: return k_gemm<NX_FMT_Q4_0, BF16, GATEUP>;
  case NX_FMT_F32: return k_gemm<NX_FMT_F32, BF16, GATEUP>;
  }
  return nullptr;
}

GemmFn pick(int fmt, bool bf16, bool gateup) {
  if (bf16) return gateup ? pick_fmt<true, true>(fmt) : pick_fmt<true, false>(fmt);
  return gateup ? pick_fmt<false, true>(fmt) : pick_fmt<false, false>(fmt);
}

void fill_weights(GemmArgs &a, const nx_experts *ex, bool gateup) {
  const RolePlane &R0 = ex->role[gateup ? NX_ROLE_GATE : NX_ROLE_DOWN];
  const RolePlane &R1 = ex->role[gateup ? NX_ROLE_UP : NX_ROLE_DOWN];
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
  if (ex->Fs > 0) {
    const RolePlane &S0 = ex->shared[gateup ? NX_ROLE_GATE : NX_ROLE_DOWN];
    const RolePlane &S1 = ex->shared[gateup ? NX_ROLE_UP : NX_ROLE_DOWN];
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
}

int run(nx_ctx *c, const GemmPlan &p, bool gateup) {
  const nx_experts *ex = p.ex;
  GemmArgs a{};
  fill_weights(a, ex, gateup);
  a.offsets = p.offsets;
  a.tiles = p.tiles;
  a.E = ex->E;
  a.T = p.T;
  a.k = p.k;
  a.has_shared = ex->Fs > 0 ? 1 : 0;
  if (gateup) {
    a.a = static_cast<const uint16_t *>(p.xh);
    a.a_stride = ex->H;
    a.a_bytes = (uint32_t)((size_t)p.T * ex->H * 2);
    a.perm_token = p.perm_token;
    a.act = static_cast<uint16_t *>(p.act);
    a.act_stride = p.act_stride;
  } else {
    a.a = static_cast<const uint16_t *>(p.act);
    a.a_stride = p.act_stride;
    a.a_bytes = (uint32_t)(p.pairs_total * p.act_stride * 2);
    a.perm_token = nullptr;
    a.y = p.ypair;
    a.y_stride = ex->H;
  }
  const int rows = a.rows > a.srows ? a.rows : a.srows;
  a.n_tiles = (rows + BN - 1) / BN;
  a.xcd_split = gateup ? 1 : 0;
  // enough workgroups for either order at the largest M-tile count
  const long wgs = a.xcd_split ? 8L * ((a.n_tiles + 7) / 8) * p.max_tiles
                               : (long)a.n_tiles * p.max_tiles;
  if (wgs > 0x7FFFFFFFL) return fail(NX_ERR_UNSUPPORTED, "grouped GEMM grid too large");
  GemmFn fn = pick(ex->fmt, p.bf16, gateup);
  if (!fn) return fail(NX_ERR_UNSUPPORTED, "no grouped-GEMM kernel for this format");
  const char *name = gateup ? "gemm_gateup" : "gemm_down";
  // (the 64 KB activation ring keeps at most two workgroups per CU, which
  // also bounds the L2 footprint of the down projection's long K)
  return launch(c, name,
                [&] { hipLaunchKernelGGL(fn, dim3((unsigned)wgs), dim3(256), 0, c->stream, a); });
}

}  // namespace

int gemm_tile_m() { return BM; }

int launch_to_half(nx_ctx *c, const float *x, size_t n, bool bf16, void *out) {
  if (n == 0) return NX_OK;
  size_t gblocks = (n + 255) / 256;
  if (gblocks > 65536) gblocks = 65536;
  uint16_t *o = static_cast<uint16_t *>(out);
  if (bf16)
    return launch(c, "to_bf16", [&] { k_to_half<true><<<(unsigned)gblocks, 256, 0, c->stream>>>(x, n, o); });
  return launch(c, "to_f16", [&] { k_to_half<false><<<(unsigned)gblocks, 256, 0, c->stream>>>(x, n, o); });
}

int launch_gemm_gateup(nx_ctx *c, const GemmPlan &p) { return run(c, p, true); }
int launch_gemm_down(nx_ctx *c, const GemmPlan &p) { return run(c, p, false); }

}  // namespace nx
