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
// pair) of BM pairs (64, 128 or 160, for gate/up and for down: one list each); the 1-D
// grid covers (M-tile, 128-row N-tile) pairs in an XCD-aware order (see
// k_gemm; extra workgroups exit).  A workgroup of 4 waves owns a BM x 64NT
// output tile (gate/up: two of them, for the gate and the up rows); wave w
// owns weight rows 16NT w .. 16NT w + 16NT - 1 of the tile for all BM pairs,
// as NT x BM/16 v_mfma_f32_16x16x32 tiles per matrix (NT = 2; see
// GemmShape).
//
// Operand order.  The K loop takes 64 positions per step.  Position
// j = 64 ks + 16 q + i is value i of the lanes of quarter q (lanes 16q ..
// 16q+15) at step ks: with the 16x16x32 MFMA, the four lanes of a weight row
// (one per quarter) cover 64 consecutive operand positions, and the order is
// chosen per format so that those four lanes read 32-64 contiguous bytes of
// one 128-byte line of the resident code plane, and so that a lane's scales
// for several steps sit in one load (kpos below).  The activations are
// written in the same order by their producers (k_to_half for x, the gate/up
// epilogue for act), so the activation tile of a step is still one
// contiguous 128-byte run per row.  A Q4_K row whose width is 256 past a
// multiple of 512 ends in a half window of one block, which the down pass
// takes in element order over 4 steps (half_win_of, the HWK instances).
//
// Pipeline.  The activation tile of a step goes into a 4-stage LDS ring by
// direct-to-LDS loads, shared by the four waves.  The weights never pass
// through LDS: each lane dequantizes its 16 values of each of its two rows
// (bit-exact f32, rounded once to the operand type) straight into its MFMA B
// operands.  Codes are fetched two steps ahead, scales once per window of
// steps, activations three steps ahead.
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "nx_device.hpp"
#ifndef WDIST_CFG
#define WDIST_CFG 2
#endif
#include "nx_internal.hpp"

namespace nx {

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// Pairs per M-tile: 128, or 160 when experts hold about 100-160 pairs each,
// so that most of them stream and decode their weights once instead of
// twice (DeepSeek T = 4096, ~128 pairs per expert: gate/up 2.82 -> 2.44 ms,
// down 1.76 -> 1.45 ms).  Elsewhere 128 is as fast or faster (Qwen3 T = 512,
// 32 per expert: down 80 -> 85 us with 160; the Mixtral prefill, ~500 per
// expert, gains 13 us in the down pass and loses 20 us to a second K
// split).  Gate/up on 160-pair tiles holds its two matrices' accumulators
// with one code buffer (codes one step ahead) and one M-tile per scheduling
// group; Q8_0's operands do not fit beside them, so Q8_0 gate/up stays at
// 128.  With 160 the LDS ring is 80 KB: two workgroups fill a CU.
// 64-pair tiles when experts hold at most 48 pairs each: a 32 KB ring and
// a third (gate/up, 158 VGPRs) or fourth (down, 111 VGPRs) workgroup per
// CU, so more waves hide the weight loads of the short tiles (Qwen3 T = 512:
// gate/up 101 -> 90 us, down 81 -> 70 us; Mixtral T = 128: down 125 ->
// 101 us; DeepSeek T = 256: 2.41 -> 2.17 ms).  At 64 pairs per expert
// (Mixtral T = 256, Qwen3 T = 1024) they are slower (gate/up 226 -> 294,
// 115 -> 136 us): the experts past 64 pairs stream their weights twice.
constexpr int BM_GATEUP = 128, BM_WIDE = 160, BM_NARROW = 64;
constexpr double NARROW_PER_MAX = 48.0;  // expected pairs per active expert
constexpr int OCC_NARROW = 3;            // workgroups per CU the 64-pair gate/up is built for
constexpr int BK = 64;    // K positions per step

template <bool BF16>
struct OpT;
template <>
struct OpT<false> {
  using T = _Float16;
  using V8 = f16x8;
  __device__ __forceinline__ static uint16_t bits(float v) {
    return __builtin_bit_cast(uint16_t, (_Float16)v);
  }
  __device__ __forceinline__ static f32x4 mfma(const V8 &a, const V8 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct OpT<true> {
  using T = __bf16;
  using V8 = bf16x8;
  __device__ __forceinline__ static uint16_t bits(float v) {
    return __builtin_bit_cast(uint16_t, (__bf16)v);
  }
  __device__ __forceinline__ static f32x4 mfma(const V8 &a, const V8 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

// ---- operand order --------------------------------------------------------
//
// Window = the K positions whose scales one lane loads at once.  Within a
// window of format FMT, operand position j (step s = (j / 64) % steps, lane
// quarter q = (j / 16) % 4, value i = j % 16) holds activation element
// kpos(j):
//   Q8_0 (window 256 = blocks 8u .. 8u+7, 4 steps): quarter q takes block
//        8u + 2q + s%2, code-plane half s/2, so e = 256u + 64q + 32(s%2) +
//        16(s/2) + i; its two scales are one dword, and steps 2k, 2k+1 read
//        the two halves of the same 128-byte lines.
//   Q4_K (window 512 = blocks 2u, 2u+1, 8 steps): quarter q takes block
//        2u + q/2, sub-block (s%4) + 4(s/4), bytes 8(q%2) .. +7 of its
//        16-byte half: e = 512u + 256(q/2) + 128(s/4) + 32(s%4) + 16(q%2) + i;
//        its scales are the block's 16 bytes.
//   Q4_0 (window 512 = segments 8u .. 8u+7, 8 steps): quarter q takes
//        segment 8u + 4(q/2) + s%4, block half s/4 (block 2*segment + s/4),
//        bytes 8(q%2) .. +7: e = 512u + 256(q/2) + 64(s%4) + 32(s/4) +
//        16(q%2) + i; its scales are 16 bytes (4 segments).
//   F32 (window 64): e = j.
template <int FMT>
__host__ __device__ constexpr int kwin() {
  return FMT == NX_FMT_Q8_0 ? 256 : (FMT == NX_FMT_F32 ? 64 : 512);
}

template <int FMT>
__host__ __device__ __forceinline__ int kpos(int j) {
  if constexpr (FMT == NX_FMT_Q8_0) {
    const int s = (j >> 6) & 3, q = (j >> 4) & 3;
    return (j & ~255) | (q << 6) | ((s & 1) << 5) | ((s >> 1) << 4) | (j & 15);
  } else if constexpr (FMT == NX_FMT_Q4_K || FMT == NX_FMT_Q4_0) {
    const int s = (j >> 6) & 7, q = (j >> 4) & 3;
    const int p = s >> 2, t = s & 3;
    const int mid = FMT == NX_FMT_Q4_K ? 128 * p + 32 * t : 64 * t + 32 * p;
    return (j & ~511) + 256 * (q >> 1) + mid + 16 * (q & 1) + (j & 15);
  } else {
    return j;
  }
}

// inverse of kpos: operand position of activation element e
template <int FMT>
__host__ __device__ __forceinline__ int kslot(int e) {
  if constexpr (FMT == NX_FMT_Q8_0) {
    const int q = (e >> 6) & 3, s = ((e >> 5) & 1) | (((e >> 4) & 1) << 1);
    return (e & ~255) | (s << 6) | (q << 4) | (e & 15);
  } else if constexpr (FMT == NX_FMT_Q4_K || FMT == NX_FMT_Q4_0) {
    const int a = (e >> 8) & 1, b = (e >> 4) & 1;
    const int p = FMT == NX_FMT_Q4_K ? (e >> 7) & 1 : (e >> 5) & 1;
    const int t = FMT == NX_FMT_Q4_K ? (e >> 5) & 3 : (e >> 6) & 3;
    return (e & ~511) + 64 * (4 * p + t) + 16 * (2 * a + b) + (e & 15);
  } else {
    return e;
  }
}

int kpad_of(int fmt, int cols) {
  const int w = fmt == NX_FMT_Q8_0 ? kwin<NX_FMT_Q8_0>()
                                   : (fmt == NX_FMT_F32 ? kwin<NX_FMT_F32>() : kwin<NX_FMT_Q4_K>());
  return (cols + w - 1) / w * w;
}

struct GemmArgs {
  // weights: role bases (gate, up) or (down, -), per-expert strides, row bytes
  const uint8_t *qs0, *qs1, *meta0, *meta1;
  size_t qs_stride, meta_stride;
  uint32_t row_qs, row_meta;
  int rows, cols, nseg;
  const uint8_t *sqs0, *sqs1, *smeta0, *smeta1;
  uint32_t srow_qs, srow_meta;
  int srows, scols, snseg;
  // activations (operand type, operand order), [rows][a_stride]; a_bytes =
  // size of the buffer
  const uint16_t *a;
  int a_stride;
  uint32_t a_bytes;
  const int32_t *perm_token;  // gate/up: pair -> token row of `a`; down: null (a is per pair)
  const int32_t *offsets;
  const int32_t *tiles;  // [0] = count, then (expert, first pair) pairs; expert E = shared
  int E, T, k, has_shared;
  // outputs
  uint16_t *act;  // gate/up: [pairs][act_stride] operand type, operand order
  int act_stride;
  float *y;       // down: [ksplit][pairs][H], one partial sum per K split
  uint16_t *yb;   // down, bf16 kernels, when set instead of y: the partial sums as bf16
  int y_stride;
  size_t y_split;  // elements between the K splits' partial sums
  // grid decomposition (see k_gemm): N-tiles, the tile order, and (down)
  // the K splits, each over wg_per_split workgroups
  int n_tiles, xcd_split, ksplit, wg_per_split;
  // Q4_K down pass: the window that holds only one block (the expert width
  // is 256 past a multiple of 512), routed and shared expert, or -1
  int half_win, shalf_win;
};

__device__ __forceinline__ uint2 bload8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
  return make_uint2(v[0], v[1]);
}

// ---- weights: one lane's codes of one step, and scales of one window ------
//
// A lane holds weight rows n0 + 16 NT w + 16 n + l%16, n = 0 .. NT-1.
template <int FMT, int NT>
struct WCodes {
  uint4 c[NT];
};
template <int NT>
struct WCodes<NX_FMT_Q4_K, NT> {
  uint2 c[NT];
};
template <int NT>
struct WCodes<NX_FMT_Q4_0, NT> {
  uint2 c[NT];
};
template <int NT>
struct WCodes<NX_FMT_F32, NT> {
  uint4 c[NT][4];
};
template <int FMT, int NT>
struct WMeta {
  uint4 m[NT];
};
template <int NT>
struct WMeta<NX_FMT_Q8_0, NT> {
  uint32_t m[NT];
};
template <int NT>
struct WMeta<NX_FMT_F32, NT> {};

// code loads per matrix row set per step, scale loads per row set per window
template <int FMT>
constexpr int n_code_loads() {
  return FMT == NX_FMT_F32 ? 4 : 1;
}
template <int FMT>
constexpr int n_meta_loads() {
  return FMT == NX_FMT_F32 ? 0 : 1;
}
// steps per window
template <int FMT>
constexpr int win_steps() {
  return kwin<FMT>() / BK;
}
// steps over a row of `cols` activations padded to whole windows
template <int FMT>
__device__ __forceinline__ int kpad_steps(int cols) {
  return (cols + kwin<FMT>() - 1) / kwin<FMT>() * win_steps<FMT>();
}

// Weight addressing.  The planes are in panels of 64 segments (nx_device.hpp):
// window win lies in panel g = win / 8, and every row has prq code bytes and
// prm scale bytes in each panel.  A lane's loads of row n are at lane base
// lq[n] (the row times prq plus the lane quarter's place in the line) + a
// wave-uniform part (panel base, plane half and line of the step's window) +
// a constant.  Every part goes into the range-checked offset: the plane ends
// at the last panel, where rows past the matrix read zero (rows past the
// matrix in an earlier panel read the next panel's finite weights; their
// outputs are never written); blocks past a row's end (last partial window
// only) read finite neighbours or the zero padding of a short last panel,
// which meet zero activations.
template <int FMT>
__device__ __forceinline__ uint32_t code_lane_off(uint32_t row_off, int q) {
  if constexpr (FMT == NX_FMT_Q4_K || FMT == NX_FMT_Q4_0)
    return row_off + 64u * (q >> 1) + 8u * (q & 1);
  return row_off + 32u * q;  // Q8_0: blocks 8u + 2q (+1); F32: segments 8u + 2q (+1)
}
template <int FMT>
__device__ __forceinline__ uint32_t meta_lane_off(uint32_t row_off, int q) {
  if constexpr (FMT == NX_FMT_Q8_0) return row_off + 4u * q;
  return row_off + 16u * (q >> 1);
}
// uniform part of window win, code-plane half p: panel (64 segments), half,
// 8-segment line
__device__ __forceinline__ uint32_t code_win_off(int win, int p, int rows, int nseg) {
  const int g = win >> 3;
  return (uint32_t)g * (uint32_t)rows * panel_row_bytes(nseg, 32) +
         (uint32_t)(p * panel_gsz(g, nseg) * 16 + (win & 7) * 128);
}

// Q4_K half window (a row's last window when its width is 256 past a
// multiple of 512: one block, 2u, of the two).  Its four steps take the
// block's sub-blocks in order: quarter q of step S holds sub-block
// 2S + q/2, half q%2, i.e. operand position j of the window is element
// 512u + j.  In the code plane that is plane half S/2, 16-byte group
// 2(S%2) + q/2 of the block's 64 bytes of the line: lane base row + 16(q/2)
// + 8(q%2) (the full window's base minus 48(q/2)), uniform part line + 32(S%2).
// All four quarters use block 2u's scales (lane base minus 16(q/2)).
__host__ __device__ constexpr int half_win_of(int fmt, int cols) {
  return fmt == NX_FMT_Q4_K && cols % 512 == 256 ? cols / 512 : -1;
}

// codes of step S of window win (half: the Q4_K half window, lane bases lqh)
template <int FMT, int S, int NT>
__device__ __forceinline__ void fetch_codes(WCodes<FMT, NT> &w, __amdgpu_buffer_rsrc_t rq,
                                            const uint32_t (&lq)[NT], int win, int rows, int nseg,
                                            bool half = false, const uint32_t *lqh = nullptr) {
  if constexpr (FMT == NX_FMT_Q4_K) {
    const uint32_t u = code_win_off(win, S >> 2, rows, nseg) + 16u * (S & 3);
    // steps 4..7 of a half window do not exist: out of range, read as zero
    const uint32_t uh = S < 4 ? code_win_off(win, S >> 1, rows, nseg) + 32u * (S & 1) : 0u;
#pragma unroll
    for (int n = 0; n < NT; ++n)
      w.c[n] = bload8(rq, half ? (S < 4 ? lqh[n] + uh : OOB) : lq[n] + u);
  } else if constexpr (FMT == NX_FMT_Q8_0) {
    const uint32_t u = code_win_off(win, S >> 1, rows, nseg);
#pragma unroll
    for (int n = 0; n < NT; ++n) w.c[n] = bload16(rq, lq[n] + u + 16u * (S & 1));
  } else if constexpr (FMT == NX_FMT_Q4_0) {
    const uint32_t u = code_win_off(win, S >> 2, rows, nseg);
#pragma unroll
    for (int n = 0; n < NT; ++n) w.c[n] = bload8(rq, lq[n] + u + 16u * (S & 3));
  } else {  // F32: segments 8 win + 2q (+1), both halves: floats 64 win + 16q ..
    const uint32_t u0 = code_win_off(win, 0, rows, nseg), u1 = code_win_off(win, 1, rows, nseg);
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
      for (int k = 0; k < 4; ++k) w.c[n][k] = bload16(rq, lq[n] + ((k & 1) ? u1 : u0) + 16u * (k >> 1));
  }
}

// scales of window win: Q8_0 blocks 8 win + 2q, +1 (one dword, panel rows
// padded to whole dwords); Q4_K block 2 win + q/2; Q4_0 segments 8 win +
// 4(q/2) .. +3.  A window's scales are 8 MU bytes of its panel row (MU scale
// bytes per segment), full panel rows 64 MU.
template <int FMT, int NT>
__device__ __forceinline__ void fetch_meta(WMeta<FMT, NT> &m, __amdgpu_buffer_rsrc_t rm,
                                           const uint32_t (&lm)[NT], int win, int rows, int nseg,
                                           bool half = false, const uint32_t *lmh = nullptr) {
  constexpr int MU = Seg<FMT>::MU;
  if constexpr (MU > 0) {
    const int g = win >> 3;
    const uint32_t u = (uint32_t)g * (uint32_t)rows * panel_row_bytes(nseg, MU) +
                       (uint32_t)(win & 7) * (8u * MU);
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      if constexpr (FMT == NX_FMT_Q8_0) m.m[n] = bload4(rm, lm[n] + u);
      else if constexpr (FMT == NX_FMT_Q4_K) m.m[n] = bload16(rm, (half ? lmh[n] : lm[n]) + u);
      else m.m[n] = bload16(rm, lm[n] + u);
    }
  }
}

// byte N of x as a float (v_cvt_f32_ubyteN).  The compiler forms only
// ubyte0 from a shift and mask; the others are written out, so that one
// masked word feeds four conversions without a shift each.
template <int N>
__device__ __forceinline__ float ubyte_f32(uint32_t x) {
  float r;
  if constexpr (N == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(x));
  else if constexpr (N == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(x));
  else if constexpr (N == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(x));
  else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(x));
  return r;
}

// bf16(a) in the low half, bf16(b) in the high half, each rounded to
// nearest even (v_cvt_pk_bf16_f32, the conversion the compiler emits for a
// float -> __bf16 cast)
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  uint32_t r;
  asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// values 8M .. 8M+7 of the 16 of row n at step S of the window, as a B
// operand (HALF: step S of a Q4_K half window, for the lane's quarter pair
// qh = q / 2)
template <int FMT, bool BF16, int S, int M, bool HALF = false, typename WC, typename WM>
__device__ __forceinline__ typename OpT<BF16>::V8 w_operand(const WC &w, const WM &mt, int n,
                                                            int qh = 0) {
  using Op = OpT<BF16>;
  if constexpr (FMT == NX_FMT_Q8_0 && !BF16) {
    // fp16 without a float detour: byte u = q ^ 0x80 becomes the f16 1024 + u
    // (exponent byte 0x64 above it), minus 1152 gives q exactly, and the f16
    // product with the f16 scale is q * d rounded once, as from the exact value
#pragma clang fp contract(off)
    const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)(mt.m[n] >> (16 * (S & 1))));
    const h2 dd = {d, d}, off = {(_Float16)1152.0f, (_Float16)1152.0f};
    const uint32_t ws[2] = {M ? w.c[n].z : w.c[n].x, M ? w.c[n].w : w.c[n].y};
    h2 r[4];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t u = ws[j] ^ 0x80808080u;
      const h2 lo = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u));
      const h2 hi = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u));
      r[2 * j] = (lo - off) * dd;
      r[2 * j + 1] = (hi - off) * dd;
    }
    return typename Op::V8{r[0][0], r[0][1], r[1][0], r[1][1], r[2][0], r[2][1], r[3][0], r[3][1]};
  } else {
    float v[8];
    if constexpr (FMT == NX_FMT_Q8_0) {
      const float d = h2f((mt.m[n] >> (16 * (S & 1))) & 0xFFFFu);
      const uint32_t ws[2] = {M ? w.c[n].z : w.c[n].x, M ? w.c[n].w : w.c[n].y};
#pragma unroll
      for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          v[4 * k + i] = (float)(int32_t)(int8_t)((ws[k] >> (8 * i)) & 0xFFu) * d;
    } else if constexpr (FMT == NX_FMT_Q4_K || FMT == NX_FMT_Q4_0) {
      // value = A q + B for the nibble q = 0..15 of the sub-block:
      // Q4_K (src/quant/mod.rs:841) d * sc * q - dmin * m, A = d sc and
      // B = -dmin m; Q4_0 (q - 8) d, A = d and B = -8 d (exact, so the fma
      // rounds (q - 8) d once)
      // sub-block t + 4p of the block: in a half window t = 2(S%2) + q/2,
      // p = S/2 (t per lane)
      const int t = HALF ? 2 * (S & 1) + qh : (S & 3);
      constexpr int p = HALF ? (S >> 1) : (S >> 2);
      float A, B;
      if constexpr (FMT == NX_FMT_Q4_K) {
        const uint4 Q = mt.m[n];
        const float d = h2f(Q.x & 0xFFFFu), dmin = h2f(Q.x >> 16);
        const uint32_t b0 = (Q.y >> (8 * t)) & 0xFFu;
        const uint32_t b4 = (Q.z >> (8 * t)) & 0xFFu;
        const uint32_t b8 = (Q.w >> (8 * t)) & 0xFFu;
        const float sc = p ? (float)((b8 & 15u) | ((b0 >> 6) << 4)) : (float)(b0 & 63u);
        const float mn = p ? (float)((b8 >> 4) | ((b4 >> 6) << 4)) : (float)(b4 & 63u);
        A = d * sc;
        B = -(dmin * mn);
      } else {
        // segment 8u + 4(q/2) + t: dword t of the scales, block half p
        const uint32_t mw = t == 0 ? mt.m[n].x : (t == 1 ? mt.m[n].y : (t == 2 ? mt.m[n].z : mt.m[n].w));
        A = h2f((mw >> (16 * p)) & 0xFFFFu);
        B = -8.0f * A;
      }
      // the eight nibbles at once: stored nibbles are q ^ 8; value i is the
      // low nibble of byte i, value 4 + i its high nibble (each conversion
      // reads one byte of a masked word)
      const uint32_t u = (M ? w.c[n].y : w.c[n].x) ^ 0x88888888u;
      const uint32_t lo = u & 0x0F0F0F0Fu, hi = (u >> 4) & 0x0F0F0F0Fu;
      v[0] = __builtin_fmaf(ubyte_f32<0>(lo), A, B);
      v[1] = __builtin_fmaf(ubyte_f32<1>(lo), A, B);
      v[2] = __builtin_fmaf(ubyte_f32<2>(lo), A, B);
      v[3] = __builtin_fmaf(ubyte_f32<3>(lo), A, B);
      v[4] = __builtin_fmaf(ubyte_f32<0>(hi), A, B);
      v[5] = __builtin_fmaf(ubyte_f32<1>(hi), A, B);
      v[6] = __builtin_fmaf(ubyte_f32<2>(hi), A, B);
      v[7] = __builtin_fmaf(ubyte_f32<3>(hi), A, B);
    } else {
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const uint4 c = w.c[n][2 * M + k];
        v[4 * k] = __uint_as_float(c.x);
        v[4 * k + 1] = __uint_as_float(c.y);
        v[4 * k + 2] = __uint_as_float(c.z);
        v[4 * k + 3] = __uint_as_float(c.w);
      }
    }
    if constexpr (BF16) {
      // pairs packed in operand order (the compiler otherwise pairs
      // neighbours across the pairs and realigns them)
      const uint4 u = {pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]), pack_bf16(v[4], v[5]),
                       pack_bf16(v[6], v[7])};
      return __builtin_bit_cast(typename Op::V8, u);
    } else {
      typename Op::V8 b;
#pragma unroll
      for (int i = 0; i < 8; ++i) b[i] = (typename Op::T)v[i];
      return b;
    }
  }
}

// LDS ring of activation stages: stage = the BM x 64 activation tile of one
// K step as BM rows of eight 16-byte chunks (chunk c = operand positions
// 8c .. 8c+7 of the step); chunk c of row r is stored at slot c ^ swz(r),
// swz(r) = (r ^ (r / 8 % 2)) % 8.  ds_read_b128 serves eight lanes per
// cycle from 32 four-byte banks (128 bytes); an MFMA operand read takes one
// chunk of 16 consecutive rows, lanes 8j .. 8j+7 rows 8j .. 8j+7, and swz
// sends those eight rows to eight different 16-byte slots, so the read is
// free of bank conflicts (SQ_LDS_BANK_CONFLICT reads 0; (r / 2) % 8, which
// pairs rows 2k and 2k+1 on one slot, read 4 conflict cycles per
// ds_read_b128).  Distinct arrays per stage let the
// compiler track each stage's direct-to-LDS loads separately.
constexpr int RING = 4;
typedef __attribute__((address_space(3))) void lds_void;

// the slot permutation of row r: chunk c is stored at slot c ^ swz(r)
__device__ __forceinline__ int swz(int r) { return (r ^ ((r >> 3) & 1)) & 7; }

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

template <int V>
using IC = std::integral_constant<int, V>;

// compile-time loop: f(IC<I>{}), ..., f(IC<N-1>{})
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (I < N) {
    f(IC<I>{});
    static_for<I + 1, N>(f);
  }
}

// Kernel shape per format and pass.  NT = 16-row weight sets per wave
// (the tile has 64 NT weight rows), GRP > 1: the code loads of steps
// GRP k .. GRP k + GRP - 1 issued back to back (they read parts of the same
// lines, so a line is fetched once while all of them are in flight), OCC =
// workgroups per CU.  Both passes keep 32 rows per wave
// (NT = 2) and two workgroups per CU (three on 64-pair tiles); F32 takes one
// workgroup per CU.
// Measured on the Qwen3 (E = 128, T = 512) and DeepSeek (E = 256,
// T = 4096) Q4_K layers and the Mixtral Q8_0 prefill: NT = 1 and NT = 4
// are slower in both passes, and fetching the codes 3 to 8 steps ahead
// instead of 2 gains nothing.
// weight rows per wave (16 NT) per format family and pass
#ifndef NX_GEMM_NT_Q4
#define NX_GEMM_NT_Q4 2
#endif
#ifndef NX_GEMM_NT_Q4_DOWN
#define NX_GEMM_NT_Q4_DOWN 2
#endif
#ifndef NX_GEMM_NT_Q8
#define NX_GEMM_NT_Q8 2
#endif
__host__ __device__ constexpr int gemm_nt(int fmt, bool gateup) {
  return (fmt == NX_FMT_Q4_K || fmt == NX_FMT_Q4_0) ? (gateup ? NX_GEMM_NT_Q4 : NX_GEMM_NT_Q4_DOWN)
                                                     : (fmt == NX_FMT_Q8_0 ? NX_GEMM_NT_Q8 : 2);
}
// steps the codes are fetched ahead, and whether the scales of the 4-bit
// formats are double-buffered (fetched with the codes of a window's first
// step) rather than reloaded after a window's last decode
#ifndef NX_GEMM_WDIST_Q4
#define NX_GEMM_WDIST_Q4 WDIST_CFG
#endif
#ifndef NX_GEMM_META2_Q4
#define NX_GEMM_META2_Q4 0
#endif
#ifndef NX_GEMM_GRP_Q4
#define NX_GEMM_GRP_Q4 1
#endif
template <int FMT, bool GATEUP, int BM>
struct GemmShape {
  static constexpr int NT = gemm_nt(FMT, GATEUP);
  static constexpr bool Q4 = FMT == NX_FMT_Q4_K || FMT == NX_FMT_Q4_0;
  static constexpr int GRP = Q4 ? NX_GEMM_GRP_Q4 : 1;
  // gate/up on 160-pair tiles fetches codes one step ahead: one code buffer,
  // so that its 160 accumulators fit beside the operands without spilling
  static constexpr int WDIST = Q4 ? (GATEUP && BM > BM_GATEUP ? 1 : NX_GEMM_WDIST_Q4) : WDIST_CFG;
  static constexpr bool META2 = FMT == NX_FMT_Q8_0 || (Q4 && NX_GEMM_META2_Q4);
  static constexpr int OCC =
      (NT == 4 || FMT == NX_FMT_F32) ? 1 : (BM <= BM_NARROW ? OCC_NARROW : 2);
};
int gemm_bn(int fmt, bool gateup) { return 64 * gemm_nt(fmt, gateup); }

// Load schedule of the K loop (body positions; it repeats every body).
// Step t issues, in this order: at its start the activation stage
// t + RING - 1; after its last decode, for single-buffered scales the
// scales of a window starting at t+1, then the codes of the steps it
// prefetches (t+2 and t+3 at even t when paired, else t+2), each window's
// first step preceded by that window's double-buffered scales.  The wait at
// step P lets through the loads issued after the last one P needs (its
// activation stage, its codes, its window's scales).
struct LoadSchedule {
  int ring, ws, na, ncw, nmw, wdist, grp;
  bool meta2;
  static constexpr int mod(int x, int m) { return ((x % m) + m) % m; }
  constexpr int outstanding(int P) const {
    const int wstart = P - mod(P, ws);
    int after = 0;
    // loads whose target step or window lies before step 0 are never issued
    for (int t = P - 40; t < P; ++t) {
      if (t + ring - 1 >= 0) after += na;
      if (t + ring - 1 == P) after = 0;
      if (!meta2 && nmw > 0 && mod(t + 1, ws) == 0 && t + 1 >= 0) {
        after += nmw;
        if (t + 1 == wstart) after = 0;
      }
      const int nj = grp > 1 ? (mod(t, grp) == 0 ? grp : 0) : 1;
      for (int k = 0; k < nj; ++k) {
        const int j = t + (grp > 1 ? grp : wdist) + k;
        if (j < 0) continue;
        if (meta2 && nmw > 0 && mod(j, ws) == 0) {
          after += nmw;
          if (j == wstart) after = 0;
        }
        after += ncw;
        if (j == P) after = 0;
      }
    }
    return after;
  }
};

// HWK: the Q4_K down pass of experts with a half window (its own
// instances, so that the others keep their registers)
template <int FMT, bool BF16, bool GATEUP, int BMT, bool HWK = false>
__global__ __launch_bounds__(256, (GemmShape<FMT, GATEUP, BMT>::OCC)) void k_gemm(const GemmArgs g) {
  using Op = OpT<BF16>;
  using V8 = typename Op::V8;
  using Shape = GemmShape<FMT, GATEUP, BMT>;
  constexpr int NT = Shape::NT;
  constexpr int GRP = Shape::GRP;
  static_assert(GRP == 1 || GRP == 2 || GRP == 4, "code load groups");
  constexpr int BN = 64 * NT;
  constexpr int NMAT = GATEUP ? 2 : 1;
  constexpr int WS = win_steps<FMT>();
  // Scales: Q8_0 (one dword per row) double-buffers them, loaded just before
  // the codes of a window's first step; the 16-byte scales of the 4-bit
  // formats have one buffer, reloaded right after the last decode of a
  // window.
  constexpr bool META2 = Shape::META2;
  constexpr int NMB = META2 ? 2 : 1;
  constexpr int WDIST = Shape::WDIST;
  // code buffers (steps mod NBUF)
  constexpr int NBUF = GRP > 1 ? 2 * GRP : (WDIST <= 1 ? 1 : (WDIST <= 2 ? 2 : (WDIST <= 4 ? 4 : 8)));
  static_assert(GRP > 1 || WDIST <= NBUF, "code buffers");  // issued after the decode
  // a window's double-buffered scales are fetched after the last decode of
  // the window two back
  static_assert(!META2 || (GRP > 1 ? 2 * GRP <= win_steps<FMT>() + 2
                                     : WDIST <= win_steps<FMT>() + 1), "scale buffers");
  // steps per loop body: whole rounds of the ring, of the code buffers and
  // of the scale buffers
  constexpr int NB0 = RING > NBUF ? RING : NBUF, NB1 = META2 ? 2 * WS : WS;
  constexpr int NB = NB0 > NB1 ? NB0 : NB1;
  static_assert(NB % RING == 0 && NB % NBUF == 0 && NB % (NMB * WS) == 0, "loop body");
  constexpr int BM = BMT;  // pairs per tile
  static_assert(BM % 32 == 0, "whole activation loads per wave");
  constexpr int MB = BM / 16;  // 16-pair MFMA row sets per tile
  constexpr int NA = BM / 32;  // activation loads per wave and step (8 rows each)
  // M-tiles per scheduling group (gate/up on 160-pair tiles: one, for the
  // registers)
  constexpr int IG = GATEUP ? (BM > BM_GATEUP ? 1 : 2) : (MB % 4 ? 2 : 4);
  static_assert(MB % IG == 0, "whole scheduling groups");
  constexpr LoadSchedule sched{RING, WS, NA, NMAT * NT * n_code_loads<FMT>(),
                               NMAT * NT * n_meta_loads<FMT>(), WDIST, GRP, META2};
  __shared__ __attribute__((aligned(16))) uint4 ring0[BM * 8];
  __shared__ __attribute__((aligned(16))) uint4 ring1[BM * 8];
  __shared__ __attribute__((aligned(16))) uint4 ring2[BM * 8];
  __shared__ __attribute__((aligned(16))) uint4 ring3[BM * 8];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Tile order.  xcd_split 1 (gate/up): workgroup L runs on XCD L % 8; XCD x
  // owns N-tiles [x * npx, (x+1) * npx) and takes the experts in tile-list
  // order, each as a block of (its m_e M-tiles) x (the XCD's N-tiles), in
  // groups of g_e = XCD_WGS / m_e N-tiles with the M-tiles fastest: about
  // XCD_WGS workgroups, as many as an XCD runs at once, share g_e weight
  // tiles and m_e activation tiles through the XCD's L2.  xcd_split 2
  // (few pairs per expert, gate/up or down): XCD x runs one contiguous chunk
  // of the M-tile-major list (N-tiles fastest), so an M-tile's N-tiles share
  // its activation tile through one L2.  xcd_split 0 (down, many pairs per
  // expert, whose activation tiles span K = the expert width and are the
  // larger operand): N-tiles fastest, so the N-tiles of one activation tile
  // run together.
  constexpr int XCD_WGS = 32 * Shape::OCC;  // 32 CUs x OCC workgroups
  int L = blockIdx.x;
  // down: K split `split` of ksplit (whole loop bodies each)
  const int split = g.ksplit > 1 ? L / g.wg_per_split : 0;
  L -= split * g.wg_per_split;
  const int mcount = g.tiles[0];
  if (mcount <= 0) return;
  int tile, ntile;
  if (g.xcd_split == 1) {
    const int xcd = L & 7, j = L >> 3, npx = (g.n_tiles + 7) >> 3;
    // the expert's block: tiles of one expert are consecutive, first rows
    // 0, BM, 2 BM, ...
    const int tg = j / npx;
    if (tg >= mcount) return;  // workgroup-uniform
    const int eg = g.tiles[2 + 2 * tg];
    const int te = tg - g.tiles[3 + 2 * tg] / BM;
    const int cnt = eg < g.E ? g.offsets[eg + 1] - g.offsets[eg] : g.T;
    const int me = (cnt + BM - 1) / BM;
    const int ge = max(1, XCD_WGS / me);
    const int r = j - te * npx;
    const int grp = r / (ge * me), r2 = r - grp * ge * me;
    tile = te + r2 % me;
    ntile = xcd * npx + grp * ge + r2 / me;
    if (ntile >= g.n_tiles) return;  // workgroup-uniform
  } else if (g.xcd_split == 2) {
    // XCD x runs items [x per, (x+1) per) of the list: the N-tiles of an
    // M-tile, and the M-tiles of an expert, run together on one XCD
    const int xcd = L & 7, j = L >> 3;
    const long items = (long)mcount * g.n_tiles;
    const long per = (items + 7) >> 3;
    if (j >= per) return;  // workgroup-uniform
    const long it = xcd * per + j;
    if (it >= items) return;
    tile = (int)(it / g.n_tiles);
    ntile = (int)(it - (long)tile * g.n_tiles);
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

  // ---- activation chunks: instruction i of this wave fills stage chunks
  // (NA * wave + i) * 64 + lane, i.e. row r_i = (NA * wave + i) * 8 + lane / 8,
  // slot lane % 8, which holds chunk (lane % 8) ^ swz(r_i) of that row
  // (gathered through the permutation for gate/up).  One wave-uniform
  // resource spans the activation buffer; absent rows, and every step past
  // the padded width, read zero (rows are zero between the width and the
  // padded width).
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(g.a, g.a_bytes);
  uint32_t abase[NA];
  int arow[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int r = (NA * wave + i) * 8 + (lane >> 3);
    // absent rows look up the tile's first pair (always present) and are
    // masked below, so the four lookups go out together
    const int p = pair0 + m0 + (r < mrows ? r : 0);
    arow[i] = GATEUP ? (routed ? g.perm_token[p] : p - pair0) : p;
  }
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int r = (NA * wave + i) * 8 + (lane >> 3);
    const int chunk = (lane & 7) ^ swz(r);
    abase[i] = r < mrows ? (uint32_t)arow[i] * (uint32_t)g.a_stride * 2u + 16u * chunk : OOB;
  }
  // steps holding data (the padded width), and this workgroup's steps:
  // its split's share of the whole loop bodies (the steps past the padded
  // width load zeros and add nothing)
  const int nk_data = kpad_steps<FMT>(cols);
  const int nbody = (nk_data + NB - 1) / NB;
  const int ks_begin = split * nbody / g.ksplit * NB;
  const int ks_end = (split + 1) * nbody / g.ksplit * NB;

  // ---- weights: rows n0 + 16 NT wave + 16 n + lane % 16, quarter lane / 16
  // (lane bases at the rows' offsets in a panel)
  const int l16 = lane & 15, q = lane >> 4;
  const uint32_t rbq = panel_row_bytes(nseg, 32), rbm = panel_row_bytes(nseg, Seg<FMT>::MU);
  uint32_t lq[NT], lm[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const uint32_t wrow = (uint32_t)(n0 + 16 * NT * wave + 16 * n + l16);
    lq[n] = code_lane_off<FMT>(wrow * rbq, q);
    lm[n] = meta_lane_off<FMT>(wrow * rbm, q);
  }
  // Q4_K down: the row's last window may be a half window (see
  // half_win_of), run as 4 steps of its one block instead of 8 half-empty
  // steps; its lane bases
  constexpr bool HW = HWK && FMT == NX_FMT_Q4_K && !GATEUP;
  static_assert(!HW || NB == WS, "a half window is one loop body");
  const int half_win = HW ? (routed ? g.half_win : g.shalf_win) : -1;
  uint32_t lqh[NT], lmh[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    lqh[n] = lq[n] - 48u * (uint32_t)(q >> 1);
    lmh[n] = lm[n] - 16u * (uint32_t)(q >> 1);
  }

  // activation loads I0 .. I1-1 of stage ks
  auto issue_a_part = [&](auto stage, int ks, auto i0, auto i1) {
    constexpr int S = decltype(stage)::value;
    uint4 *dst = ring_stage<S>(ring0, ring1, ring2, ring3);
    // wave-uniform step offset; past the padded width it pushes every lane
    // out of range (bases stay below 2^31, so the sum does not wrap)
    const uint32_t koff = ks < nk_data ? (uint32_t)ks * (2u * BK) : OOB;
#pragma unroll
    for (int i = decltype(i0)::value; i < decltype(i1)::value; ++i) {
      const uint32_t off = abase[i] + koff;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void *)(dst + (NA * wave + i) * 64), 16, off,
                                               0, 0, 0);
    }
  };
  auto issue_a = [&](auto stage, int ks) { issue_a_part(stage, ks, IC<0>{}, IC<NA>{}); };
  WCodes<FMT, NT> wbuf[NBUF][NMAT];
  WMeta<FMT, NT> mbuf[NMB][NMAT];
  // codes (and double-buffered scales) of step J of a loop body (J may reach
  // into the next body) whose first window is wbase
  auto issue_w = [&](auto pos, int wbase) {
    constexpr int J = decltype(pos)::value;
    constexpr int S = J % WS;
    const int win = wbase + J / WS;
    const bool hwin = HW && win == half_win;
    if constexpr (META2 && S == 0) {
#pragma unroll
      for (int mt = 0; mt < NMAT; ++mt)
        fetch_meta<FMT, NT>(mbuf[(J / WS) % NMB][mt], mt == 0 ? rm0 : rm1, lm, win, rows, nseg,
                            hwin, lmh);
    }
#pragma unroll
    for (int mt = 0; mt < NMAT; ++mt)
      fetch_codes<FMT, S, NT>(wbuf[J % NBUF][mt], mt == 0 ? rq0 : rq1, lq, win, rows, nseg, hwin,
                              lqh);
  };
  // single-buffered scales of the window that starts at step J
  auto issue_meta1 = [&](auto pos, int wbase) {
    constexpr int J = decltype(pos)::value;
    if constexpr (!META2 && n_meta_loads<FMT>() > 0) {
      const int win = wbase + J / WS;
#pragma unroll
      for (int mt = 0; mt < NMAT; ++mt)
        fetch_meta<FMT, NT>(mbuf[0][mt], mt == 0 ? rm0 : rm1, lm, win, rows, nseg,
                            HW && win == half_win, lmh);
    }
  };
  // the late issues of step T (see LoadSchedule)
  auto issue_late = [&](auto pos, int wbase) {
    constexpr int T = decltype(pos)::value;
    if constexpr ((T + 1) % WS == 0) issue_meta1(IC<T + 1>{}, wbase);
    if constexpr (GRP > 1) {
      if constexpr (T % GRP == 0)
        static_for<0, GRP>([&](auto k) { issue_w(IC<T + GRP + decltype(k)::value>{}, wbase); });
    } else {
      issue_w(IC<T + WDIST>{}, wbase);
    }
  };

  // ---- accumulators: acc[mt][n][i] = pairs 16i .. 16i+15 x rows 16n .. of this wave
  f32x4 acc[NMAT][NT][MB];
#pragma unroll
  for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
      for (int i = 0; i < MB; ++i) acc[mt][n][i] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Software pipeline.  Step ks: wait until this wave's loads of activation
  // stage ks, codes ks and its window's scales have landed (the loads issued
  // after them may stay in flight), barrier (every wave's share of the stage
  // is in LDS, and every wave is done reading stage ks-1's slot), issue
  // activation stage ks+3 into that slot, decode the codes into B operands
  // and run the step's MFMAs, half by half, with the step's late loads
  // after the last decode.  Every step issues its loads unconditionally (a
  // conditional load would make the compiler copy its registers, waiting for
  // all loads in flight).
  const int sw = swz(l16);
  // 16-row sets of the tile holding pairs (workgroup-uniform)
  const int msub = __builtin_amdgcn_readfirstlane((mrows + 15) >> 4);
  // HB: the body of a Q4_K half window, of which only steps 0..3 run (the
  // loads they issue for later steps are past the row and are drained by
  // the last wait)
  auto step = [&](auto pos, int ks0, int wbase, auto hb) {
    constexpr int P = decltype(pos)::value;
    constexpr int S = P % WS;
    constexpr bool HB = decltype(hb)::value;
    static_assert(!HB || (HW && S < 4), "half-window steps");
    wait_vm<sched.outstanding(P)>();
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    const uint4 *src = ring_stage<P % RING>(ring0, ring1, ring2, ring3);
    // two halves of 32 K positions: B operands of the half, then its MFMAs
    // in groups of IG M-tiles (scheduling fences between the groups bound
    // the live operands).  The step's loads go between MFMA groups, so that
    // a wave held up issuing a load (memory pipeline full) still has MFMAs
    // queued: the activation loads after the first-half groups, the late
    // loads after the first second-half group.
    constexpr int NG = MB / IG;         // groups per half
    constexpr int APG = (NA + NG - 1) / NG;  // activation loads per group
    // A operands are read one group ahead (across the halves too), so each
    // group's MFMAs cover the LDS latency of the next group's reads
    auto read_a = [&](auto grp, V8 (&af)[IG]) {
      constexpr int G2 = decltype(grp)::value, M = G2 / NG, G = G2 % NG;
#pragma unroll
      for (int k = 0; k < IG; ++k) {
        const int i = IG * G + k;
        af[k] = __builtin_bit_cast(V8, src[(16 * i + l16) * 8 + ((2 * q + M) ^ sw)]);
      }
    };
    V8 bf[NMAT][NT];
    V8 an[IG];
    read_a(IC<0>{}, an);
    static_for<0, 2 * NG>([&](auto grp) {
      constexpr int G2 = decltype(grp)::value, M = G2 / NG, G = G2 % NG;
      if constexpr (G == 0) {
        // B operands of the half
#pragma unroll
        for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
          for (int n = 0; n < NT; ++n) {
            bf[mt][n] = w_operand<FMT, BF16, S, M, HB>(wbuf[P % NBUF][mt], mbuf[(P / WS) % NMB][mt],
                                                       n, q >> 1);
            // float decodes: one operand's temporaries at a time
            if constexpr (!(FMT == NX_FMT_Q8_0 && !BF16)) __builtin_amdgcn_sched_barrier(0);
          }
      }
      V8 af[IG];
#pragma unroll
      for (int k = 0; k < IG; ++k) af[k] = an[k];
      if constexpr (G2 + 1 < 2 * NG) read_a(IC<G2 + 1>{}, an);
      if (IG * G < msub) {  // groups of 16-row sets past the tile's last pair are skipped
#pragma unroll
        for (int k = 0; k < IG; ++k) {
          const int i = IG * G + k;
#pragma unroll
          for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
            for (int n = 0; n < NT; ++n) acc[mt][n][i] = Op::mfma(af[k], bf[mt][n], acc[mt][n][i]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      constexpr int a0 = G * APG < NA ? G * APG : NA;
      constexpr int a1 = (G + 1) * APG < NA ? (G + 1) * APG : NA;
      if constexpr (M == 0 && a0 < a1)
        issue_a_part(IC<(P + RING - 1) % RING>{}, ks0 + P + RING - 1, IC<a0>{}, IC<a1>{});
      if constexpr (M == 1 && G == 0) issue_late(IC<P>{}, wbase);
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // prologue: the loads the schedule issues at steps -PRO .. -1 (those
  // whose target step or window is >= 0), in schedule order: at step t the
  // activation stage t + RING - 1, then the late loads
  // (ks_begin is a whole number of bodies: ring stages and code buffers
  // keep their step-relative indices, wb0 is its window)
  const int wb0 = ks_begin / WS;
  constexpr int WD = GRP > 1 ? GRP : WDIST;  // first code step issued at step -WD
  constexpr int PRO = WD > RING - 1 ? WD : RING - 1;
  static_for<0, PRO>([&](auto i) {
    constexpr int t = (int)decltype(i)::value - PRO;
    if constexpr (t + RING - 1 >= 0) issue_a(IC<t + RING - 1>{}, ks_begin + t + RING - 1);
    if constexpr (t == -1) issue_meta1(IC<0>{}, wb0);
    if constexpr (GRP > 1) {
      if constexpr (((t % GRP) + GRP) % GRP == 0 && t + GRP >= 0)
        static_for<0, GRP>([&](auto k) { issue_w(IC<t + GRP + decltype(k)::value>{}, wb0); });
    } else if constexpr (t + WDIST >= 0) {
      issue_w(IC<t + WDIST>{}, wb0);
    }
  });
  // a split whose last body is the row's half window runs it on its own
  const bool tail_half = HW && half_win >= 0 && ks_end / WS - 1 == half_win;
  const int ks_full = tail_half ? ks_end - NB : ks_end;
  int ks0 = ks_begin, wbase = wb0;
  for (; ks0 < ks_full; ks0 += NB, wbase += NB / WS)
    static_for<0, NB>([&](auto pos) { step(pos, ks0, wbase, IC<false>{}); });
  if constexpr (HW) {
    if (tail_half) static_for<0, 4>([&](auto pos) { step(pos, ks0, wbase, IC<true>{}); });
  }
  // no direct-to-LDS write may land after the workgroup has ended
  wait_vm<0>();

  // ---- epilogue.  16x16 accumulator layout: lane holds column (lane % 16),
  // register j holds row 4 * (lane / 16) + j.
  // gate/up: act slot of down-pass K position e (operand order; element
  // order over a Q4_K half window, the down pass's last window when the
  // width is 256 past a multiple of 512)
  const int act_hs = half_win_of(FMT, rows) >= 0 ? rows - 256 : 0x7fffffff;
  auto act_slot = [&](int e) { return e >= act_hs ? e : kslot<FMT>(e); };
  if constexpr (!GATEUP && BF16) {
    if (g.yb) {
      // bf16 partial sums, two columns per 32-bit store: lanes 2c and 2c+1
      // swap one value of each register pair (j, j+1), so the even lane
      // holds columns (2c, 2c+1) of row j and the odd lane those of row j+1.
      // Rows are even (H % 2 == 0, checked by the host), so a lane pair is
      // in or out of range together.
      const bool odd = l16 & 1;
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        const int col = n0 + 16 * NT * wave + 16 * n + (l16 & ~1);
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
          for (int j = 0; j < 4; j += 2) {
            const float a0 = acc[0][n][i][j], a1 = acc[0][n][i][j + 1];
            const float other = __int_as_float(
                __builtin_amdgcn_mov_dpp(__float_as_int(odd ? a0 : a1), 0xB1, 0xF, 0xF, false));
            const float lo = odd ? other : a0, hi = odd ? a1 : other;
            const int row = 16 * i + 4 * q + j + (odd ? 1 : 0);
            if (col < rows && row < mrows) {
              const size_t p = (size_t)(pair0 + m0 + row);
              *reinterpret_cast<uint32_t *>(g.yb + split * g.y_split + p * g.y_stride + col) =
                  (uint32_t)OpT<true>::bits(lo) | ((uint32_t)OpT<true>::bits(hi) << 16);
            }
          }
      }
      return;
    }
  }
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int col = n0 + 16 * NT * wave + 16 * n + l16;
    if (col >= rows) continue;
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = 16 * i + 4 * q + j;
        if (row < mrows) {
          const size_t p = (size_t)(pair0 + m0 + row);
          if constexpr (GATEUP) {
            const float v = silu_mul(acc[0][n][i][j], acc[1][n][i][j]);
            g.act[p * g.act_stride + act_slot(col)] = Op::bits(v);
          } else {
            g.y[split * g.y_split + p * g.y_stride + col] = acc[0][n][i][j];
          }
        }
      }
  }
  // gate/up: the workgroup holding the matrix's last rows also writes the
  // zeros between the expert's width and act's padded width for its pairs
  // (the down pass reads whole windows; kslot permutes within a window, so
  // these slots are not any column's)
  if constexpr (GATEUP) {
    const int span = g.act_stride - rows;
    if (span > 0 && n0 + BN >= rows) {
      for (int i = tid; i < mrows * span; i += 256) {
        const int r = i / span, e = rows + (i - r * span);
        g.act[(size_t)(pair0 + m0 + r) * g.act_stride + act_slot(e)] = 0;
      }
    }
  }
}

// f32 activations [T][H] -> operand type in operand order [T][kpad]
// (positions past H are zero).  kslot keeps runs of 16 consecutive elements
// together, so slots 16g .. 16g+15 of a row are elements kpos(16g) .. +15:
// a thread converts one such run of token blockIdx.y (four 16-byte loads
// when the row allows them, two 16-byte stores).
template <int FMT, bool BF16>
__global__ __launch_bounds__(256) void k_to_half16(const float *__restrict__ x, int H, int kpad,
                                                   bool vec, uint16_t *__restrict__ out) {
  const int t = blockIdx.y;
  const int ng = kpad >> 4;
  const float *xr = x + (size_t)t * H;
  uint4 *orow = reinterpret_cast<uint4 *>(out + (size_t)t * kpad);
  for (int g = blockIdx.x * 256 + threadIdx.x; g < ng; g += gridDim.x * 256) {
    const int e0 = kpos<FMT>(g << 4);
    float v[16];
    if (vec && e0 + 16 <= H) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 f = *reinterpret_cast<const float4 *>(xr + e0 + 4 * q);
        v[4 * q] = f.x;
        v[4 * q + 1] = f.y;
        v[4 * q + 2] = f.z;
        v[4 * q + 3] = f.w;
      }
    } else {
#pragma unroll
      for (int q = 0; q < 16; ++q) v[q] = e0 + q < H ? xr[e0 + q] : 0.f;
    }
    uint32_t w[8];
#pragma unroll
    for (int q = 0; q < 8; ++q)
      w[q] = (uint32_t)OpT<BF16>::bits(v[2 * q]) | ((uint32_t)OpT<BF16>::bits(v[2 * q + 1]) << 16);
    orow[2 * g] = make_uint4(w[0], w[1], w[2], w[3]);
    orow[2 * g + 1] = make_uint4(w[4], w[5], w[6], w[7]);
  }
}

template <int FMT, bool BF16>
__global__ __launch_bounds__(256) void k_to_half(const float *__restrict__ x, int T, int H, int kpad,
                                                 uint16_t *__restrict__ out) {
  const size_t n = (size_t)T * kpad;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t t = i / (size_t)kpad;
    const int e = kpos<FMT>((int)(i - t * kpad));
    out[i] = e < H ? OpT<BF16>::bits(x[t * H + e]) : (uint16_t)0;
  }
}

using GemmFn = void (*)(GemmArgs);

template <bool BF16, bool GATEUP, int BMT>
GemmFn pick_fmt(int fmt, bool half) {
  switch (fmt) {
  case NX_FMT_Q4_K:
    if constexpr (!GATEUP) {
      if (half) return k_gemm<NX_FMT_Q4_K, BF16, GATEUP, BMT, true>;
    }
    return k_gemm<NX_FMT_Q4_K, BF16, GATEUP, BMT>;
  case NX_FMT_Q4_0: return k_gemm<NX_FMT_Q4_0, BF16, GATEUP, BMT>;
  }
  if constexpr (!GATEUP || BMT <= BM_GATEUP) {
    if (fmt == NX_FMT_Q8_0) return k_gemm<NX_FMT_Q8_0, BF16, GATEUP, BMT>;
  }
  if constexpr (BMT == BM_GATEUP || (!GATEUP && BMT == BM_WIDE)) {
    if (fmt == NX_FMT_F32) return k_gemm<NX_FMT_F32, BF16, GATEUP, BMT>;
  }
  return nullptr;
}

GemmFn pick(int fmt, bool bf16, bool gateup, int bm, bool half = false) {
  if (bm == BM_NARROW) {
    if (gateup)
      return bf16 ? pick_fmt<true, true, BM_NARROW>(fmt, half)
                  : pick_fmt<false, true, BM_NARROW>(fmt, half);
    return bf16 ? pick_fmt<true, false, BM_NARROW>(fmt, half)
                : pick_fmt<false, false, BM_NARROW>(fmt, half);
  }
  if (bm == BM_WIDE) {
    if (gateup)
      return bf16 ? pick_fmt<true, true, BM_WIDE>(fmt, half) : pick_fmt<false, true, BM_WIDE>(fmt, half);
    return bf16 ? pick_fmt<true, false, BM_WIDE>(fmt, half) : pick_fmt<false, false, BM_WIDE>(fmt, half);
  }
  if (gateup)
    return bf16 ? pick_fmt<true, true, BM_GATEUP>(fmt, half)
                : pick_fmt<false, true, BM_GATEUP>(fmt, half);
  return bf16 ? pick_fmt<true, false, BM_GATEUP>(fmt, half)
              : pick_fmt<false, false, BM_GATEUP>(fmt, half);
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
  a.half_win = gateup ? -1 : half_win_of(ex->fmt, a.cols);
  a.shalf_win = gateup || ex->Fs <= 0 ? -1 : half_win_of(ex->fmt, a.scols);
  a.offsets = p.offsets;
  a.tiles = gateup ? p.tiles : p.tiles_down;
  const int max_tiles = gateup ? p.max_tiles : p.max_tiles_down;
  a.E = ex->E;
  a.T = p.T;
  a.k = p.k;
  a.has_shared = ex->Fs > 0 ? 1 : 0;
  if (gateup) {
    a.a = static_cast<const uint16_t *>(p.xh);
    a.a_stride = p.x_stride;
    a.a_bytes = (uint32_t)((size_t)p.T * p.x_stride * 2);
    a.perm_token = p.perm_token;
    a.act = static_cast<uint16_t *>(p.act);
    a.act_stride = p.act_stride;
  } else {
    a.a = static_cast<const uint16_t *>(p.act);
    a.a_stride = p.act_stride;
    a.a_bytes = (uint32_t)(p.pairs_total * p.act_stride * 2);
    a.perm_token = nullptr;
    if (p.ypair_bf16 && p.bf16)
      a.yb = reinterpret_cast<uint16_t *>(p.ypair);
    else
      a.y = p.ypair;
    a.y_stride = ex->H;
    a.y_split = p.pairs_total * (size_t)ex->H;
  }
  const int rows = a.rows > a.srows ? a.rows : a.srows;
  const int BN = gemm_bn(ex->fmt, gateup);
  a.n_tiles = (rows + BN - 1) / BN;
  // tile order (see k_gemm): gate/up with at most two M-tiles per active
  // expert on average takes the XCD-chunked M-tile-major order (an M-tile's
  // N-tiles share its activation tile in one L2), with more the XCD split
  // by N-tiles (an N-tile group's weights serve all of the expert's
  // M-tiles).  Down takes the chunked order on the same condition, else
  // N-tiles fastest.  Measured: Qwen3 T = 512 gate/up 120 -> 101 us and
  // DeepSeek T = 4096 2.93 -> 2.82 ms (HBM reads 14.7 -> 9.9 GB) with the
  // chunked order; Mixtral Q8_0 prefill (four M-tiles per expert) 0.98 ->
  // 1.17 ms with it, so it keeps the split.  Down, chunked against N-tiles
  // fastest: Qwen3 T = 512 64.8 -> 62.4 us, T = 256 60.6 -> 59.5 us (the
  // M-tile's activation rows read through one L2 instead of every XCD's;
  // 49.7 -> 48.3 us and 46.2 -> 45.9 us with the half-window tail),
  // DeepSeek T = 4096 unchanged.  For many pairs per expert (Mixtral Q8_0
  // prefill) the chunked order or gate/up's XCD split by N-tiles is slower
  // (down 0.550 -> 0.559-0.569 ms).
  const long pairs = (long)p.T * p.k;
  const long active = std::max<long>(1, std::min<long>(ex->E, pairs));
  a.xcd_split = gateup ? (pairs <= 2L * p.tile_m * active ? 2 : 1)
                       : (pairs <= 2L * p.tile_m_down * active ? 2 : 0);
  // enough workgroups for the order at the largest M-tile count
  const long per = a.xcd_split == 1 ? 8L * ((a.n_tiles + 7) / 8) * max_tiles
                   : a.xcd_split == 2 ? 8L * (((long)a.n_tiles * max_tiles + 7) / 8)
                                      : (long)a.n_tiles * max_tiles;
  a.ksplit = gateup ? 1 : p.ksplit;
  a.wg_per_split = (int)per;
  const long wgs = per * a.ksplit;
  if (wgs > 0x7FFFFFFFL) return fail(NX_ERR_UNSUPPORTED, "grouped GEMM grid too large");
  GemmFn fn = pick(ex->fmt, p.bf16, gateup, gateup ? p.tile_m : p.tile_m_down,
                   a.half_win >= 0 || a.shalf_win >= 0);
  if (!fn) return fail(NX_ERR_UNSUPPORTED, "no grouped-GEMM kernel for this format");
  const char *name = gateup ? "gemm_gateup" : "gemm_down";
  return launch(c, name,
                [&] { go(c, fn, dim3((unsigned)wgs), dim3(256), 0, a); });
}

template <int FMT>
int to_half_fmt(nx_ctx *c, const float *x, int T, int H, int kpad, bool bf16, uint16_t *o) {
  if (kpad % 16 == 0 && T <= 65535 && ((uintptr_t)o & 15) == 0) {
    const bool vec = H % 4 == 0 && ((uintptr_t)x & 15) == 0;
    const int ng = kpad / 16;
    const dim3 grid((unsigned)std::max(1, std::min((ng + 255) / 256, 64)), (unsigned)T);
    if (bf16)
      return launch(c, "to_bf16", [&] {
        go(c, k_to_half16<FMT, true>, dim3(grid), dim3(256), 0, x, H, kpad, vec, o);
      });
    return launch(c, "to_f16", [&] {
      go(c, k_to_half16<FMT, false>, dim3(grid), dim3(256), 0, x, H, kpad, vec, o);
    });
  }
  size_t gblocks = ((size_t)T * kpad + 255) / 256;
  if (gblocks > 65536) gblocks = 65536;
  const unsigned gb = (unsigned)gblocks;
  if (bf16)
    return launch(c, "to_bf16",
                  [&] { go(c, k_to_half<FMT, true>, dim3(gb), dim3(256), 0, x, T, H, kpad, o); });
  return launch(c, "to_f16",
                [&] { go(c, k_to_half<FMT, false>, dim3(gb), dim3(256), 0, x, T, H, kpad, o); });
}

}  // namespace

int gemm_tile_m(int fmt, bool gateup, int T, int k, int E) {
  // pairs per active expert, with the active count expected under uniform
  // routing, E (1 - (1 - k/E)^T)
  const double kk = std::min(1.0, (double)k / E);
  const double act = std::max(1.0, E * (1.0 - std::pow(1.0 - kk, (double)T)));
  const double per = (double)T * k / act;
  if (fmt != NX_FMT_F32 && per <= NARROW_PER_MAX) return BM_NARROW;
  // down: 160-pair tiles whenever experts average more than 96 pairs (fewer
  // tiles decode fewer weight tiles: Mixtral Q8_0 prefill, 512 per expert,
  // down 0.571 -> 0.552 ms, GEMMs 0.372 -> 0.375 of peak, step -2 us);
  // gate/up (Q4 formats) when one tile holds an expert's pairs (on Q8_0 the
  // 160-pair gate/up fits only with its codes one step ahead, and was
  // slower: 0.970 -> 0.985 ms)
  if (!gateup) return per > 96.0 ? BM_WIDE : BM_GATEUP;
  const bool wide_ok = fmt == NX_FMT_Q4_K || fmt == NX_FMT_Q4_0;
  return wide_ok && per > 96.0 && per <= BM_WIDE ? BM_WIDE : BM_GATEUP;
}

// workgroups per CU of the grouped GEMM on M-tiles of tile_m pairs
int gemm_wg_per_cu(int fmt, int tile_m) {
  if (fmt == NX_FMT_F32 || gemm_nt(fmt, false) == 4) return 1;
  return tile_m <= BM_NARROW ? OCC_NARROW : 2;
}

// K splits of the down pass: the count (1-4, each split at least four loop
// bodies) that best fills whole rounds of `slots` concurrent workgroups,
// with `tiles` M-tiles expected.
int gemm_down_ksplit(int fmt, int F, int H, int tiles, int slots) {
  const int steps = kpad_of(fmt, F) / BK;
  const int body = fmt == NX_FMT_F32 ? 4 : (fmt == NX_FMT_Q8_0 ? 8 : 16);
  const int nbody = (steps + body - 1) / body;
  const long wgs = (long)tiles * ((H + 127) / 128);
  int best = 1;
  double best_eff = 0;
  for (int ks = 1; ks <= 4; ++ks) {
    if (ks > 1 && nbody / ks < 4) break;
    const long w = wgs * ks;
    const long rounds = (w + slots - 1) / slots;
    const double eff = (double)w / (double)(rounds * slots);
    if (eff > best_eff + 0.02) {
      best = ks;
      best_eff = eff;
    }
  }
  return best;
}

int gemm_kpad(int fmt, int cols) { return kpad_of(fmt, cols); }

int launch_to_half(nx_ctx *c, int fmt, const float *x, int T, int H, int kpad, bool bf16,
                   void *out) {
  if (T == 0) return NX_OK;
  uint16_t *o = static_cast<uint16_t *>(out);
  switch (fmt) {
  case NX_FMT_Q4_K: return to_half_fmt<NX_FMT_Q4_K>(c, x, T, H, kpad, bf16, o);
  case NX_FMT_Q8_0: return to_half_fmt<NX_FMT_Q8_0>(c, x, T, H, kpad, bf16, o);
  case NX_FMT_Q4_0: return to_half_fmt<NX_FMT_Q4_0>(c, x, T, H, kpad, bf16, o);
  case NX_FMT_F32: return to_half_fmt<NX_FMT_F32>(c, x, T, H, kpad, bf16, o);
  }
  return fail(NX_ERR_UNSUPPORTED, "no operand conversion for this format");
}

int launch_gemm_gateup(nx_ctx *c, const GemmPlan &p) {
  // (act's pad columns are zeroed by the gate/up kernel's epilogue)
  return run(c, p, true);
}
int launch_gemm_down(nx_ctx *c, const GemmPlan &p) { return run(c, p, false); }

}  // namespace nx
