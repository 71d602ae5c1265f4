// nx_device.hpp — device helpers shared by the gfx950 kernels: f16 decode,
// resident-layout segment decoders, wavefront (DPP) reductions.
//
// Resident code-plane layout.  Each matrix row is cut into 32-byte
// "segments" of its code plane:
//   Q4_K (src/quant/mod.rs:820-849): segment j = block b = j/4, sub-block pair
//        s = j%4: half 0 holds the 32 codes of sub-block s (block elements
//        32s ..), half 1 those of sub-block s+4 (elements 128 + 32s ..);
//        y = d*sc*q - dmin*m.
//   Q4_0 (src/quant/mod.rs:723-745): segment j = blocks 2j (half 0) and 2j+1
//        (half 1); y = (q - 8) * d.
//   In both 4-bit formats the 16 bytes of a half hold one 32-element
//   sub-block: byte 4k+i has element 8k+i in its low nibble and element
//   8k+4+i in its high nibble, each stored as q ^ 8 (the two's-complement
//   4-bit form of q - 8).
//   Q8_0 (src/quant/mod.rs:689-703): segment j = block j in element order,
//        y = (int8)q * d.
//   F32: segment j = floats 8j .. 8j+7.
// Segments are stored half-interleaved per group of 64: within a group of G
// segments, half h (16 B) of segment j lives at h*G*16 + (j%64)*16, so the
// 64 lanes of a wave that own 64 consecutive segments read two fully
// contiguous 1 KB runs.  Rows longer than one group are stored in panels, one
// per group (see panel_row_off below).  Each segment's values are ordered so
// that its x operand is one or two contiguous runs of the activation row.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/nexus_hip.h"

namespace nx {

__device__ __forceinline__ float h2f(uint32_t bits16) {
  _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits16);
  return (float)h;
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Raw buffer resources: 32-bit byte offsets, and any load at or beyond
// `bytes` returns zeros instead of touching memory, so out-of-range rows and
// segments need no branches.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                           0x00020000);
}
__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint32_t bload4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}
// cache policy of the GEMV's scale-plane loads (2: non-temporal)
#ifndef NX_GEMV_META_CPOL
#define NX_GEMV_META_CPOL 0
#endif
__device__ __forceinline__ uint4 bload16m(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, NX_GEMV_META_CPOL);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint32_t bload4m(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, NX_GEMV_META_CPOL);
}
// offset that lies past any matrix (loads there return zeros)
constexpr uint32_t OOB = 0x7FFFFFF0u;

// streaming 16-byte load (weights are read once per pass)
__device__ __forceinline__ uint4 ld_stream16(const uint8_t *p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// ---- Panels.  A matrix whose rows hold more than 64 segments is stored one
// panel per group of 64 segments: group g of every row (gsz = min(64, nseg -
// 64 g) segments) forms the panel [rows x 64 segments] at g * rows * 64 *
// unit bytes (unit = a segment's bytes in the plane), its row parts one after
// another; inside a panel row the group keeps the layout above, and the last
// group, when shorter, is followed by zeros up to the panel row's end.  A
// kernel that streams one group of many rows (the K-sliced decode down pass)
// then reads one contiguous run: 2 KB pieces of rows 7 KB apart (the
// row-major form of Mixtral's down rows) read at 3.6 TB/s on one MI355X, the
// same bytes in panels at 5.3 TB/s.  Rows of at most 64 segments are one
// panel without padding: the plain row-major layout.
__host__ __device__ __forceinline__ int panel_gsz(int g, int nseg) {
  const int s = nseg - 64 * g;
  return s < 0 ? 0 : (s > 64 ? 64 : s);
}
// panels of a row of nseg segments
__host__ __device__ __forceinline__ int panel_count(int nseg) { return nseg > 64 ? (nseg + 63) / 64 : 1; }
// bytes of one row's part of a panel: 64 segments' when the row spans several
// panels, else the row's own (in whole dwords: Q8_0's 2-byte scales)
__host__ __device__ __forceinline__ uint32_t panel_row_bytes(int nseg, int unit) {
  return nseg > 64 ? 64u * (uint32_t)unit : ((uint32_t)(nseg * unit) + 3u) & ~3u;
}
// offset of row r's part of panel g in a plane of `rows` rows
__host__ __device__ __forceinline__ uint32_t panel_row_off(int r, int g, int rows, int nseg,
                                                           int unit) {
  return ((uint32_t)g * (uint32_t)rows + (uint32_t)r) * panel_row_bytes(nseg, unit);
}
// offset of half h of segment j within its panel row (32-byte segments)
__host__ __device__ __forceinline__ uint32_t seg_off(int j, int h, int nseg) {
  return (uint32_t)(h * panel_gsz(j >> 6, nseg) * 16 + (j & 63) * 16);
}
// offset of half h of segment j of row r in a code plane of 32-byte segments
__host__ __device__ __forceinline__ uint32_t code_off(int r, int j, int h, int rows, int nseg) {
  return panel_row_off(r, j >> 6, rows, nseg, 32) + seg_off(j, h, nseg);
}

// 16-byte code chunks per segment: two (the halves above) for every format
// but Q2_K, whose 2-bit codes fill one chunk per segment, stored at 16 j
template <int FMT>
constexpr int code_chunks() {
  return FMT == NX_FMT_Q2_K ? 1 : 2;
}

// ---- Integer-dot GEMV operands.
//
// The decode GEMV computes sum_i q_i x_i with exact integer dot products.  A
// lane's activations over one segment are put in 24-bit block fixed point:
// with E the binary exponent of max|x| (max|x| < 2^E), X_i = round(x_i *
// 2^(22-E)) is an integer in [-2^22, 2^22] and x_i = X_i * 2^(E-22) up to
// half a unit of 2^(E-22) (relative precision 2^-23 of the block maximum).
// X is computed with the 1.5*2^23 rounding constant: the bits of
// fma(x, 2^(22-E), 1.5*2^23) are 0x4B400000 + X.
//
// 4-bit codes (Q4_K, Q4_0) are stored as signed nibbles c = q - 8.  X is
// split into six balanced 4-bit digits D_d in [-8, 8): Z = X + 0x888888 lies
// in [0, 2^24) and D_d = digit_d(Z) - 8, the signed nibble digit_d(Z) ^ 8.
// The repacked code dword k of a 32-element sub-block holds elements 8k+i
// (low nibble of byte i) and 8k+4+i (high nibble); digit plane d holds D_d of
// the same elements at the same nibble positions, so one v_dot8_i32_i4 per
// digit gives a_d = sum_i c_i D_d,i, and sum_i c_i X_i = sum_d 16^d a_d is
// exact in 32 bits; then sum_i q_i x_i = 2^(E-22) * that + 8 * sum_i x_i.
//
// Q8_0: Z = X + 0x808080 has base-256 digits z_d in [0, 256); z_d - 128 =
// (z_d ^ 0x80) as a signed byte is a balanced digit D_d with X = D0 + 256 D1 +
// 65536 D2, so three v_dot4_i32_i8 per code dword give the sums exactly.
//
// Non-finite activations give NaN for the whole segment.

// binary exponent of m (m < 2^E), clamped so that both 2^(22-E) and
// 2^(E-22) stay normal floats
__device__ __forceinline__ int blk_exp(float m) {
  const int e = __builtin_amdgcn_frexp_expf(m);
  return e < -100 ? -100 : (e > 128 ? 128 : e);
}

__device__ __forceinline__ float abs_max(const float *x, int n) {
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < n; ++i) m = fmaxf(m, fabsf(x[i]));
  return m;
}

// bytes b of four words -> one word (b in 0..1 pairs, b = 2 alone)
__device__ __forceinline__ void byte_transpose4(const uint32_t *y, uint32_t &b0, uint32_t &b1,
                                                uint32_t &b2) {
  const uint32_t t01 = __builtin_amdgcn_perm(y[1], y[0], 0x05010400u);
  const uint32_t t23 = __builtin_amdgcn_perm(y[3], y[2], 0x05010400u);
  b0 = __builtin_amdgcn_perm(t23, t01, 0x05040100u);
  b1 = __builtin_amdgcn_perm(t23, t01, 0x07060302u);
  const uint32_t u01 = __builtin_amdgcn_perm(y[1], y[0], 0x0C0C0602u);
  const uint32_t u23 = __builtin_amdgcn_perm(y[3], y[2], 0x0C0C0602u);
  b2 = __builtin_amdgcn_perm(u23, u01, 0x05040100u);
}

// 8 activations (one code dword) -> their six 4-bit digit-plane dwords
__device__ __forceinline__ void plane4_dword(const float *x, float sc, uint32_t (&o)[6]) {
  uint32_t y[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    y[i] = (__float_as_uint(fmaf(x[i], sc, 12582912.0f)) - (0x4B400000u - 0x888888u)) ^ 0x888888u;
  uint32_t lo[3], hi[3];
  byte_transpose4(y, lo[0], lo[1], lo[2]);
  byte_transpose4(y + 4, hi[0], hi[1], hi[2]);
  constexpr uint32_t M = 0x0F0F0F0Fu;
#pragma unroll
  for (int b = 0; b < 3; ++b) {
    o[2 * b] = (lo[b] & M) | ((hi[b] << 4) & ~M);
    o[2 * b + 1] = ((lo[b] >> 4) & M) | (hi[b] & ~M);
  }
}

// 32 activations of one 4-bit sub-block -> digit planes p[digit][dword]
__device__ __forceinline__ void planes4(const float *x, float sc, uint32_t (&p)[6][4]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    uint32_t o[6];
    plane4_dword(x + 8 * k, sc, o);
#pragma unroll
    for (int d = 0; d < 6; ++d) p[d][k] = o[d];
  }
}

// 4 activations (one Q8_0 code dword) -> their three byte-digit plane dwords
__device__ __forceinline__ void plane8_dword(const float *x, float sc, uint32_t &p0, uint32_t &p1,
                                             uint32_t &p2) {
  uint32_t z[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    z[i] = (__float_as_uint(fmaf(x[i], sc, 12582912.0f)) - (0x4B400000u - 0x808080u)) ^ 0x808080u;
  byte_transpose4(z, p0, p1, p2);
}

// Per-token accumulator state of the integer dot.  The signed dot
// instructions of gfx950 accumulate in place (v_dot8c / v_dot4c).
//   4-bit: each sub-block's digits are accumulated Horner-style into one
//     register, acc = 16 * acc + sum_i c_i D_d,i for d = 5 .. 0, which ends as
//     sum_i c_i X_i exactly (|sum| <= 32 * 8 * 2^22 < 2^31).
//   Q8_0: the sum does not fit in 32 bits, so D1 and D0 share one register
//     (256 * a1 + a0, < 2^28) and D2 has its own; these run for the whole
//     kernel and each segment's sums are differences of snapshots taken
//     modulo 2^32 (exact, since one segment's true sums fit).
struct Run4 {};
struct Run8 {
  int32_t i, a2;
  uint32_t si, sa2;  // last snapshot
};
template <class R>
__device__ __forceinline__ void run_init(R &) {}
__device__ __forceinline__ void run_init(Run8 &r) { r.i = r.a2 = 0, r.si = r.sa2 = 0; }

// sum_i c_i X_i over one 4-bit sub-block (signed codes w, planes p)
__device__ __forceinline__ float sumcx4(const uint4 &w, const uint32_t (&p)[6][4], Run4 &) {
  const int ws[4] = {(int)w.x, (int)w.y, (int)w.z, (int)w.w};
  int32_t acc = 0;
#pragma unroll
  for (int d = 5; d >= 0; --d) {
    if (d < 5) acc = (int32_t)((uint32_t)acc << 4);
#pragma unroll
    for (int k = 0; k < 4; ++k) acc = __builtin_amdgcn_sdot8(ws[k], (int)p[d][k], acc, false);
  }
  return (float)acc;
}

// activations of one 64-element 4-bit segment (two sub-blocks)
struct X4 {
  uint32_t p[2][6][4];
  float post;  // 2^(E-22), or NaN for non-finite activations
  float s[2];  // sub-block sums of x
};

// ---- Quad-cooperative preparation: the lanes 4i .. 4i+3 of a wave build one
// segment's operand together, lane q from the q-th quarter of its elements
// (EPS/4 consecutive values of the segment order); the block exponent and the
// sums come from quad DPP reductions.  o points into LDS.
__device__ __forceinline__ float quad_max(float m) {
  m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0xB1, 0xF, 0xF, true)));
  return fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x4E, 0xF, 0xF, true)));
}
__device__ __forceinline__ float quad_pair_sum(float v) {  // lanes (0,1), (2,3)
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, true));
}
__device__ __forceinline__ float quad_swap_halves(float v) {  // lanes (0,1) <-> (2,3)
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, true));
}

// quarter q of a 4-bit segment = dwords 2(q&1), 2(q&1)+1 of sub-block q>>1
__device__ __forceinline__ void prep4_quarter(const float *x, int q, X4 *o) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += x[i];
  const float sp = quad_pair_sum(s);        // this sub-block
  const float sa = sp + quad_swap_halves(sp);  // the segment
  const int e = blk_exp(quad_max(abs_max(x, 16)));
  const float sc = __builtin_amdgcn_ldexpf(1.0f, 22 - e);
  const int h = q >> 1, k0 = (q & 1) * 2;
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    uint32_t pd[6];
    plane4_dword(x + 8 * kk, sc, pd);
#pragma unroll
    for (int d = 0; d < 6; ++d) o->p[h][d][k0 + kk] = pd[d];
  }
  if ((q & 1) == 0) o->s[h] = sp;
  if (q == 0)
    o->post = fabsf(sa) <= 3.4e38f ? __builtin_amdgcn_ldexpf(1.0f, e - 22) : __builtin_nanf("");
}

__device__ __forceinline__ void prep4(const float *x, X4 &o) {
  float a = 0.f, b = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) a += x[i];
#pragma unroll
  for (int i = 0; i < 32; ++i) b += x[32 + i];
  o.s[0] = a;
  o.s[1] = b;
  const int e = blk_exp(abs_max(x, 64));
  const float sc = __builtin_amdgcn_ldexpf(1.0f, 22 - e);
  o.post = fabsf(a + b) <= 3.4e38f ? __builtin_amdgcn_ldexpf(1.0f, e - 22) : __builtin_nanf("");
  planes4(x, sc, o.p[0]);
  planes4(x + 32, sc, o.p[1]);
}

// activations of one 64-element Q2_K segment: the digit planes of its two
// 32-element halves plus the sum of each 16-element sub-block
struct X2 {
  uint32_t p[2][6][4];
  float post;
  float s[4];
};

__device__ __forceinline__ void prep2(const float *x, X2 &o) {
  float a = 0.f;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    float su = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) su += x[16 * u + i];
    o.s[u] = su;
    a += su;
  }
  const int e = blk_exp(abs_max(x, 64));
  const float sc = __builtin_amdgcn_ldexpf(1.0f, 22 - e);
  o.post = fabsf(a) <= 3.4e38f ? __builtin_amdgcn_ldexpf(1.0f, e - 22) : __builtin_nanf("");
  planes4(x, sc, o.p[0]);
  planes4(x + 32, sc, o.p[1]);
}

// quarter q of a Q2_K segment = its sub-block q (dwords 2(q&1), 2(q&1)+1 of
// half q>>1)
__device__ __forceinline__ void prep2_quarter(const float *x, int q, X2 *o) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += x[i];
  const float sp = quad_pair_sum(s);
  const float sa = sp + quad_swap_halves(sp);
  const int e = blk_exp(quad_max(abs_max(x, 16)));
  const float sc = __builtin_amdgcn_ldexpf(1.0f, 22 - e);
  const int h = q >> 1, k0 = (q & 1) * 2;
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    uint32_t pd[6];
    plane4_dword(x + 8 * kk, sc, pd);
#pragma unroll
    for (int d = 0; d < 6; ++d) o->p[h][d][k0 + kk] = pd[d];
  }
  o->s[q] = s;
  if (q == 0)
    o->post = fabsf(sa) <= 3.4e38f ? __builtin_amdgcn_ldexpf(1.0f, e - 22) : __builtin_nanf("");
}

// sum_i c_i X_i over the two 16-element sub-blocks of a 4-bit code half:
// dwords 0-1 (first) and 2-3 (second)
__device__ __forceinline__ void sumcx4_split(const uint4 &w, const uint32_t (&p)[6][4], float &f0,
                                             float &f1) {
  const int ws[4] = {(int)w.x, (int)w.y, (int)w.z, (int)w.w};
  int32_t a0 = 0, a1 = 0;
#pragma unroll
  for (int d = 5; d >= 0; --d) {
    if (d < 5) {
      a0 = (int32_t)((uint32_t)a0 << 4);
      a1 = (int32_t)((uint32_t)a1 << 4);
    }
    a0 = __builtin_amdgcn_sdot8(ws[0], (int)p[d][0], a0, false);
    a0 = __builtin_amdgcn_sdot8(ws[1], (int)p[d][1], a0, false);
    a1 = __builtin_amdgcn_sdot8(ws[2], (int)p[d][2], a1, false);
    a1 = __builtin_amdgcn_sdot8(ws[3], (int)p[d][3], a1, false);
  }
  f0 = (float)a0;
  f1 = (float)a1;
}

template <int FMT>
struct Seg;

template <>
struct Seg<NX_FMT_Q4_K> {
  static constexpr int EPS = 64;  // elements per segment
  using Meta = uint4;
  using X = X4;
  using Run = Run4;
  // segment element v: sub-block s = j%4 (v < 32), sub-block s+4 (v >= 32)
  __device__ __forceinline__ static int xidx(int j, int v) {
    return (j >> 2) * 256 + (j & 3) * 32 + (v & 31) + ((v >> 5) << 7);
  }
  static constexpr int MU = 4;  // scale-plane bytes per segment (16 per block)
  // scale-plane byte offset of segment j within its panel row (OOB when
  // invalid)
  __device__ __forceinline__ static uint32_t meta_off(int j, bool valid) {
    return valid ? (uint32_t)(((j & 63) >> 2) * 16) : OOB;
  }
  __device__ __forceinline__ static Meta load_meta(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return bload16m(r, off);
  }
  __device__ __forceinline__ static void prep(const float *x, X &o) { prep4(x, o); }
  __device__ __forceinline__ static void prep_quarter(const float *x, int q, X *o) {
    prep4_quarter(x, q, o);
  }
  // sum over the segment of w*x for NT tokens; src/quant/mod.rs:841 gives
  // w = d*sc*q - dmin*m per element, summed here with q = c + 8 as
  // d*(sc_a*sum c x + sc_b*sum c x) + (8*d*sc - dmin*m) * sum x per sub-block
  template <int NT>
  __device__ __forceinline__ static void dot(const uint4 &q0, const uint4 &q1, const Meta &m,
                                             int j, const X *xv, Run *run, float *acc) {
    const float d = h2f(m.x & 0xFFFFu), dmin = h2f(m.x >> 16);
    const int s = j & 3;
    const uint32_t b0 = (m.y >> (8 * s)) & 0xFFu;  // scales12[s]
    const uint32_t b4 = (m.z >> (8 * s)) & 0xFFu;  // scales12[s+4]
    const uint32_t b8 = (m.w >> (8 * s)) & 0xFFu;  // scales12[s+8]
    const float sa = (float)(b0 & 63u), ma = (float)(b4 & 63u);
    const float sb = (float)((b8 & 15u) | ((b0 >> 6) << 4));
    const float mb = (float)((b8 >> 4) | ((b4 >> 6) << 4));
    const float ka = 8.0f * d * sa - dmin * ma, kb = 8.0f * d * sb - dmin * mb;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const float fa = sumcx4(q0, xv[t].p[0], run[t]);
      const float fb = sumcx4(q1, xv[t].p[1], run[t]);
      const float cx = fmaf(sa, fa, sb * fb) * (d * xv[t].post);
      acc[t] += cx + fmaf(ka, xv[t].s[0], kb * xv[t].s[1]);
    }
  }
};

template <>
struct Seg<NX_FMT_Q8_0> {
  static constexpr int EPS = 32;
  using Meta = uint32_t;
  using Run = Run8;
  struct X {
    uint32_t p[3][8];
    float post;
  };
  __device__ __forceinline__ static int xidx(int j, int v) { return j * 32 + v; }
  static constexpr int MU = 2;  // scale-plane bytes per segment
  __device__ __forceinline__ static uint32_t meta_off(int j, bool valid) {
    return valid ? (uint32_t)((j & 63) * 2) : OOB;
  }
  // the f16 scale may sit in either half of an aligned dword
  __device__ __forceinline__ static Meta load_meta(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const uint32_t w = bload4m(r, off & ~3u);
    return (off & 2u) ? (w >> 16) : (w & 0xFFFFu);
  }
  __device__ __forceinline__ static void prep(const float *x, X &o) {
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) a += x[i];
    const int e = blk_exp(abs_max(x, 32));
    const float sc = __builtin_amdgcn_ldexpf(1.0f, 22 - e);
    o.post = fabsf(a) <= 3.4e38f ? __builtin_amdgcn_ldexpf(1.0f, e - 22) : __builtin_nanf("");
#pragma unroll
    for (int k = 0; k < 8; ++k) plane8_dword(x + 4 * k, sc, o.p[0][k], o.p[1][k], o.p[2][k]);
  }
  // quarter q = dwords 2q, 2q+1
  __device__ __forceinline__ static void prep_quarter(const float *x, int q, X *o) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) s += x[i];
    const float sa = quad_pair_sum(s) + quad_swap_halves(quad_pair_sum(s));
    const int e = blk_exp(quad_max(abs_max(x, 8)));
    const float sc = __builtin_amdgcn_ldexpf(1.0f, 22 - e);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      uint32_t a, b, c;
      plane8_dword(x + 4 * kk, sc, a, b, c);
      o->p[0][2 * q + kk] = a;
      o->p[1][2 * q + kk] = b;
      o->p[2][2 * q + kk] = c;
    }
    if (q == 0)
      o->post = fabsf(sa) <= 3.4e38f ? __builtin_amdgcn_ldexpf(1.0f, e - 22) : __builtin_nanf("");
  }
  // src/quant/mod.rs:689-703: w = (int8)q * d
  template <int NT>
  __device__ __forceinline__ static void dot(const uint4 &q0, const uint4 &q1, const Meta &m, int,
                                             const X *xv, Run *run, float *acc) {
    const float d = h2f(m);
    const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      Run8 &r = run[t];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        r.a2 = __builtin_amdgcn_sdot4((int)w[k], (int)xv[t].p[2][k], r.a2, false);
        r.i = __builtin_amdgcn_sdot4((int)w[k], (int)xv[t].p[1][k], r.i, false);
      }
      // the shared register holds 256 * (sum over D1) + (sum over D0)
      r.i = (int32_t)((uint32_t)r.i << 8);
#pragma unroll
      for (int k = 0; k < 8; ++k)
        r.i = __builtin_amdgcn_sdot4((int)w[k], (int)xv[t].p[0][k], r.i, false);
      // this segment's sums (the shift also scaled the previous value P by
      // 256): |256 * D1 part + D0 part| < 2^28, |D2 part| < 2^19
      const int32_t di = (int32_t)((uint32_t)r.i - (r.si << 8));
      const int32_t d2 = (int32_t)((uint32_t)r.a2 - r.sa2);
      r.si = (uint32_t)r.i;
      r.sa2 = (uint32_t)r.a2;
      const float f = fmaf((float)d2, 65536.0f, (float)di);
      acc[t] += f * d * xv[t].post;
    }
  }
};

template <>
struct Seg<NX_FMT_Q4_0> {
  static constexpr int EPS = 64;
  using Meta = uint32_t;  // two f16 scales (blocks 2j, 2j+1)
  using X = X4;
  using Run = Run4;
  __device__ __forceinline__ static int xidx(int j, int v) { return j * 64 + v; }
  static constexpr int MU = 4;  // scale-plane bytes per segment
  __device__ __forceinline__ static uint32_t meta_off(int j, bool valid) {
    return valid ? (uint32_t)((j & 63) * 4) : OOB;
  }
  __device__ __forceinline__ static Meta load_meta(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return bload4m(r, off);
  }
  __device__ __forceinline__ static void prep(const float *x, X &o) { prep4(x, o); }
  __device__ __forceinline__ static void prep_quarter(const float *x, int q, X *o) {
    prep4_quarter(x, q, o);
  }
  // src/quant/mod.rs:723-745: w = (q - 8) * d per block, and c = q - 8
  template <int NT>
  __device__ __forceinline__ static void dot(const uint4 &q0, const uint4 &q1, const Meta &m, int,
                                             const X *xv, Run *run, float *acc) {
    const float d0 = h2f(m & 0xFFFFu), d1 = h2f(m >> 16);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const float fa = sumcx4(q0, xv[t].p[0], run[t]);
      const float fb = sumcx4(q1, xv[t].p[1], run[t]);
      acc[t] += fmaf(d0, fa, d1 * fb) * xv[t].post;
    }
  }
};

// Q2_K (src/quant/mod.rs:913-937): the resident codes of a 64-element
// segment (block j/4, elements 64(j%4) ..) are its 2-bit q in one 16-byte
// chunk.  Dword k packs nibble dword k of both 32-element halves in the 4-bit
// dword order (byte 4k+i: elements 8k+i, 8k+4+i of the half): half 0's codes
// in bits 0-1 of each nibble, half 1's in bits 2-3, so
//   half 0 = c & 0x33333333,  half 1 = (c >> 2) & 0x33333333
// are the widened non-negative 4-bit codes (no offset).  The scale plane
// holds per segment {f16 d, f16 dmin, the four scale/min bytes}.
// w = d*sc*q - dmin*m per 16-element sub-block u:
//   sum w*x = d*sc_u * sum q x - dmin*m_u * sum x
template <>
struct Seg<NX_FMT_Q2_K> {
  static constexpr int EPS = 64;
  using Meta = uint2;
  using X = X2;
  using Run = Run4;
  __device__ __forceinline__ static int xidx(int j, int v) {
    return (j >> 2) * 256 + (j & 3) * 64 + v;
  }
  static constexpr int MU = 8;  // scale-plane bytes per segment
  __device__ __forceinline__ static uint32_t meta_off(int j, bool valid) {
    return valid ? (uint32_t)((j & 63) * 8) : OOB;
  }
  __device__ __forceinline__ static Meta load_meta(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, NX_GEMV_META_CPOL);
    return make_uint2(v[0], v[1]);
  }
  __device__ __forceinline__ static void prep(const float *x, X &o) { prep2(x, o); }
  __device__ __forceinline__ static void prep_quarter(const float *x, int q, X *o) {
    prep2_quarter(x, q, o);
  }
  // (q1, the second chunk of the other formats, is not loaded)
  template <int NT>
  __device__ __forceinline__ static void dot(const uint4 &q, const uint4 &, const Meta &m, int,
                                             const X *xv, Run *, float *acc) {
    constexpr uint32_t M2 = 0x33333333u;
    const uint4 q0 = make_uint4(q.x & M2, q.y & M2, q.z & M2, q.w & M2);
    const uint4 q1 = make_uint4((q.x >> 2) & M2, (q.y >> 2) & M2, (q.z >> 2) & M2, (q.w >> 2) & M2);
    const float d = h2f(m.x & 0xFFFFu), dmin = h2f(m.x >> 16);
    float ds[4], dm[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t b = (m.y >> (8 * u)) & 0xFFu;
      ds[u] = d * (float)(b & 15u);
      dm[u] = dmin * (float)(b >> 4);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      float f[4];
      sumcx4_split(q0, xv[t].p[0], f[0], f[1]);
      sumcx4_split(q1, xv[t].p[1], f[2], f[3]);
      const float cx = fmaf(ds[0], f[0], fmaf(ds[1], f[1], fmaf(ds[2], f[2], ds[3] * f[3])));
      const float mx = fmaf(dm[0], xv[t].s[0], fmaf(dm[1], xv[t].s[1],
                                                     fmaf(dm[2], xv[t].s[2], dm[3] * xv[t].s[3])));
      acc[t] += cx * xv[t].post - mx;
    }
  }
};

template <>
struct Seg<NX_FMT_F32> {
  static constexpr int EPS = 8;
  using Meta = uint32_t;
  struct Run {};
  struct X {
    float x[8];
  };
  __device__ __forceinline__ static int xidx(int j, int v) { return j * 8 + v; }
  static constexpr int MU = 0;  // no scale plane
  __device__ __forceinline__ static uint32_t meta_off(int, bool) { return 0; }
  __device__ __forceinline__ static Meta load_meta(__amdgpu_buffer_rsrc_t, uint32_t) { return 0; }
  __device__ __forceinline__ static void prep(const float *x, X &o) {
#pragma unroll
    for (int i = 0; i < 8; ++i) o.x[i] = x[i];
  }
  __device__ __forceinline__ static void prep_quarter(const float *, int, X *) {}
  template <int NT>
  __device__ __forceinline__ static void dot(const uint4 &q0, const uint4 &q1, const Meta &, int,
                                             const X *xv, Run *, float *acc) {
    const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      float a = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) a = fmaf(__uint_as_float(w[i]), xv[t].x[i], a);
      acc[t] += a;
    }
  }
};

// 16-bit floats: a 32-byte segment is 16 consecutive values of the row,
// converted exactly to f32 and fma'd with the activations
template <int FMT>
struct Seg16 {
  static constexpr int EPS = 16;
  using Meta = uint32_t;
  struct Run {};
  struct X {
    float x[16];
  };
  __device__ __forceinline__ static int xidx(int j, int v) { return j * 16 + v; }
  static constexpr int MU = 0;  // no scale plane
  __device__ __forceinline__ static uint32_t meta_off(int, bool) { return 0; }
  __device__ __forceinline__ static Meta load_meta(__amdgpu_buffer_rsrc_t, uint32_t) { return 0; }
  __device__ __forceinline__ static void prep(const float *x, X &o) {
#pragma unroll
    for (int i = 0; i < 16; ++i) o.x[i] = x[i];
  }
  __device__ __forceinline__ static void prep_quarter(const float *, int, X *) {}
  __device__ __forceinline__ static float lo(uint32_t w) {
    if constexpr (FMT == NX_FMT_F16) return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu));
    return __uint_as_float(w << 16);
  }
  __device__ __forceinline__ static float hi(uint32_t w) {
    if constexpr (FMT == NX_FMT_F16) return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
    return __uint_as_float(w & 0xFFFF0000u);
  }
  template <int NT>
  __device__ __forceinline__ static void dot(const uint4 &q0, const uint4 &q1, const Meta &, int,
                                             const X *xv, Run *, float *acc) {
    const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      float a = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        a = fmaf(lo(w[i]), xv[t].x[2 * i], a);
        a = fmaf(hi(w[i]), xv[t].x[2 * i + 1], a);
      }
      acc[t] += a;
    }
  }
};
template <>
struct Seg<NX_FMT_F16> : Seg16<NX_FMT_F16> {};
template <>
struct Seg<NX_FMT_BF16> : Seg16<NX_FMT_BF16> {};

// ---- DPP reductions.  After group_sum<L>, the last lane of each group of L
// lanes (L = 16, 32, 64) holds the group's sum.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dppf(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, true));
}

template <int L>
__device__ __forceinline__ float group_sum(float v) {
  v += dppf<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dppf<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dppf<0x114>(v);  // row_shr:4
  v += dppf<0x118>(v);  // row_shr:8
  if constexpr (L >= 32) v += dppf<0x142, 0xA>(v);  // row_bcast:15
  if constexpr (L >= 64) v += dppf<0x143, 0xC>(v);  // row_bcast:31
  return v;
}

// the same reduction applied step by step to N independent values, so the
// DPP read-after-write waits of one chain are filled by the others
template <int L, int N>
__device__ __forceinline__ void group_sum_n(float *v) {
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dppf<0xB1>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dppf<0x4E>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dppf<0x114>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dppf<0x118>(v[i]);
  if constexpr (L >= 32) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += dppf<0x142, 0xA>(v[i]);
  }
  if constexpr (L >= 64) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += dppf<0x143, 0xC>(v[i]);
  }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// SwiGLU: silu(g) * u = g * u / (1 + e^-g), with the hardware exp2 and
// reciprocal (about 1 ulp each); g -> -inf gives g*u*0 (NaN for infinite g,
// as the quotient form does)
__device__ __forceinline__ float silu_mul(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(-1.4426950408889634f * g);
  return (g * u) * __builtin_amdgcn_rcpf(1.0f + e);
}

}  // namespace nx
