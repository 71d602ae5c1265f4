// nx_device.hpp — device helpers shared by the gfx950 kernels: f16 decode,
// resident-layout segment decoders, wavefront (DPP) reductions.
//
// Resident code-plane layout.  Each matrix row is cut into 32-byte
// "segments" of its code plane:
//   Q4_K (src/quant/mod.rs:820-849): segment j = block b = j/4, sub-block pair
//        s = j%4: qs bytes [32s, 32s+32) of the block.  Byte i holds element
//        b*256 + 32s + i (low nibble, sub-block s) and b*256 + 128 + 32s + i
//        (high nibble, sub-block s+4); y = d*sc*q - dmin*m.
//   Q8_0 (src/quant/mod.rs:689-703): segment j = block j, y = (int8)q * d.
//   Q4_0 (src/quant/mod.rs:723-745): segment j = blocks 2j and 2j+1 (16 B
//        each); byte i of block c holds c*32 + i (low) and c*32 + 16 + i
//        (high), y = (q - 8) * d.
//   F32: segment j = floats 8j .. 8j+7.
// Segments are stored half-interleaved per group of 64: half h (16 B) of
// segment j lives at (j/64)*2048 + h*G*16 + (j%64)*16 with G the group's
// size, so the 64 lanes of a wave that own 64 consecutive segments read two
// fully contiguous 1 KB runs.  Each segment's values are ordered so that its
// x operand is one or two contiguous runs of the activation row.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/nexus_hip.h"

namespace nx {

__device__ __forceinline__ float h2f(uint32_t bits16) {
  _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits16);
  return (float)h;
}

// Nibble masks reach the kernels as arguments (GemvArgs::mask_lo/mask_hi):
// with compile-time masks the compiler folds mask-then-convert into a 4-bit
// field extract plus a convert; with opaque masks each byte of the masked
// word converts with a single v_cvt_f32_ubyteN.
__device__ __forceinline__ float ub0(uint32_t w) { return (float)(w & 0xFFu); }
__device__ __forceinline__ float ub1(uint32_t w) { return (float)((w >> 8) & 0xFFu); }
__device__ __forceinline__ float ub2(uint32_t w) { return (float)((w >> 16) & 0xFFu); }
__device__ __forceinline__ float ub3(uint32_t w) { return (float)(w >> 24); }

// sum_i byte_i(w) * x[i] for the four bytes of w
__device__ __forceinline__ float dot4u(uint32_t w, const float *x, float acc) {
  acc = fmaf(ub0(w), x[0], acc);
  acc = fmaf(ub1(w), x[1], acc);
  acc = fmaf(ub2(w), x[2], acc);
  acc = fmaf(ub3(w), x[3], acc);
  return acc;
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
// offset that lies past any matrix (loads there return zeros)
constexpr uint32_t OOB = 0x7FFFFFF0u;

// streaming 16-byte load (weights are read once per pass)
__device__ __forceinline__ uint4 ld_stream16(const uint8_t *p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// half-interleaved offset of half h of segment j in a row of nseg segments
__device__ __forceinline__ uint32_t seg_off(int j, int h, int nseg) {
  const int g = j >> 6;
  const int gsz = min(64, nseg - (g << 6));
  return (uint32_t)(g * 2048 + h * gsz * 16 + (j & 63) * 16);
}

template <int FMT>
struct Seg;

template <>
struct Seg<NX_FMT_Q4_K> {
  static constexpr int EPS = 64;  // elements per segment
  static constexpr int NXS = 2;   // x partial sums kept per segment
  using Meta = uint4;
  __device__ __forceinline__ static int xidx(int j, int v) {
    return (j >> 2) * 256 + (j & 3) * 32 + (v & 31) + ((v >> 5) << 7);
  }
  // scale-plane byte offset of segment j within its row (OOB when invalid)
  __device__ __forceinline__ static uint32_t meta_off(int j, bool valid) {
    return valid ? (uint32_t)((j >> 2) * 16) : OOB;
  }
  __device__ __forceinline__ static Meta load_meta(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return bload16(r, off);
  }
  __device__ __forceinline__ static void xsums(const float *x, float *xs) {
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) a += x[i];
#pragma unroll
    for (int i = 0; i < 32; ++i) b += x[32 + i];
    xs[0] = a;
    xs[1] = b;
  }
  // sum over the segment of w*x for NT tokens
  template <int NT>
  __device__ __forceinline__ static void dot(const uint4 &q0, const uint4 &q1, const Meta &m,
                                             int j, const float (*x)[EPS],
                                             const float (*xs)[NXS], float *acc, uint32_t mlo,
                                             uint32_t mhi) {
    const float d = h2f(m.x & 0xFFFFu), dmin = h2f(m.x >> 16);
    const int s = j & 3;
    const uint32_t b0 = (m.y >> (8 * s)) & 0xFFu;  // scales12[s]
    const uint32_t b4 = (m.z >> (8 * s)) & 0xFFu;  // scales12[s+4]
    const uint32_t b8 = (m.w >> (8 * s)) & 0xFFu;  // scales12[s+8]
    const float s_lo = d * (float)(b0 & 63u);
    const float m_lo = dmin * (float)(b4 & 63u);
    // high nibbles are converted in place (16*q), so their scale carries 1/16
    const float s_hi = d * (float)((b8 & 15u) | ((b0 >> 6) << 4)) * 0.0625f;
    const float m_hi = dmin * (float)((b8 >> 4) | ((b4 >> 6) << 4));
    const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    float lo[NT], hi[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) lo[t] = hi[t] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t l = w[i] & mlo;
      const uint32_t h = w[i] & mhi;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        lo[t] = dot4u(l, &x[t][4 * i], lo[t]);
        hi[t] = dot4u(h, &x[t][32 + 4 * i], hi[t]);
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t)
      acc[t] += (s_lo * lo[t] - m_lo * xs[t][0]) + (s_hi * hi[t] - m_hi * xs[t][1]);
  }
};

template <>
struct Seg<NX_FMT_Q8_0> {
  static constexpr int EPS = 32;
  static constexpr int NXS = 1;
  using Meta = uint32_t;
  __device__ __forceinline__ static int xidx(int j, int v) { return j * 32 + v; }
  __device__ __forceinline__ static uint32_t meta_off(int j, bool valid) {
    return valid ? (uint32_t)(j * 2) : OOB;
  }
  // the f16 scale may sit in either half of an aligned dword
  __device__ __forceinline__ static Meta load_meta(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const uint32_t w = bload4(r, off & ~3u);
    return (off & 2u) ? (w >> 16) : (w & 0xFFFFu);
  }
  __device__ __forceinline__ static void xsums(const float *x, float *xs) {
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) a += x[i];
    xs[0] = a;
  }
  // signed codes are read as unsigned q + 128 (byte xor 0x80): sum (q+128) x - 128 sum x
  template <int NT>
  __device__ __forceinline__ static void dot(const uint4 &q0, const uint4 &q1, const Meta &m,
                                             int, const float (*x)[EPS],
                                             const float (*xs)[NXS], float *acc, uint32_t,
                                             uint32_t mflip) {
    const float d = h2f(m);
    const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    uint32_t u[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) u[i] = w[i] ^ mflip;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      float a = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) a = dot4u(u[i], &x[t][4 * i], a);
      acc[t] += d * (a - 128.f * xs[t][0]);
    }
  }
};

template <>
struct Seg<NX_FMT_Q4_0> {
  static constexpr int EPS = 64;
  static constexpr int NXS = 2;
  using Meta = uint32_t;  // two f16 scales (blocks 2j, 2j+1)
  __device__ __forceinline__ static int xidx(int j, int v) { return j * 64 + v; }
  __device__ __forceinline__ static uint32_t meta_off(int j, bool valid) {
    return valid ? (uint32_t)(j * 4) : OOB;
  }
  __device__ __forceinline__ static Meta load_meta(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return bload4(r, off);
  }
  __device__ __forceinline__ static void xsums(const float *x, float *xs) {
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) a += x[i];
#pragma unroll
    for (int i = 0; i < 32; ++i) b += x[32 + i];
    xs[0] = a;
    xs[1] = b;
  }
  template <int NT>
  __device__ __forceinline__ static void dot(const uint4 &q0, const uint4 &q1, const Meta &m,
                                             int, const float (*x)[EPS],
                                             const float (*xs)[NXS], float *acc, uint32_t mlo,
                                             uint32_t mhi) {
    const float d0 = h2f(m & 0xFFFFu), d1 = h2f(m >> 16);
    const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      float a0 = 0.f, b0 = 0.f, a1 = 0.f, b1 = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t l0 = w[i] & mlo, h0 = w[i] & mhi;
        const uint32_t l1 = w[4 + i] & mlo, h1 = w[4 + i] & mhi;
        a0 = dot4u(l0, &x[t][4 * i], a0);
        b0 = dot4u(h0, &x[t][16 + 4 * i], b0);
        a1 = dot4u(l1, &x[t][32 + 4 * i], a1);
        b1 = dot4u(h1, &x[t][48 + 4 * i], b1);
      }
      acc[t] += d0 * (a0 + 0.0625f * b0 - 8.f * xs[t][0]) + d1 * (a1 + 0.0625f * b1 - 8.f * xs[t][1]);
    }
  }
};

template <>
struct Seg<NX_FMT_F32> {
  static constexpr int EPS = 8;
  static constexpr int NXS = 1;
  using Meta = uint32_t;
  __device__ __forceinline__ static int xidx(int j, int v) { return j * 8 + v; }
  __device__ __forceinline__ static uint32_t meta_off(int, bool) { return 0; }
  __device__ __forceinline__ static Meta load_meta(__amdgpu_buffer_rsrc_t, uint32_t) { return 0; }
  __device__ __forceinline__ static void xsums(const float *, float *xs) { xs[0] = 0.f; }
  template <int NT>
  __device__ __forceinline__ static void dot(const uint4 &q0, const uint4 &q1, const Meta &, int,
                                             const float (*x)[EPS], const float (*)[NXS],
                                             float *acc, uint32_t, uint32_t) {
    const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      float a = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) a = fmaf(__uint_as_float(w[i]), x[t][i], a);
      acc[t] += a;
    }
  }
};

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

__device__ __forceinline__ float silu_mul(float g, float u) {
  return (g / (1.0f + expf(-g))) * u;
}

}  // namespace nx
