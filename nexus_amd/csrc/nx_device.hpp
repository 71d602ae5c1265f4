// nx_device.hpp — device helpers shared by the gfx950 kernels: f16 decode,
// per-format chunk decoders, wavefront reductions.
//
// A "chunk" is the 16-byte unit one lane loads from a matrix row's code plane.
// Its element mapping follows the reference block layouts:
//   Q4_K (src/quant/mod.rs:820-849): block b = c/8, part p = c%8; byte i of the
//        chunk holds element b*256 + p*16 + i in its low nibble (sub-block p/2)
//        and element b*256 + 128 + p*16 + i in its high nibble (sub-block p/2+4);
//        y = d*sc*q - dmin*m.
//   Q8_0 (src/quant/mod.rs:689-703): block b = c/2, half h = c%2; byte i is
//        element b*32 + h*16 + i, y = (int8)q * d.
//   Q4_0 (src/quant/mod.rs:723-745): block b = c; byte i holds element b*32 + i
//        (low nibble) and b*32 + 16 + i (high nibble), y = (q - 8) * d.
//   F32: 4 consecutive floats.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/nexus_hip.h"

namespace nx {

__device__ __forceinline__ float h2f(uint32_t bits16) {
  _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits16);
  return (float)h;
}

__device__ __forceinline__ float ubyte(uint32_t w, int i) {
  return (float)((w >> (8 * i)) & 0xFFu);
}

__device__ __forceinline__ float sbyte(uint32_t w, int i) {
  return (float)(int32_t)((int8_t)((w >> (8 * i)) & 0xFFu));
}

template <int FMT>
struct Fmt;

template <>
struct Fmt<NX_FMT_Q4_K> {
  static constexpr int XPC = 32;  // x values per chunk
  static constexpr int CHUNKS_PER_BLOCK = 8;
  static constexpr int META = 16;
  // x index of value v (v < 16: low nibbles, v >= 16: high nibbles)
  __device__ __forceinline__ static int xidx(int c, int v) {
    return (c >> 3) * 256 + (c & 7) * 16 + (v & 15) + ((v >> 4) << 7);
  }
  // Decoded chunk: 32 code values as floats plus the affine terms per half.
  struct Dec {
    float q[32];
    float s_lo, m_lo, s_hi, m_hi;  // d*sc, dmin*m for low / high half
  };
  __device__ __forceinline__ static void decode(const uint4 &w, const uint8_t *meta_row, int c,
                                                Dec &o) {
    const uint4 m = *reinterpret_cast<const uint4 *>(meta_row + (c >> 3) * 16);
    const float d = h2f(m.x & 0xFFFFu), dmin = h2f(m.x >> 16);
    const int s = (c & 7) >> 1;
    const uint32_t b0 = (m.y >> (8 * s)) & 0xFFu;  // scales12[s]
    const uint32_t b4 = (m.z >> (8 * s)) & 0xFFu;  // scales12[s+4]
    const uint32_t b8 = (m.w >> (8 * s)) & 0xFFu;  // scales12[s+8]
    o.s_lo = d * (float)(b0 & 63u);
    o.m_lo = dmin * (float)(b4 & 63u);
    o.s_hi = d * (float)((b8 & 15u) | ((b0 >> 6) << 4));
    o.m_hi = dmin * (float)((b8 >> 4) | ((b4 >> 6) << 4));
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t lo = ws[j] & 0x0F0F0F0Fu;
      const uint32_t hi = (ws[j] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o.q[j * 4 + i] = ubyte(lo, i);
        o.q[16 + j * 4 + i] = ubyte(hi, i);
      }
    }
  }
  // sum over the chunk of w * x, with x given in xidx order and xs = {sum lo, sum hi}
  __device__ __forceinline__ static float dot(const Dec &d, const float *x, const float *xs) {
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) a = fmaf(d.q[i], x[i], a);
#pragma unroll
    for (int i = 0; i < 16; ++i) b = fmaf(d.q[16 + i], x[16 + i], b);
    return (d.s_lo * a - d.m_lo * xs[0]) + (d.s_hi * b - d.m_hi * xs[1]);
  }
  static constexpr int NXS = 2;  // x partial sums needed per chunk
  __device__ __forceinline__ static void xsums(const float *x, float *xs) {
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) a += x[i];
#pragma unroll
    for (int i = 0; i < 16; ++i) b += x[16 + i];
    xs[0] = a;
    xs[1] = b;
  }
};

template <>
struct Fmt<NX_FMT_Q8_0> {
  static constexpr int XPC = 16;
  static constexpr int CHUNKS_PER_BLOCK = 2;
  static constexpr int META = 2;
  __device__ __forceinline__ static int xidx(int c, int v) { return c * 16 + v; }
  struct Dec {
    float q[16];
    float d;
  };
  __device__ __forceinline__ static void decode(const uint4 &w, const uint8_t *meta_row, int c,
                                                Dec &o) {
    const uint16_t dh = *reinterpret_cast<const uint16_t *>(meta_row + (c >> 1) * 2);
    o.d = h2f(dh);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) o.q[j * 4 + i] = sbyte(ws[j], i);
  }
  static constexpr int NXS = 1;
  __device__ __forceinline__ static void xsums(const float *, float *xs) { xs[0] = 0.f; }
  __device__ __forceinline__ static float dot(const Dec &d, const float *x, const float *) {
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) a = fmaf(d.q[i], x[i], a);
    return d.d * a;
  }
};

template <>
struct Fmt<NX_FMT_Q4_0> {
  static constexpr int XPC = 32;
  static constexpr int CHUNKS_PER_BLOCK = 1;
  static constexpr int META = 2;
  __device__ __forceinline__ static int xidx(int c, int v) { return c * 32 + v; }
  struct Dec {
    float q[32];
    float d;
  };
  __device__ __forceinline__ static void decode(const uint4 &w, const uint8_t *meta_row, int c,
                                                Dec &o) {
    const uint16_t dh = *reinterpret_cast<const uint16_t *>(meta_row + c * 2);
    o.d = h2f(dh);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t lo = ws[j] & 0x0F0F0F0Fu;
      const uint32_t hi = (ws[j] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o.q[j * 4 + i] = ubyte(lo, i);
        o.q[16 + j * 4 + i] = ubyte(hi, i);
      }
    }
  }
  static constexpr int NXS = 1;
  __device__ __forceinline__ static void xsums(const float *x, float *xs) {
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) a += x[i];
    xs[0] = a;
  }
  __device__ __forceinline__ static float dot(const Dec &d, const float *x, const float *xs) {
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) a = fmaf(d.q[i], x[i], a);
    return d.d * (a - 8.f * xs[0]);
  }
};

template <>
struct Fmt<NX_FMT_F32> {
  static constexpr int XPC = 4;
  static constexpr int CHUNKS_PER_BLOCK = 1;
  static constexpr int META = 0;
  __device__ __forceinline__ static int xidx(int c, int v) { return c * 4 + v; }
  struct Dec {
    float q[4];
  };
  __device__ __forceinline__ static void decode(const uint4 &w, const uint8_t *, int, Dec &o) {
    o.q[0] = __uint_as_float(w.x);
    o.q[1] = __uint_as_float(w.y);
    o.q[2] = __uint_as_float(w.z);
    o.q[3] = __uint_as_float(w.w);
  }
  static constexpr int NXS = 1;
  __device__ __forceinline__ static void xsums(const float *, float *xs) { xs[0] = 0.f; }
  __device__ __forceinline__ static float dot(const Dec &d, const float *x, const float *) {
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) a = fmaf(d.q[i], x[i], a);
    return a;
  }
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  return (g / (1.0f + expf(-g))) * u;
}

}  // namespace nx
