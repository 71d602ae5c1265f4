// nx_quant.hip — GGUF block formats on gfx950: bit-exact dequantization,
// a device restatement of the reference quantizer, and the repack of GGUF
// payloads into the resident split code/scale planes.
//
// Dequantization (src/gguf/mod.rs:962-1088 == src/quant/mod.rs:689-937):
// every decoded value is an exact product (Q8_0 q*d, Q4_0 (q-8)*d) or the
// single rounding of the difference of two exact products (Q4_K and Q2_K
// d*sc*q - dmin*m), so the device result is bit-identical to the reference
// whatever the contraction.  Quantization (src/quant/mod.rs:669-818) uses IEEE
// division, roundf (half away from zero), minNum/maxNum and hardware RNE f16
// conversion; contraction is switched off so each expression rounds as the
// Rust f32 expression does.
#include "nx_device.hpp"
#include "nx_internal.hpp"

namespace nx {

namespace {

__device__ __forceinline__ float ld_f16(const uint8_t *p) {
  return h2f((uint32_t)p[0] | ((uint32_t)p[1] << 8));
}

// ---------------------------------------------------------------- dequant
template <int FMT>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t *__restrict__ src, size_t n,
                                                 float *__restrict__ dst) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    float v;
    if constexpr (FMT == NX_FMT_F16) {  // src/gguf/mod.rs:921-933
      v = ld_f16(src + 2 * i);
    } else if constexpr (FMT == NX_FMT_BF16) {  // src/gguf/mod.rs:934-946
      v = __uint_as_float((uint32_t)(src[2 * i] | (src[2 * i + 1] << 8)) << 16);
    } else if constexpr (FMT == NX_FMT_Q8_0) {
      const uint8_t *b = src + (i / 32) * 34;
      v = (float)(int8_t)b[2 + i % 32] * ld_f16(b);
    } else if constexpr (FMT == NX_FMT_Q4_0) {
      const uint8_t *b = src + (i / 32) * 18;
      const int j = (int)(i % 32);
      const int q = j < 16 ? (b[2 + j] & 15) : (b[2 + j - 16] >> 4);
      v = (float)(q - 8) * ld_f16(b);
    } else if constexpr (FMT == NX_FMT_Q2_K) {  // src/quant/mod.rs:913-937
      const uint8_t *b = src + (i / 256) * 84;
      const int j = (int)(i % 256);
      const uint32_t q = (b[16 + j / 4] >> (2 * (j % 4))) & 3u;
      const uint32_t packed = b[j / 16];
      v = ld_f16(b + 80) * (float)(packed & 15u) * (float)q - ld_f16(b + 82) * (float)(packed >> 4);
    } else {  // Q4_K
      const uint8_t *b = src + (i / 256) * 144;
      const int j = (int)(i % 256);
      const int s = j / 32;
      const uint8_t *p = b + 4;
      uint32_t sc, mn;
      if (s < 4) {
        sc = p[s] & 63;
        mn = p[s + 4] & 63;
      } else {
        sc = (p[s + 4] & 15) | ((p[s - 4] >> 6) << 4);
        mn = (p[s + 4] >> 4) | ((p[s] >> 6) << 4);
      }
      const uint8_t packed = b[16 + (j & 127)];
      const uint32_t q = j < 128 ? (packed & 15u) : (packed >> 4);
      v = ld_f16(b) * (float)sc * (float)q - ld_f16(b + 2) * (float)mn;
    }
    dst[i] = v;
  }
}

// ---------------------------------------------------------------- quantize
#pragma clang fp contract(off)

__device__ __forceinline__ void st_f16(uint8_t *p, float v) {
  const uint16_t h = __builtin_bit_cast(uint16_t, (_Float16)v);
  p[0] = (uint8_t)(h & 0xFF);
  p[1] = (uint8_t)(h >> 8);
}
// Rust `as u8` / `as i8` after clamp: saturating, NaN -> 0.
__device__ __forceinline__ uint8_t sat_u8(float v) {
  if (!(v > 0.0f)) return 0;
  if (v >= 255.0f) return 255;
  return (uint8_t)v;
}
__device__ __forceinline__ int8_t sat_i8(float v) {
  if (v != v) return 0;
  if (v <= -128.0f) return -128;
  if (v >= 127.0f) return 127;
  return (int8_t)v;
}
__device__ __forceinline__ float clampf(float v, float lo, float hi) {
  if (v < lo) v = lo;
  if (v > hi) v = hi;
  return v;
}

// one thread per 32-element block (src/quant/mod.rs:669-687, 705-721, 747-754)
template <int FMT>
__global__ __launch_bounds__(256) void k_quant32(const float *__restrict__ src, size_t n,
                                                 uint8_t *__restrict__ dst) {
  const size_t nb = (n + 31) / 32;
  for (size_t b = blockIdx.x * (size_t)blockDim.x + threadIdx.x; b < nb;
       b += (size_t)gridDim.x * blockDim.x) {
    const size_t base = b * 32;
    const int len = (int)(n - base < 32 ? n - base : 32);
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = i < len ? src[base + i] : 0.0f;
    float max_abs = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i)
      if (i < len) max_abs = fmaxf(max_abs, fabsf(v[i]));
    if constexpr (FMT == NX_FMT_Q8_0) {
      uint8_t *o = dst + b * 34;
      const float scale = max_abs > 0.0f ? max_abs / 127.0f : 0.0f;
      st_f16(o, scale);
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        int8_t q = 0;
        if (scale > 0.0f) q = sat_i8(clampf(roundf(v[i] / scale), -128.0f, 127.0f));
        o[2 + i] = (uint8_t)q;
      }
    } else {
      uint8_t *o = dst + b * 18;
      const float scale = max_abs > 0.0f ? max_abs / 7.0f : 0.0f;
      st_f16(o, scale);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        uint8_t lo = 8, hi = 8;
        if (scale > 0.0f) {
          const float ql = clampf(roundf(v[i] / scale), -8.0f, 7.0f);
          const float qh = clampf(roundf(v[i + 16] / scale), -8.0f, 7.0f);
          lo = (uint8_t)((ql != ql ? 0 : (int)ql) + 8);
          hi = (uint8_t)((qh != qh ? 0 : (int)qh) + 8);
        }
        o[2 + i] = (uint8_t)((lo & 15) | ((hi & 15) << 4));
      }
    }
  }
}

__device__ __forceinline__ uint8_t quantize_u6(float value, float scale) {
  if (scale > 0.0f && value > 0.0f) return sat_u8(clampf(roundf(value / scale), 1.0f, 63.0f));
  return 0;
}
__device__ __forceinline__ uint8_t q4k_value(float value, float d, float dmin, uint32_t sq,
                                             uint32_t mq) {
  const float scale = d * (float)sq;
  const float offset = dmin * (float)mq;
  if (scale > 0.0f) return sat_u8(clampf(roundf((value + offset) / scale), 0.0f, 15.0f));
  return 0;
}

// Q4_K (src/quant/mod.rs:756-818): eight lanes per 256-element block; lane j
// owns sub-block j for the statistics, lanes 0..3 then write the 32 code
// bytes holding sub-blocks j (low nibbles) and j+4 (high nibbles).
__global__ __launch_bounds__(256) void k_quant_q4k(const float *__restrict__ src, size_t n,
                                                   uint8_t *__restrict__ dst) {
  const size_t nb = (n + 255) / 256;
  const int j = threadIdx.x & 7;
  const int lane = threadIdx.x & 63;
  // each wave owns 8 consecutive blocks per step; the loop bound is uniform
  // across the wave so the shuffles below always see all eight lanes of a block
  const size_t wave_id = blockIdx.x * (size_t)(blockDim.x / 64) + (threadIdx.x >> 6);
  const size_t wave_stride = (size_t)gridDim.x * (blockDim.x / 64) * 8;
  for (size_t wb = wave_id * 8; wb < nb; wb += wave_stride) {
    const size_t b = wb + (size_t)(lane >> 3);
    const bool live = b < nb;
    const size_t base = b * 256;
    auto val = [&](int i) -> float {
      const size_t idx = base + (size_t)i;
      return (live && idx < n) ? src[idx] : 0.0f;
    };
    float mn = INFINITY, mx = -INFINITY;
    for (int i = 0; i < 32; ++i) mn = fminf(mn, val(j * 32 + i));
    for (int i = 0; i < 32; ++i) mx = fmaxf(mx, val(j * 32 + i));
    const float offset = mn < 0.0f ? -mn : 0.0f;
    const float scale = fmaxf((mx + offset) / 15.0f, 0.0f);
    // neither value can be NaN, so the fold order of max does not matter
    float max_scale = scale, max_offset = offset;
#pragma unroll
    for (int m = 1; m < 8; m <<= 1) {
      max_scale = fmaxf(max_scale, __shfl_xor(max_scale, m, 64));
      max_offset = fmaxf(max_offset, __shfl_xor(max_offset, m, 64));
    }
    max_scale = fmaxf(0.0f, max_scale);
    max_offset = fmaxf(0.0f, max_offset);
    const float d = max_scale > 0.0f ? max_scale / 63.0f : 0.0f;
    const float dmin = max_offset > 0.0f ? max_offset / 63.0f : 0.0f;
    const uint32_t sq = quantize_u6(scale, d);
    const uint32_t mq = quantize_u6(offset, dmin);
    // gather the eight (scale, min) codes of the block into every lane
    uint32_t sc[8], mi[8];
    const int lane0 = lane & ~7;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      sc[s] = __shfl(sq, lane0 + s, 64);
      mi[s] = __shfl(mq, lane0 + s, 64);
    }
    if (live) {
      uint8_t *o = dst + b * 144;
      if (j == 0) {
        st_f16(o, d);
        st_f16(o + 2, dmin);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          o[4 + i] = (uint8_t)((sc[i] & 0x3F) | ((sc[i + 4] >> 4) << 6));
          o[8 + i] = (uint8_t)((mi[i] & 0x3F) | ((mi[i + 4] >> 4) << 6));
          o[12 + i] = (uint8_t)((sc[i + 4] & 0x0F) | ((mi[i + 4] & 0x0F) << 4));
        }
      }
      if (j < 4) {
        for (int i = 0; i < 32; ++i) {
          const int e = j * 32 + i;
          const uint8_t lo = q4k_value(val(e), d, dmin, sc[j], mi[j]);
          const uint8_t hi = q4k_value(val(e + 128), d, dmin, sc[j + 4], mi[j + 4]);
          o[16 + e] = (uint8_t)((lo & 0x0F) | ((hi & 0x0F) << 4));
        }
      }
    }
  }
}

__device__ __forceinline__ uint8_t quantize_u4(float value, float scale) {
  if (scale > 0.0f && value > 0.0f) return sat_u8(clampf(roundf(value / scale), 1.0f, 15.0f));
  return 0;
}
__device__ __forceinline__ uint8_t q2k_value(float value, float d, float dmin, uint32_t sq,
                                             uint32_t mq) {
  const float scale = d * (float)sq;
  const float offset = dmin * (float)mq;
  if (scale > 0.0f) return sat_u8(clampf(roundf((value + offset) / scale), 0.0f, 3.0f));
  return 0;
}

// Q2_K (src/quant/mod.rs:851-911): sixteen lanes per 256-element block; lane
// u owns sub-block u (16 values): its statistics, its scale/min byte and the
// four code bytes of its values.
__global__ __launch_bounds__(256) void k_quant_q2k(const float *__restrict__ src, size_t n,
                                                   uint8_t *__restrict__ dst) {
  const size_t nb = (n + 255) / 256;
  const int u = threadIdx.x & 15;
  const int lane = threadIdx.x & 63;
  // each wave owns 4 consecutive blocks per step; the loop bound is uniform
  // across the wave so the shuffles below always see all sixteen lanes
  const size_t wave_id = blockIdx.x * (size_t)(blockDim.x / 64) + (threadIdx.x >> 6);
  const size_t wave_stride = (size_t)gridDim.x * (blockDim.x / 64) * 4;
  for (size_t wb = wave_id * 4; wb < nb; wb += wave_stride) {
    const size_t b = wb + (size_t)(lane >> 4);
    const bool live = b < nb;
    const size_t base = b * 256;
    auto val = [&](int i) -> float {
      const size_t idx = base + (size_t)i;
      return (live && idx < n) ? src[idx] : 0.0f;
    };
    float mn = INFINITY, mx = -INFINITY;
    for (int i = 0; i < 16; ++i) mn = fminf(mn, val(u * 16 + i));
    for (int i = 0; i < 16; ++i) mx = fmaxf(mx, val(u * 16 + i));
    const float offset = mn < 0.0f ? -mn : 0.0f;
    const float scale = fmaxf((mx + offset) / 3.0f, 0.0f);
    // neither value can be NaN, so the fold order of max does not matter
    float max_scale = scale, max_offset = offset;
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) {
      max_scale = fmaxf(max_scale, __shfl_xor(max_scale, m, 64));
      max_offset = fmaxf(max_offset, __shfl_xor(max_offset, m, 64));
    }
    max_scale = fmaxf(0.0f, max_scale);
    max_offset = fmaxf(0.0f, max_offset);
    const float d = max_scale > 0.0f ? max_scale / 15.0f : 0.0f;
    const float dmin = max_offset > 0.0f ? max_offset / 15.0f : 0.0f;
    const uint32_t sq = quantize_u4(scale, d) & 15u;
    const uint32_t mq = quantize_u4(offset, dmin) & 15u;
    if (live) {
      uint8_t *o = dst + b * 84;
      o[u] = (uint8_t)(sq | (mq << 4));
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        uint32_t byte = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          byte |= (uint32_t)(q2k_value(val(u * 16 + 4 * k + i), d, dmin, sq, mq) & 3u) << (2 * i);
        o[16 + 4 * u + k] = (uint8_t)byte;
      }
      if (u == 0) {
        st_f16(o + 80, d);
        st_f16(o + 82, dmin);
      }
    }
  }
}

#pragma clang fp contract(on)

// ---------------------------------------------------------------- repack
// GGUF row-major blocks -> resident planes (nx_device.hpp): the code plane is
// written as 16-byte halves of 32-byte segments at their half-interleaved
// offsets within the panels of 64 segments, the scale plane as {d, dmin,
// scales12} (Q4_K) or d (Q8_0, Q4_0) in the same panels.  One thread per
// 16-byte code half; byte copies because GGUF blocks are not 4-byte aligned.
template <int FMT>
__global__ __launch_bounds__(256) void k_repack_codes(const uint8_t *__restrict__ src, int rows,
                                                      int cols, int nseg,
                                                      uint8_t *__restrict__ qs) {
  const size_t total = (size_t)rows * nseg * 2;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const int h = (int)(i & 1);
    const size_t rj = i >> 1;
    const int r = (int)(rj / nseg), j = (int)(rj - (size_t)r * nseg);
    uint8_t *dst = qs + code_off(r, j, h, rows, nseg);
    if constexpr (FMT == NX_FMT_F32) {
      const float *sf = reinterpret_cast<const float *>(src) + (size_t)r * cols;
      float *df = reinterpret_cast<float *>(dst);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int c = 8 * j + 4 * h + v;
        df[v] = c < cols ? sf[c] : 0.0f;
      }
    } else if constexpr (FMT == NX_FMT_F16 || FMT == NX_FMT_BF16) {
      // segment j = values 16 j .. 16 j + 15 of the row, half h the 8 from 16 j + 8 h
      const uint16_t *sh = reinterpret_cast<const uint16_t *>(src) + (size_t)r * cols;
      uint16_t *dh = reinterpret_cast<uint16_t *>(dst);
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const int c = 16 * j + 8 * h + v;
        dh[v] = c < cols ? sh[c] : (uint16_t)0;
      }
    } else if constexpr (FMT == NX_FMT_Q8_0) {
      const int nb = cols / 32;
      const uint8_t *b = src + ((size_t)r * nb + j) * 34 + 2 + h * 16;
#pragma unroll
      for (int v = 0; v < 16; ++v) dst[v] = b[v];
    } else {
      // the 32 codes of one sub-block in element order ...
      uint8_t q[32];
      if constexpr (FMT == NX_FMT_Q4_K) {
        // qs byte 32s + i: element 32s + i (low nibble), 128 + 32s + i (high)
        const int nb = cols / 256;
        const uint8_t *b = src + ((size_t)r * nb + (j >> 2)) * 144 + 16 + (j & 3) * 32;
#pragma unroll
        for (int i = 0; i < 32; ++i) q[i] = h ? (b[i] >> 4) : (b[i] & 15);
      } else {  // Q4_0: segment j = blocks 2j, 2j+1; byte i: element i (low), 16 + i (high)
        const int nb = cols / 32;
        const int blk = 2 * j + h;
        const uint8_t *b = blk < nb ? src + ((size_t)r * nb + blk) * 18 + 2 : nullptr;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          q[i] = b ? (b[i] & 15) : 0;
          q[16 + i] = b ? (b[i] >> 4) : 0;
        }
      }
      // ... stored as signed nibbles q ^ 8 = q - 8: byte 4k+i = element 8k+i
      // (low) | element 8k+4+i (high)
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          dst[4 * k + i] = (uint8_t)(((q[8 * k + i] ^ 8) | ((q[8 * k + 4 + i] ^ 8) << 4)) & 0xFF);
    }
  }
}

template <int FMT>
__global__ __launch_bounds__(256) void k_repack_meta(const uint8_t *__restrict__ src, int rows,
                                                     int cols, int nseg,
                                                     uint8_t *__restrict__ meta) {
  constexpr int BLK = FMT == NX_FMT_Q4_K ? 256 : 32;
  constexpr int BB = FMT == NX_FMT_Q4_K ? 144 : (FMT == NX_FMT_Q8_0 ? 34 : 18);
  constexpr int MB = FMT == NX_FMT_Q4_K ? 16 : 2;
  // scale bytes per segment, and blocks per panel of 64 segments
  constexpr int MU = Seg<FMT>::MU, BPP = MU > 0 ? 64 * MU / MB : 1;
  const int nb = cols / BLK;
  // Q4_0 rows are padded to an even block count (two blocks per segment)
  const int slots = FMT == NX_FMT_Q4_0 ? 2 * nseg : nb;
  const size_t total = (size_t)rows * slots;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const int r = (int)(i / slots), b = (int)(i - (size_t)r * slots);
    uint8_t *dst = meta + panel_row_off(r, b / BPP, rows, nseg, MU) + (uint32_t)(b % BPP) * MB;
    const uint8_t *s = b < nb ? src + ((size_t)r * nb + b) * BB : nullptr;
#pragma unroll
    for (int v = 0; v < MB; ++v) dst[v] = s ? s[v] : (uint8_t)0;
  }
}

// Q2_K code plane: one thread per 64-element segment j (block j/4, elements
// 64(j%4) ..), its 16 bytes at 16 (j % 64) in its panel row (16 bytes per
// segment).  Element e of a block sits in bits
// 2(e%4) of qs byte e/4; resident byte 4k+i holds, from bit 0, the codes of
// elements 8k+i and 32+8k+i, then 8k+4+i and 32+8k+4+i of the segment (the
// 4-bit dword order of each half, the halves two bits apart).
__global__ __launch_bounds__(256) void k_repack_codes_q2k(const uint8_t *__restrict__ src, int rows,
                                                          int cols, int nseg,
                                                          uint8_t *__restrict__ qs) {
  const int nb = cols / 256;
  const size_t total = (size_t)rows * nseg;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const int r = (int)(i / nseg), j = (int)(i - (size_t)r * nseg);
    const uint8_t *b = src + ((size_t)r * nb + (j >> 2)) * 84 + 16;
    const int e0 = (j & 3) * 64;
    auto code = [&](int e) { return (uint32_t)(b[(e0 + e) >> 2] >> (2 * ((e0 + e) & 3))) & 3u; };
    uint8_t *dst = qs + panel_row_off(r, j >> 6, rows, nseg, 16) + (uint32_t)(j & 63) * 16;
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        dst[4 * k + c] = (uint8_t)(code(8 * k + c) | (code(32 + 8 * k + c) << 2) |
                                   (code(8 * k + 4 + c) << 4) | (code(32 + 8 * k + 4 + c) << 6));
  }
}

// Q2_K scale plane: per segment j (block j/4, sub-blocks 4(j%4) ..) the
// eight bytes {d, dmin, four scale/min bytes}
__global__ __launch_bounds__(256) void k_repack_meta_q2k(const uint8_t *__restrict__ src, int rows,
                                                         int cols, int nseg,
                                                         uint8_t *__restrict__ meta) {
  const int nb = cols / 256;
  const size_t total = (size_t)rows * nseg;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const int r = (int)(i / nseg), j = (int)(i - (size_t)r * nseg);
    uint8_t *dst = meta + panel_row_off(r, j >> 6, rows, nseg, 8) + (uint32_t)(j & 63) * 8;
    const uint8_t *b = src + ((size_t)r * nb + (j >> 2)) * 84;
#pragma unroll
    for (int v = 0; v < 4; ++v) dst[v] = b[80 + v];
#pragma unroll
    for (int v = 0; v < 4; ++v) dst[4 + v] = b[(j & 3) * 4 + v];
  }
}

unsigned grid_for(size_t items, unsigned per_block) {
  size_t g = (items + per_block - 1) / per_block;
  if (g < 1) g = 1;
  if (g > 65535u * 16u) g = 65535u * 16u;
  return (unsigned)g;
}

}  // namespace

int launch_dequant(nx_ctx *c, int fmt, const void *d_src, size_t n, float *d_dst) {
  if (n == 0) return NX_OK;
  const uint8_t *s = static_cast<const uint8_t *>(d_src);
  const unsigned g = grid_for(n, 256);
  switch (fmt) {
  case NX_FMT_Q8_0:
    return launch(c, "dequant_q8_0", [&] { k_dequant<NX_FMT_Q8_0><<<g, 256, 0, c->stream>>>(s, n, d_dst); });
  case NX_FMT_Q4_0:
    return launch(c, "dequant_q4_0", [&] { k_dequant<NX_FMT_Q4_0><<<g, 256, 0, c->stream>>>(s, n, d_dst); });
  case NX_FMT_Q4_K:
    return launch(c, "dequant_q4_k", [&] { k_dequant<NX_FMT_Q4_K><<<g, 256, 0, c->stream>>>(s, n, d_dst); });
  case NX_FMT_Q2_K:
    return launch(c, "dequant_q2_k", [&] { k_dequant<NX_FMT_Q2_K><<<g, 256, 0, c->stream>>>(s, n, d_dst); });
  case NX_FMT_F16:
    return launch(c, "dequant_f16", [&] { k_dequant<NX_FMT_F16><<<g, 256, 0, c->stream>>>(s, n, d_dst); });
  case NX_FMT_BF16:
    return launch(c, "dequant_bf16", [&] { k_dequant<NX_FMT_BF16><<<g, 256, 0, c->stream>>>(s, n, d_dst); });
  case NX_FMT_F32:
    NX_HIP(hipMemcpyAsync(d_dst, d_src, n * 4, hipMemcpyDeviceToDevice, c->stream));
    return NX_OK;
  }
  return fail(NX_ERR_INVALID_ARG, "unknown weight format " + std::to_string(fmt));
}

int launch_quantize(nx_ctx *c, int fmt, const float *d_src, size_t n, void *d_dst) {
  if (n == 0) return NX_OK;
  uint8_t *d = static_cast<uint8_t *>(d_dst);
  switch (fmt) {
  case NX_FMT_Q8_0: {
    const unsigned g = grid_for((n + 31) / 32, 256);
    return launch(c, "quantize_q8_0", [&] { k_quant32<NX_FMT_Q8_0><<<g, 256, 0, c->stream>>>(d_src, n, d); });
  }
  case NX_FMT_Q4_0: {
    const unsigned g = grid_for((n + 31) / 32, 256);
    return launch(c, "quantize_q4_0", [&] { k_quant32<NX_FMT_Q4_0><<<g, 256, 0, c->stream>>>(d_src, n, d); });
  }
  case NX_FMT_Q4_K: {
    const unsigned g = grid_for((n + 255) / 256, 32);
    return launch(c, "quantize_q4_k", [&] { k_quant_q4k<<<g, 256, 0, c->stream>>>(d_src, n, d); });
  }
  case NX_FMT_Q2_K: {
    const unsigned g = grid_for((n + 255) / 256, 16);
    return launch(c, "quantize_q2_k", [&] { k_quant_q2k<<<g, 256, 0, c->stream>>>(d_src, n, d); });
  }
  case NX_FMT_F32:
    NX_HIP(hipMemcpyAsync(d_dst, d_src, n * 4, hipMemcpyDeviceToDevice, c->stream));
    return NX_OK;
  }
  return fail(NX_ERR_INVALID_ARG, "unknown weight format " + std::to_string(fmt));
}

int launch_repack(nx_ctx *c, int fmt, const void *d_src, const RolePlane &pl, uint8_t *qs,
                  uint8_t *meta) {
  const uint8_t *s = static_cast<const uint8_t *>(d_src);
  const unsigned gc = grid_for((size_t)pl.rows * pl.nseg * 2, 256);
  const unsigned gm = grid_for((size_t)pl.rows * (size_t)(pl.row_meta ? pl.row_meta : 1), 256);
#define NX_RP(F, NAME)                                                                          \
  do {                                                                                          \
    NX_TRY(launch(c, NAME, [&] {                                                                \
      k_repack_codes<F><<<gc, 256, 0, c->stream>>>(s, pl.rows, pl.cols, pl.nseg, qs); \
    }));                                                                                        \
    if (F != NX_FMT_F32 && F != NX_FMT_F16 && F != NX_FMT_BF16)                                \
      NX_TRY(launch(c, NAME, [&] {                                                              \
        k_repack_meta<F><<<gm, 256, 0, c->stream>>>(s, pl.rows, pl.cols, pl.nseg, \
                                                    meta);                                      \
      }));                                                                                      \
    return NX_OK;                                                                               \
  } while (0)
  switch (fmt) {
  case NX_FMT_Q4_K: NX_RP(NX_FMT_Q4_K, "repack_q4_k");
  case NX_FMT_Q8_0: NX_RP(NX_FMT_Q8_0, "repack_q8_0");
  case NX_FMT_Q4_0: NX_RP(NX_FMT_Q4_0, "repack_q4_0");
  case NX_FMT_F32: NX_RP(NX_FMT_F32, "repack_f32");
  case NX_FMT_F16: NX_RP(NX_FMT_F16, "repack_f16");
  case NX_FMT_BF16: NX_RP(NX_FMT_BF16, "repack_bf16");
  case NX_FMT_Q2_K: {
    const unsigned g2 = grid_for((size_t)pl.rows * pl.nseg, 256);
    NX_TRY(launch(c, "repack_q2_k", [&] {
      k_repack_codes_q2k<<<g2, 256, 0, c->stream>>>(s, pl.rows, pl.cols, pl.nseg, qs);
    }));
    return launch(c, "repack_q2_k", [&] {
      k_repack_meta_q2k<<<g2, 256, 0, c->stream>>>(s, pl.rows, pl.cols, pl.nseg, meta);
    });
  }
  }
#undef NX_RP
  return fail(NX_ERR_INVALID_ARG, "unknown weight format");
}

}  // namespace nx
