/*
 * nx_oracle.c — CPU restatement of the Nexus MoE routed-FFN path.
 *
 * TEST INFRASTRUCTURE ONLY (the test oracle).  It is never linked into or called
 * by the product library; only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load it.
 *
 * Build: -O2 -ffp-contract=off, no fast-math (oracle/Makefile).  x86-64 float
 * arithmetic is SSE single precision, so each C expression below rounds the
 * way the corresponding Rust f32 expression does.  Rust `f32::exp` is glibc
 * expf, `f32::round` is roundf, `f32::max/min` are fmaxf/fminf and `as u8/i8`
 * is a saturating cast with NaN -> 0 (restated explicitly where it matters).
 *
 * Pinning (see tests/test_oracle_*.py): the Q8_0 known-answer test of
 * src/gguf/mod.rs:1681-1695, the round-trip tolerances of
 * src/quant/mod.rs:1287-1325, the router test of src/engine/mod.rs:1622-1630,
 * the closed form of the dispatch test src/engine/mod.rs:1632-1656, the matmul
 * known answer of src/backend/cpu.rs:234-241, numpy float16 for the f16
 * conversions, brute-force enumeration for the dequantizers and router, and
 * independent numpy restatements for the layer.  The permutation and the
 * sigmoid score mode have no reference counterpart: they are pinned by
 * brute force and invariants only (no reference vector exists for them).
 */
#include "nx_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define GGUF_F32 0
#define GGUF_Q4_0 2
#define GGUF_Q8_0 8
#define GGUF_Q4_K 12
#define GGUF_Q2_K 10
#define GGUF_F16 1
#define GGUF_BF16 28 /* the reference's id (src/gguf/mod.rs:135) */

/* ------------------------------------------------------------------------ */
/* parallel-for helper                                                       */
/* ------------------------------------------------------------------------ */
typedef void (*range_fn)(void *ctx, size_t lo, size_t hi);
typedef struct {
    range_fn fn;
    void *ctx;
    size_t lo, hi;
} range_job;

static void *range_thread(void *p) {
    range_job *j = (range_job *)p;
    j->fn(j->ctx, j->lo, j->hi);
    return NULL;
}

static void parallel_for(size_t n, int nthreads, range_fn fn, void *ctx) {
    if (nthreads <= 1 || n < 2) {
        fn(ctx, 0, n);
        return;
    }
    if ((size_t)nthreads > n) nthreads = (int)n;
    if (nthreads > 256) nthreads = 256;
    pthread_t th[256];
    range_job jobs[256];
    size_t per = (n + (size_t)nthreads - 1) / (size_t)nthreads;
    int started = 0;
    for (int i = 0; i < nthreads; ++i) {
        size_t lo = (size_t)i * per, hi = lo + per;
        if (lo >= n) break;
        if (hi > n) hi = n;
        jobs[i].fn = fn;
        jobs[i].ctx = ctx;
        jobs[i].lo = lo;
        jobs[i].hi = hi;
        if (pthread_create(&th[i], NULL, range_thread, &jobs[i]) != 0) {
            fn(ctx, lo, hi); /* run inline if a thread cannot start */
            jobs[i].fn = NULL;
        }
        started = i + 1;
    }
    for (int i = 0; i < started; ++i)
        if (jobs[i].fn) pthread_join(th[i], NULL);
}

/* ------------------------------------------------------------------------ */
/* f16 <-> f32 (half 2.x semantics)                                          */
/* ------------------------------------------------------------------------ */
static inline uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static inline float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

float nxo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0x1F) return u2f(sign | 0x7F800000u | (m << 13)); /* inf / nan */
    if (e == 0) {
        /* zero or subnormal: value = m * 2^-24, exact in f32 */
        float v = (float)m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t nxo_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) {               /* inf or nan */
        if (ax == 0x7F800000u) return sign | 0x7C00u;
        return sign | 0x7E00u | (uint16_t)((ax & 0x7FFFFFu) >> 13); /* quiet nan */
    }
    int exp = (int)(ax >> 23) - 127;       /* unbiased f32 exponent */
    if (exp > 15) return sign | 0x7C00u;   /* |f| >= 2^16 -> inf */
    uint32_t mant = (ax & 0x7FFFFFu) | (ax >= 0x00800000u ? 0x800000u : 0u);
    int shift;                             /* right shift taking the 24-bit significand to f16 units */
    uint32_t base;
    if (exp >= -14) {                      /* normal f16 range: keep 11 bits */
        shift = 13;
        base = (uint32_t)(exp + 15) << 10;
        mant &= 0x7FFFFFu;                 /* implicit bit carried by base */
    } else {                               /* subnormal f16: unit is 2^-24 */
        shift = -exp - 14 + 13;            /* value = mant * 2^(exp-23); units of 2^-24 */
        base = 0;
        if (shift > 31) return sign;       /* far below half of the smallest subnormal */
    }
    uint32_t q = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q += 1u; /* nearest, ties to even */
    /* a carry out of the significand moves into the exponent field, which is
     * exactly the next binade (or inf from 65520 upward) */
    return (uint16_t)(sign | (base + q));
}

void nxo_f32_to_f16_array(const float *src, size_t n, uint16_t *dst) {
    for (size_t i = 0; i < n; ++i) dst[i] = nxo_f32_to_f16(src[i]);
}

static inline float rd_f16(const uint8_t *p) {
    return nxo_f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
}
static inline void wr_f16(uint8_t *p, float v) {
    uint16_t h = nxo_f32_to_f16(v);
    p[0] = (uint8_t)(h & 0xFF);
    p[1] = (uint8_t)(h >> 8);
}

/* Rust `x as u8` / `x as i8` after clamp: saturating, NaN -> 0. */
static inline uint8_t sat_u8(float v) {
    if (v != v) return 0;
    if (v <= 0.0f) return 0;
    if (v >= 255.0f) return 255;
    return (uint8_t)v;
}
static inline int8_t sat_i8(float v) {
    if (v != v) return 0;
    if (v <= -128.0f) return -128;
    if (v >= 127.0f) return 127;
    return (int8_t)v;
}
/* f32::clamp: NaN stays NaN. */
static inline float clampf(float v, float lo, float hi) {
    if (v < lo) v = lo;
    if (v > hi) v = hi;
    return v;
}

/* ------------------------------------------------------------------------ */
/* quantizers / dequantizers                                                 */
/* ------------------------------------------------------------------------ */
size_t nxo_quant_bytes(int t, size_t n) {
    switch (t) {
    case GGUF_F32: return n * 4;
    case GGUF_Q4_0: return (n + 31) / 32 * 18; /* src/gguf/mod.rs:262-264 */
    case GGUF_Q8_0: return (n + 31) / 32 * 34; /* src/gguf/mod.rs:268 */
    case GGUF_Q4_K: return (n + 255) / 256 * 144; /* src/gguf/mod.rs:272 */
    case GGUF_Q2_K: return (n + 255) / 256 * 84;  /* src/gguf/mod.rs:270 */
    case GGUF_F16:
    case GGUF_BF16: return n * 2; /* src/gguf/mod.rs:249-293 */
    default: return 0;
    }
}

/* src/quant/mod.rs:669-687 */
static void q8_0_block(const float *chunk, size_t len, uint8_t *out) {
    float max_abs = 0.0f;
    for (size_t i = 0; i < len; ++i) max_abs = fmaxf(max_abs, fabsf(chunk[i]));
    float scale = max_abs > 0.0f ? max_abs / 127.0f : 0.0f;
    wr_f16(out, scale);
    for (size_t i = 0; i < 32; ++i) {
        float value = i < len ? chunk[i] : 0.0f;
        int8_t q = 0;
        if (scale > 0.0f) q = sat_i8(clampf(roundf(value / scale), -128.0f, 127.0f));
        out[2 + i] = (uint8_t)q;
    }
}

/* src/quant/mod.rs:747-754 */
static uint8_t q4_sym(float value, float scale) {
    if (scale > 0.0f) {
        float q = clampf(roundf(value / scale), -8.0f, 7.0f);
        int32_t qi = (q != q) ? 0 : (int32_t)q;
        return (uint8_t)(qi + 8);
    }
    return 8;
}

/* src/quant/mod.rs:705-721 */
static void q4_0_block(const float *chunk, size_t len, uint8_t *out) {
    float max_abs = 0.0f;
    for (size_t i = 0; i < len; ++i) max_abs = fmaxf(max_abs, fabsf(chunk[i]));
    float scale = max_abs > 0.0f ? max_abs / 7.0f : 0.0f;
    wr_f16(out, scale);
    for (size_t i = 0; i < 16; ++i) {
        uint8_t lo = q4_sym(i < len ? chunk[i] : 0.0f, scale);
        uint8_t hi = q4_sym(i + 16 < len ? chunk[i + 16] : 0.0f, scale);
        out[2 + i] = (uint8_t)((lo & 0x0F) | ((hi & 0x0F) << 4));
    }
}

/* src/quant/mod.rs:1117-1123 */
static uint8_t quantize_u6(float value, float scale) {
    if (scale > 0.0f && value > 0.0f) return sat_u8(clampf(roundf(value / scale), 1.0f, 63.0f));
    return 0;
}

/* src/quant/mod.rs:1133-1141 */
static uint8_t q4k_value(float value, float d, float dmin, uint8_t scale_q, uint8_t min_q) {
    float scale = d * (float)scale_q;
    float offset = dmin * (float)min_q;
    if (scale > 0.0f) return sat_u8(clampf(roundf((value + offset) / scale), 0.0f, 15.0f));
    return 0;
}

/* src/quant/mod.rs:1153-1161 */
void nxo_pack_q4k_scales(const uint8_t *scales, const uint8_t *mins, uint8_t *out) {
    for (int i = 0; i < 4; ++i) {
        out[i] = (uint8_t)((scales[i] & 0x3F) | ((scales[i + 4] >> 4) << 6));
        out[i + 4] = (uint8_t)((mins[i] & 0x3F) | ((mins[i + 4] >> 4) << 6));
        out[i + 8] = (uint8_t)((scales[i + 4] & 0x0F) | ((mins[i + 4] & 0x0F) << 4));
    }
}

/* src/quant/mod.rs:1163-1170 (== src/gguf/mod.rs:1547-1554) */
void nxo_unpack_q4k_scales(const uint8_t *p, uint8_t *scales, uint8_t *mins) {
    for (int i = 0; i < 4; ++i) {
        scales[i] = p[i] & 0x3F;
        mins[i] = p[i + 4] & 0x3F;
        scales[i + 4] = (uint8_t)((p[i + 8] & 0x0F) | ((p[i] >> 6) << 4));
        mins[i + 4] = (uint8_t)((p[i + 8] >> 4) | ((p[i + 4] >> 6) << 4));
    }
}

/* src/quant/mod.rs:756-818 */
static void q4_k_block(const float *chunk, size_t len, uint8_t *out) {
    float block[256];
    for (size_t i = 0; i < 256; ++i) block[i] = i < len ? chunk[i] : 0.0f;
    float sub_scales[8], sub_offsets[8];
    for (int sub = 0; sub < 8; ++sub) {
        const float *v = block + sub * 32;
        float mn = INFINITY, mx = -INFINITY;
        for (int i = 0; i < 32; ++i) mn = fminf(mn, v[i]);
        for (int i = 0; i < 32; ++i) mx = fmaxf(mx, v[i]);
        float offset = mn < 0.0f ? -mn : 0.0f;
        float scale = fmaxf((mx + offset) / 15.0f, 0.0f);
        sub_scales[sub] = scale;
        sub_offsets[sub] = offset;
    }
    float max_scale = 0.0f, max_offset = 0.0f;
    for (int s = 0; s < 8; ++s) max_scale = fmaxf(max_scale, sub_scales[s]);
    for (int s = 0; s < 8; ++s) max_offset = fmaxf(max_offset, sub_offsets[s]);
    float d = max_scale > 0.0f ? max_scale / 63.0f : 0.0f;
    float dmin = max_offset > 0.0f ? max_offset / 63.0f : 0.0f;
    uint8_t scales[8], mins[8];
    for (int s = 0; s < 8; ++s) {
        scales[s] = quantize_u6(sub_scales[s], d);
        mins[s] = quantize_u6(sub_offsets[s], dmin);
    }
    wr_f16(out, d);
    wr_f16(out + 2, dmin);
    nxo_pack_q4k_scales(scales, mins, out + 4);
    uint8_t *qs = out + 16;
    for (int i = 0; i < 128; ++i) {
        uint8_t lo = q4k_value(block[i], d, dmin, scales[i / 32], mins[i / 32]);
        uint8_t hi = q4k_value(block[i + 128], d, dmin, scales[(i + 128) / 32], mins[(i + 128) / 32]);
        qs[i] = (uint8_t)((lo & 0x0F) | ((hi & 0x0F) << 4));
    }
}

/* src/quant/mod.rs:1125-1131 */
static uint8_t quantize_u4(float value, float scale) {
    if (scale > 0.0f && value > 0.0f) return sat_u8(clampf(roundf(value / scale), 1.0f, 15.0f));
    return 0;
}

/* src/quant/mod.rs:1143-1151 */
static uint8_t q2k_value(float value, float d, float dmin, uint8_t scale_q, uint8_t min_q) {
    float scale = d * (float)scale_q;
    float offset = dmin * (float)min_q;
    if (scale > 0.0f) return sat_u8(clampf(roundf((value + offset) / scale), 0.0f, 3.0f));
    return 0;
}

/* src/quant/mod.rs:851-911: 16 sub-blocks of 16; scales[16] (scale | min << 4),
 * qs[64] (element i in bits 2(i%4) of byte i/4), then f16 d and dmin */
static void q2_k_block(const float *chunk, size_t len, uint8_t *out) {
    float block[256];
    for (size_t i = 0; i < 256; ++i) block[i] = i < len ? chunk[i] : 0.0f;
    float sub_scales[16], sub_offsets[16];
    for (int sub = 0; sub < 16; ++sub) {
        const float *v = block + sub * 16;
        float mn = INFINITY, mx = -INFINITY;
        for (int i = 0; i < 16; ++i) mn = fminf(mn, v[i]);
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, v[i]);
        float offset = mn < 0.0f ? -mn : 0.0f;
        float scale = fmaxf((mx + offset) / 3.0f, 0.0f);
        sub_scales[sub] = scale;
        sub_offsets[sub] = offset;
    }
    float max_scale = 0.0f, max_offset = 0.0f;
    for (int s = 0; s < 16; ++s) max_scale = fmaxf(max_scale, sub_scales[s]);
    for (int s = 0; s < 16; ++s) max_offset = fmaxf(max_offset, sub_offsets[s]);
    float d = max_scale > 0.0f ? max_scale / 15.0f : 0.0f;
    float dmin = max_offset > 0.0f ? max_offset / 15.0f : 0.0f;
    for (int s = 0; s < 16; ++s) {
        uint8_t sq = quantize_u4(sub_scales[s], d), mq = quantize_u4(sub_offsets[s], dmin);
        out[s] = (uint8_t)((sq & 0x0F) | ((mq & 0x0F) << 4));
    }
    uint8_t *qs = out + 16;
    memset(qs, 0, 64);
    for (int i = 0; i < 256; ++i) {
        uint8_t packed = out[i / 16];
        uint8_t q = q2k_value(block[i], d, dmin, packed & 0x0F, packed >> 4);
        qs[i / 4] |= (uint8_t)((q & 0x03) << ((i % 4) * 2));
    }
    wr_f16(out + 80, d);
    wr_f16(out + 82, dmin);
}

typedef struct {
    int t;
    const float *src;
    size_t n;
    uint8_t *dst;
    size_t blk, bytes;
} quant_ctx;

static void quant_range(void *p, size_t lo, size_t hi) {
    quant_ctx *c = (quant_ctx *)p;
    for (size_t b = lo; b < hi; ++b) {
        size_t start = b * c->blk;
        size_t len = c->n - start < c->blk ? c->n - start : c->blk;
        uint8_t *o = c->dst + b * c->bytes;
        switch (c->t) {
        case GGUF_Q8_0: q8_0_block(c->src + start, len, o); break;
        case GGUF_Q4_0: q4_0_block(c->src + start, len, o); break;
        case GGUF_Q4_K: q4_k_block(c->src + start, len, o); break;
        case GGUF_Q2_K: q2_k_block(c->src + start, len, o); break;
        }
    }
}

size_t nxo_quantize(int t, const float *src, size_t n, uint8_t *dst, int nthreads) {
    quant_ctx c = {t, src, n, dst, 0, 0};
    switch (t) {
    case GGUF_F32: memcpy(dst, src, n * 4); return n * 4;
    case GGUF_Q8_0: c.blk = 32; c.bytes = 34; break;
    case GGUF_Q4_0: c.blk = 32; c.bytes = 18; break;
    case GGUF_Q4_K: c.blk = 256; c.bytes = 144; break;
    case GGUF_Q2_K: c.blk = 256; c.bytes = 84; break;
    default: return 0;
    }
    size_t nblocks = (n + c.blk - 1) / c.blk;
    parallel_for(nblocks, nthreads, quant_range, &c);
    return nblocks * c.bytes;
}

typedef struct {
    int t;
    const uint8_t *src;
    size_t out_len;
    float *dst;
    size_t blk, bytes;
} dequant_ctx;

static void dequant_range(void *p, size_t lo, size_t hi) {
    dequant_ctx *c = (dequant_ctx *)p;
    for (size_t b = lo; b < hi; ++b) {
        const uint8_t *blk = c->src + b * c->bytes;
        size_t base = b * c->blk;
        size_t lim = c->out_len - base < c->blk ? c->out_len - base : c->blk;
        float *o = c->dst + base;
        if (c->t == GGUF_Q8_0) { /* src/quant/mod.rs:689-703 */
            float scale = rd_f16(blk);
            for (size_t i = 0; i < lim; ++i) o[i] = (float)(int8_t)blk[2 + i] * scale;
        } else if (c->t == GGUF_Q4_0) { /* src/quant/mod.rs:723-745 */
            float scale = rd_f16(blk);
            const uint8_t *qs = blk + 2;
            for (size_t i = 0; i < lim; ++i) {
                int q = i < 16 ? (qs[i] & 0x0F) : (qs[i - 16] >> 4);
                o[i] = (float)(int8_t)(q - 8) * scale;
            }
        } else if (c->t == GGUF_Q2_K) { /* src/quant/mod.rs:913-937 */
            float d = rd_f16(blk + 80), dmin = rd_f16(blk + 82);
            const uint8_t *qs = blk + 16;
            for (size_t i = 0; i < lim; ++i) {
                uint8_t q = (uint8_t)((qs[i / 4] >> ((i % 4) * 2)) & 0x03);
                uint8_t packed = blk[i / 16];
                o[i] = d * (float)(packed & 0x0F) * (float)q - dmin * (float)(packed >> 4);
            }
        } else { /* Q4_K, src/quant/mod.rs:820-849 */
            float d = rd_f16(blk), dmin = rd_f16(blk + 2);
            uint8_t scales[8], mins[8];
            nxo_unpack_q4k_scales(blk + 4, scales, mins);
            const uint8_t *qs = blk + 16;
            for (size_t i = 0; i < lim; ++i) {
                uint8_t packed = qs[i % 128];
                uint8_t q = i < 128 ? (packed & 0x0F) : (packed >> 4);
                size_t sub = i / 32;
                o[i] = d * (float)scales[sub] * (float)q - dmin * (float)mins[sub];
            }
        }
    }
}

size_t nxo_dequantize(int t, const uint8_t *src, size_t src_bytes, size_t output_len, float *dst,
                      int nthreads) {
    dequant_ctx c = {t, src, 0, dst, 0, 0};
    switch (t) {
    case GGUF_F32: {
        size_t n = src_bytes / 4 < output_len ? src_bytes / 4 : output_len;
        memcpy(dst, src, n * 4);
        return n;
    }
    case GGUF_F16: /* src/gguf/mod.rs:921-933: half::f16::to_f32 */
    case GGUF_BF16: { /* src/gguf/mod.rs:934-946: bits << 16 */
        size_t n = src_bytes / 2 < output_len ? src_bytes / 2 : output_len;
        for (size_t i = 0; i < n; ++i) {
            uint16_t h = (uint16_t)(src[2 * i] | (src[2 * i + 1] << 8));
            dst[i] = t == GGUF_F16 ? nxo_f16_to_f32(h) : u2f((uint32_t)h << 16);
        }
        return n;
    }
    case GGUF_Q8_0: c.blk = 32; c.bytes = 34; break;
    case GGUF_Q4_0: c.blk = 32; c.bytes = 18; break;
    case GGUF_Q4_K: c.blk = 256; c.bytes = 144; break;
    case GGUF_Q2_K: c.blk = 256; c.bytes = 84; break;
    default: return 0;
    }
    size_t whole = src_bytes / c.bytes; /* chunks_exact drops a ragged tail */
    size_t avail = whole * c.blk;
    size_t n = output_len < avail ? output_len : avail;
    c.out_len = n;
    size_t nblocks = (n + c.blk - 1) / c.blk;
    parallel_for(nblocks, nthreads, dequant_range, &c);
    return n;
}

/* ------------------------------------------------------------------------ */
/* router, src/engine/mod.rs:918-966                                         */
/* ------------------------------------------------------------------------ */
/* f32::total_cmp key: flip the magnitude bits of negatives, compare signed. */
static inline int32_t total_key(float f) {
    int32_t b = (int32_t)f2u(f);
    b ^= (int32_t)(((uint32_t)(b >> 31)) >> 1);
    return b;
}

size_t nxo_route(const float *logits, size_t len, size_t T, size_t E, size_t k, int score_mode,
                 int32_t *experts, float *weights, int32_t *counts) {
    for (size_t i = 0; i < T * k; ++i) {
        experts[i] = -1;
        weights[i] = 0.0f;
    }
    for (size_t t = 0; t < T; ++t) counts[t] = 0;
    if (T == 0 || E == 0 || k == 0) return 0;
    size_t *idx = (size_t *)malloc(E * sizeof(size_t));
    float *val = (float *)malloc(E * sizeof(float));
    size_t produced = 0;
    for (size_t t = 0; t < T; ++t) {
        size_t start = t * E, end = start + E;
        if (end > len) break;
        size_t n = 0;
        for (size_t e = 0; e < E; ++e) {
            float l = logits[start + e];
            if (isfinite(l)) {
                /* stable insertion: move past every kept element that is >=
                 * in total order, so equal keys keep ascending index order */
                size_t pos = n;
                while (pos > 0 && total_key(val[pos - 1]) < total_key(l)) {
                    idx[pos] = idx[pos - 1];
                    val[pos] = val[pos - 1];
                    --pos;
                }
                idx[pos] = e;
                val[pos] = l;
                ++n;
            }
        }
        size_t kk = k < E ? k : E;
        if (n > kk) n = kk;
        float *w = weights + t * k;
        int32_t *ex = experts + t * k;
        if (score_mode == 0) {
            float max_logit = -INFINITY;
            for (size_t i = 0; i < n; ++i) max_logit = fmaxf(max_logit, val[i]);
            for (size_t i = 0; i < n; ++i) w[i] = expf(val[i] - max_logit);
        } else {
            for (size_t i = 0; i < n; ++i) w[i] = 1.0f / (1.0f + expf(-val[i]));
        }
        float sum = -0.0f;
        for (size_t i = 0; i < n; ++i) sum += w[i];
        if (sum > 0.0f)
            for (size_t i = 0; i < n; ++i) w[i] /= sum;
        for (size_t i = 0; i < n; ++i) ex[i] = (int32_t)idx[i];
        counts[t] = (int32_t)n;
        produced = t + 1;
    }
    free(idx);
    free(val);
    return produced;
}

size_t nxo_permute(const int32_t *experts, const int32_t *cpt, size_t T, size_t k, size_t E,
                   int32_t *ecount, int32_t *offsets, int32_t *perm_token, int32_t *perm_slot,
                   int32_t *inv_pos) {
    for (size_t e = 0; e < E; ++e) ecount[e] = 0;
    for (size_t t = 0; t < T; ++t)
        for (size_t r = 0; r < (size_t)cpt[t]; ++r) ecount[experts[t * k + r]] += 1;
    offsets[0] = 0;
    for (size_t e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + ecount[e];
    int32_t *cursor = (int32_t *)malloc((E ? E : 1) * sizeof(int32_t));
    for (size_t e = 0; e < E; ++e) cursor[e] = offsets[e];
    for (size_t t = 0; t < T; ++t) {
        for (size_t r = 0; r < k; ++r) {
            if (r >= (size_t)cpt[t]) {
                inv_pos[t * k + r] = -1;
                continue;
            }
            int32_t e = experts[t * k + r];
            int32_t p = cursor[e]++;
            perm_token[p] = (int32_t)t;
            perm_slot[p] = (int32_t)r;
            inv_pos[t * k + r] = p;
        }
    }
    free(cursor);
    return E ? (size_t)offsets[E] : 0;
}

/* ------------------------------------------------------------------------ */
/* rms_norm, src/kernel/mod.rs:199-209                                        */
/* ------------------------------------------------------------------------ */
/* variance = (x[0]^2 + x[1]^2 + ...) / dim summed left to right, every
 * product and sum rounded to f32; rstd = 1 / sqrt(variance + eps) (both
 * correctly rounded, as sqrtss and divss); out[i] = (x[i] * rstd) * w[i]. */
void nxo_rms_norm(const float *x, const float *w, size_t dim, float eps, float *out) {
    float s = 0.0f;
    for (size_t i = 0; i < dim; ++i) s = s + x[i] * x[i];
    const float variance = s / (float)dim;
    const float rstd = 1.0f / sqrtf(variance + eps);
    for (size_t i = 0; i < dim; ++i) out[i] = x[i] * rstd * w[i];
}

/* ------------------------------------------------------------------------ */
/* matvec / dispatch, src/engine/mod.rs:775-801, 969-1024                    */
/* ------------------------------------------------------------------------ */
enum { NXO_OK = 0, NXO_E_ALIGN = 1, NXO_E_HIDDEN = 2, NXO_E_NOROUTE = 3, NXO_E_MV_IN = 4,
       NXO_E_MV_W = 5 };

int nxo_matvec(const float *w, size_t w_len, size_t rows, size_t cols, const float *x,
               size_t x_len, float *y, char *err, size_t cap) {
    if (x_len != cols) {
        if (err) snprintf(err, cap, "Matvec input shape mismatch: got %zu, expected %zu", x_len, cols);
        return NXO_E_MV_IN;
    }
    if (w_len < rows * cols) {
        if (err)
            snprintf(err, cap, "Matvec weight too small: got %zu, expected at least %zu", w_len,
                     rows * cols);
        return NXO_E_MV_W;
    }
    for (size_t r = 0; r < rows; ++r) {
        float sum = 0.0f;
        const float *wr = w + r * cols;
        for (size_t c = 0; c < cols; ++c) sum += wr[c] * x[c];
        y[r] = sum;
    }
    return NXO_OK;
}

/* one routed SwiGLU expert: y = down . (silu(gate.x) * (up.x)) */
static int expert_ffn(const float *x, const float *g, size_t gl, const float *u, size_t ul,
                      const float *dn, size_t dl, size_t H, size_t F, float *y, float *tmp_g,
                      float *tmp_u, char *err, size_t cap) {
    int rc = nxo_matvec(g, gl, F, H, x, H, tmp_g, err, cap);
    if (rc) return rc;
    rc = nxo_matvec(u, ul, F, H, x, H, tmp_u, err, cap);
    if (rc) return rc;
    for (size_t i = 0; i < F; ++i) tmp_g[i] = (tmp_g[i] / (1.0f + expf(-tmp_g[i]))) * tmp_u[i];
    return nxo_matvec(dn, dl, H, F, tmp_g, F, y, err, cap);
}

int nxo_dispatch_moe_ffn(const float *hidden, size_t hidden_len, const float *logits,
                         size_t logits_len, const float *const *gate, const size_t *gate_len,
                         const float *const *up, const size_t *up_len, const float *const *down,
                         const size_t *down_len, size_t E, size_t top_k, size_t H, size_t F,
                         float *out, char *err, size_t cap) {
    (void)up_len;
    (void)down_len;
    /* src/engine/mod.rs:975-979: the aligned-list check is on the Vec counts,
     * which the C signature makes equal by construction; E == 0 still fails */
    if (E == 0) {
        if (err) snprintf(err, cap, "MoE expert weight lists must be non-empty and aligned");
        return NXO_E_ALIGN;
    }
    if (hidden_len != H) {
        if (err) snprintf(err, cap, "MoE hidden shape mismatch: got %zu, expected %zu", hidden_len, H);
        return NXO_E_HIDDEN;
    }
    int32_t *ex = (int32_t *)malloc((top_k ? top_k : 1) * sizeof(int32_t));
    float *w = (float *)malloc((top_k ? top_k : 1) * sizeof(float));
    int32_t cnt = 0;
    size_t lists = nxo_route(logits, logits_len, 1, E, top_k, 0, ex, w, &cnt);
    if (lists == 0) {
        free(ex);
        free(w);
        if (err) snprintf(err, cap, "MoE router produced no routes");
        return NXO_E_NOROUTE;
    }
    float *tg = (float *)malloc((F ? F : 1) * sizeof(float));
    float *tu = (float *)malloc((F ? F : 1) * sizeof(float));
    float *y = (float *)malloc((H ? H : 1) * sizeof(float));
    for (size_t j = 0; j < H; ++j) out[j] = 0.0f;
    int rc = NXO_OK;
    for (int32_t r = 0; r < cnt; ++r) {
        size_t e = (size_t)ex[r];
        rc = expert_ffn(hidden, gate[e], gate_len[e], up[e], up_len[e], down[e], down_len[e], H, F,
                        y, tg, tu, err, cap);
        if (rc) break;
        for (size_t j = 0; j < H; ++j) out[j] += w[r] * y[j];
    }
    free(tg);
    free(tu);
    free(y);
    free(ex);
    free(w);
    return rc;
}

typedef struct {
    const float *x, *logits;
    size_t E, k, H, F, Fs;
    int score_mode;
    const float *const *gate, *const *up, *const *down;
    const float *sg, *su, *sd;
    float *out;
} layer_ctx;

static void layer_range(void *p, size_t lo, size_t hi) {
    layer_ctx *c = (layer_ctx *)p;
    size_t fmax = c->F > c->Fs ? c->F : c->Fs;
    float *tg = (float *)malloc((fmax ? fmax : 1) * sizeof(float));
    float *tu = (float *)malloc((fmax ? fmax : 1) * sizeof(float));
    float *y = (float *)malloc((c->H ? c->H : 1) * sizeof(float));
    int32_t *ex = (int32_t *)malloc((c->k ? c->k : 1) * sizeof(int32_t));
    float *w = (float *)malloc((c->k ? c->k : 1) * sizeof(float));
    for (size_t t = lo; t < hi; ++t) {
        const float *xt = c->x + t * c->H;
        float *ot = c->out + t * c->H;
        int32_t cnt = 0;
        nxo_route(c->logits + t * c->E, c->E, 1, c->E, c->k, c->score_mode, ex, w, &cnt);
        for (size_t j = 0; j < c->H; ++j) ot[j] = 0.0f;
        size_t wl = c->H * c->F;
        for (int32_t r = 0; r < cnt; ++r) {
            size_t e = (size_t)ex[r];
            expert_ffn(xt, c->gate[e], wl, c->up[e], wl, c->down[e], wl, c->H, c->F, y, tg, tu,
                       NULL, 0);
            for (size_t j = 0; j < c->H; ++j) ot[j] += w[r] * y[j];
        }
        if (c->sg && c->su && c->sd && c->Fs) {
            size_t sl = c->H * c->Fs;
            expert_ffn(xt, c->sg, sl, c->su, sl, c->sd, sl, c->H, c->Fs, y, tg, tu, NULL, 0);
            for (size_t j = 0; j < c->H; ++j) ot[j] += y[j];
        }
    }
    free(tg);
    free(tu);
    free(y);
    free(ex);
    free(w);
}

int nxo_moe_layer(const float *x, const float *logits, size_t T, size_t E, size_t k,
                  int score_mode, const float *const *gate, const float *const *up,
                  const float *const *down, const float *sg, const float *su, const float *sd,
                  size_t H, size_t F, size_t Fs, float *out, int nthreads) {
    layer_ctx c = {x, logits, E, k, H, F, Fs, score_mode, gate, up, down, sg, su, sd, out};
    if (E == 0 || k == 0) return NXO_E_NOROUTE;
    parallel_for(T, nthreads, layer_range, &c);
    return NXO_OK;
}

/* ------------------------------------------------------------------------ */
/* baselines: kernel::swiglu_ffn and CpuBackend::matmul                      */
/* ------------------------------------------------------------------------ */
void nxo_swiglu_ffn(const float *input, size_t input_len, const float *w1, const float *w3,
                    const float *w2, size_t H, size_t F, float *out) {
    size_t B = input_len / H;
    size_t nbf = B * F > 0 ? B * F : 1;
    float *gv = (float *)malloc(nbf * sizeof(float));
    float *uv = (float *)malloc(nbf * sizeof(float));
    for (size_t b = 0; b < B; ++b) {
        for (size_t j = 0; j < F; ++j) {
            float g = 0.0f;
            for (size_t i = 0; i < H; ++i) g += w1[j * H + i] * input[b * H + i];
            gv[b * F + j] = g;
            float u = 0.0f;
            for (size_t i = 0; i < H; ++i) u += w3[j * H + i] * input[b * H + i];
            uv[b * F + j] = u;
        }
    }
    for (size_t i = 0; i < B * F; ++i) {
        float g = gv[i], u = uv[i];
        gv[i] = g * (u / (1.0f + expf(-u)));
    }
    for (size_t b = 0; b < B; ++b) {
        for (size_t i = 0; i < H; ++i) {
            float s = 0.0f;
            for (size_t j = 0; j < F; ++j) s += w2[i * F + j] * gv[b * F + j];
            out[b * H + i] = s;
        }
    }
    free(gv);
    free(uv);
}

typedef struct {
    const float *a, *b;
    size_t n, k;
    float *c;
} mm_ctx;

static void mm_range(void *p, size_t lo, size_t hi) {
    mm_ctx *c = (mm_ctx *)p;
    for (size_t i = lo; i < hi; ++i) {
        for (size_t j = 0; j < c->n; ++j) {
            float s = 0.0f;
            for (size_t kk = 0; kk < c->k; ++kk) s += c->a[i * c->k + kk] * c->b[kk * c->n + j];
            c->c[i * c->n + j] = s;
        }
    }
}

void nxo_cpu_matmul(const float *a, const float *b, size_t m, size_t n, size_t k, float *c,
                    int nthreads) {
    mm_ctx ctx = {a, b, n, k, c};
    parallel_for(m, nthreads, mm_range, &ctx);
}
