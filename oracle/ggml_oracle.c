/*
 * ggml_oracle.c -- CPU restatement of ggml's CPU arithmetic for sam3.cpp's
 * quantized mul_mat / activation quantize / attention path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker).  Loaded by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg; never by the
 * product library.  Built with -ffp-contract=off so that the only fused
 * multiply-adds are the explicit fmaf() calls that mirror ggml's
 * _mm256_fmadd_ps.
 *
 * Anchors (what pins each function; the checks live in tests/):
 *   fp16 conversion ...... numpy.float16 over every fp16 value, every
 *                           midpoint between neighbours, and random floats
 *   quantizers ........... hand-computed known-answer blocks
 *                           (tests/golden/quant_kat.json), dequant error
 *                           bounds, nibble ranges, tie cases separating the
 *                           x86 (half-even) and _ref (half-away) variants
 *   block isums .......... brute-force integer dot over dequantized blocks
 *   vec_dot / mul_mat .... long-double brute force of ggml's block formula;
 *                           numpy float64 matmul of dequantized operands;
 *                           AVX2 and AVX512-VNNI paths bit-identical to the
 *                           scalar order
 *   soft_max ............. rows sum to 1; numpy/scipy softmax
 *   flash_attn_ext ....... long-double textbook attention; key-permutation
 *                           equivariance; strided V == contiguous V bit-exact
 *                           (tests/test_v_cont_removal.cpp:156-160)
 *   ViT glue ............. numpy restatements of torch LayerNorm/erf-GELU;
 *                           RoPE tables as closed forms (tests/test_vit.cpp:
 *                           182,192,218); win_part∘win_unpart = identity
 *   Hiera pos-embed ...... torch bicubic interpolate (align_corners=False,
 *                           A = -0.75); identity at equal sizes; constant
 *                           and linear inputs reproduced in the interior
 */
#define _GNU_SOURCE
#include "ggml_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#if defined(__x86_64__)
#include <immintrin.h>
#endif

/* ------------------------------------------------------------------ */
/* block formats (ggml-common.h): little-endian, packed                 */
/* ------------------------------------------------------------------ */
#pragma pack(push, 1)
typedef struct { uint16_t d; int8_t qs[32]; } blk_q8_0;             /* 34 B */
typedef struct { uint16_t d; uint16_t s; int8_t qs[32]; } blk_q8_1; /* 36 B */
typedef struct { uint16_t d; uint8_t qs[16]; } blk_q4_0;            /* 18 B */
typedef struct { uint16_t d; uint16_t m; uint8_t qs[16]; } blk_q4_1; /* 20 B */
#pragma pack(pop)

_Static_assert(sizeof(blk_q8_0) == 34, "q8_0");
_Static_assert(sizeof(blk_q8_1) == 36, "q8_1");
_Static_assert(sizeof(blk_q4_0) == 18, "q4_0");
_Static_assert(sizeof(blk_q4_1) == 20, "q4_1");

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------ */
/* fp16 (IEEE binary16).  fp32->fp16 rounds to nearest even, following  */
/* the published "float_to_half_fast3_rtne" construction (F. Giesen):    */
/* normals by integer rebias + round-bit add, subnormals by letting the  */
/* FPU round an add of 0.5f whose ulp equals the fp16 subnormal step.    */
/* ggml uses F16C _cvtss_sh(x, 0) on x86, which is the same rounding.    */
/* ------------------------------------------------------------------ */
uint16_t orc_fp32_to_fp16(float f) {
    const uint32_t x = f2u(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t a = x & 0x7fffffffu;
    uint16_t o;
    if (a >= 0x47800000u) {            /* |f| >= 2^16, inf or nan */
        o = (a > 0x7f800000u) ? 0x7e00u : 0x7c00u;
    } else if (a < 0x38800000u) {      /* |f| < 2^-14: subnormal or zero */
        const float t = u2f(a) + 0.5f; /* ulp(0.5) == 2^-24 == fp16 subnormal step */
        o = (uint16_t)(f2u(t) - 0x3f000000u);
    } else {                           /* normal: rebias exponent, round half even */
        const uint32_t odd = (a >> 13) & 1u;
        a += ((uint32_t)(15 - 127) << 23) + 0xfffu + odd;
        o = (uint16_t)(a >> 13);       /* mantissa carry into exponent is the correct result */
    }
    return (uint16_t)(o | sign);
}

float orc_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    if (e == 0) {
        const float v = (float)m * 0x1p-24f; /* exact: m < 2^10 */
        return sign ? -v : v;
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

void orc_fp32_to_fp16_row(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_fp32_to_fp16(x[i]);
}
void orc_fp16_to_fp32_row(const uint16_t* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_fp16_to_fp32(x[i]);
}
static inline float h2f(uint16_t h) { return orc_fp16_to_fp32(h); }
static inline uint16_t f2h(float f) { return orc_fp32_to_fp16(f); }

/* ------------------------------------------------------------------ */
/* Deterministic synthetic inputs.  SplitMix64 (Steele, Lea, Flood 2014)  */
/* is counter based: element i of stream (seed, stream) is                */
/* mix(s0 + (i+1)*gamma) with s0 = seed ^ (stream * 0xd1b54a32d192ed03).  */
/* Normals by Box-Muller in double:                                       */
/*   u1 = ((z0>>11)+1)*2^-53 in (0,1],  u2 = (z1>>11)*2^-53 in [0,1)      */
/*   r = sqrt(-2 ln u1);  out[2i] = mean + sd*r*cos(2 pi u2),             */
/*                        out[2i+1] = mean + sd*r*sin(2 pi u2)            */
/* Uniform: u = (z>>40)*2^-24 (exact in float), out = lo + (hi-lo)*u.     */
/* ------------------------------------------------------------------ */
uint64_t orc_splitmix64(uint64_t* state) {
    uint64_t z = (*state += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

static uint64_t stream_state(uint64_t seed, uint64_t stream) {
    return seed ^ (stream * 0xd1b54a32d192ed03ull);
}

void orc_fill_normal(float* out, int64_t n, uint64_t seed, uint64_t stream, float mean, float stddev) {
    uint64_t st = stream_state(seed, stream);
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = 0; i < n; i += 2) {
        const uint64_t z0 = orc_splitmix64(&st);
        const uint64_t z1 = orc_splitmix64(&st);
        const double u1 = (double)((z0 >> 11) + 1) * 0x1p-53;
        const double u2 = (double)(z1 >> 11) * 0x1p-53;
        const double r = sqrt(-2.0 * log(u1));
        out[i] = (float)((double)mean + (double)stddev * r * cos(two_pi * u2));
        if (i + 1 < n) out[i + 1] = (float)((double)mean + (double)stddev * r * sin(two_pi * u2));
    }
}

void orc_fill_uniform(float* out, int64_t n, uint64_t seed, uint64_t stream, float lo, float hi) {
    uint64_t st = stream_state(seed, stream);
    for (int64_t i = 0; i < n; ++i) {
        const float u = (float)(orc_splitmix64(&st) >> 40) * 0x1p-24f;
        out[i] = lo + (hi - lo) * u;
    }
}

/* ------------------------------------------------------------------ */
/* type traits                                                           */
/* ------------------------------------------------------------------ */
int orc_blck_size(int type) {
    switch (type) {
        case ORC_TYPE_F32: case ORC_TYPE_F16: return 1;
        case ORC_TYPE_Q4_0: case ORC_TYPE_Q4_1: case ORC_TYPE_Q8_0: case ORC_TYPE_Q8_1: return ORC_QK;
        default: return 0;
    }
}
int64_t orc_type_size(int type) {
    switch (type) {
        case ORC_TYPE_F32: return 4;
        case ORC_TYPE_F16: return 2;
        case ORC_TYPE_Q4_0: return sizeof(blk_q4_0);
        case ORC_TYPE_Q4_1: return sizeof(blk_q4_1);
        case ORC_TYPE_Q8_0: return sizeof(blk_q8_0);
        case ORC_TYPE_Q8_1: return sizeof(blk_q8_1);
        default: return 0;
    }
}
int64_t orc_row_size(int type, int64_t ne0) {
    const int bs = orc_blck_size(type);
    if (bs == 0) return 0;
    return orc_type_size(type) * (ne0 / bs);
}
int orc_vec_dot_type(int type) {
    switch (type) {
        case ORC_TYPE_F32: return ORC_TYPE_F32;
        case ORC_TYPE_F16: return ORC_TYPE_F16;
        case ORC_TYPE_Q4_0: return ORC_TYPE_Q8_0;
        case ORC_TYPE_Q8_0: return ORC_TYPE_Q8_0;
        case ORC_TYPE_Q4_1: return ORC_TYPE_Q8_1;
        default: return -1;
    }
}

/* ------------------------------------------------------------------ */
/* quantizers                                                            */
/* ------------------------------------------------------------------ */

/* quantize_row_q8_0_ref: d = amax/127, id = d ? 1/d : 0, q = roundf(x*id). */
void orc_quantize_row_q8_0_ref(const float* x, void* vy, int64_t k) {
    blk_q8_0* y = (blk_q8_0*)vy;
    const int64_t nb = k / ORC_QK;
    for (int64_t i = 0; i < nb; ++i) {
        float amax = 0.0f;
        for (int j = 0; j < ORC_QK; ++j) amax = fmaxf(amax, fabsf(x[i * ORC_QK + j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = f2h(d);
        for (int j = 0; j < ORC_QK; ++j) y[i].qs[j] = (int8_t)roundf(x[i * ORC_QK + j] * id);
    }
}

/* AVX2 quantize_row_q8_0: d = amax/127, id = amax ? 127/amax : 0,
 * q = round-half-even(x*id) (_mm256_round_ps(.., _MM_ROUND_NEAREST)). */
void orc_quantize_row_q8_0_x86(const float* x, void* vy, int64_t k) {
    blk_q8_0* y = (blk_q8_0*)vy;
    const int64_t nb = k / ORC_QK;
    for (int64_t i = 0; i < nb; ++i) {
        float amax = 0.0f;
        for (int j = 0; j < ORC_QK; ++j) amax = fmaxf(amax, fabsf(x[i * ORC_QK + j]));
        const float d = amax / 127.0f;
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        y[i].d = f2h(d);
        for (int j = 0; j < ORC_QK; ++j) y[i].qs[j] = (int8_t)rintf(x[i * ORC_QK + j] * id);
    }
}

/* quantize_row_q8_1_ref: as q8_0_ref plus s = fp16(sum(q) * d). */
void orc_quantize_row_q8_1_ref(const float* x, void* vy, int64_t k) {
    blk_q8_1* y = (blk_q8_1*)vy;
    const int64_t nb = k / ORC_QK;
    for (int64_t i = 0; i < nb; ++i) {
        float amax = 0.0f;
        for (int j = 0; j < ORC_QK; ++j) amax = fmaxf(amax, fabsf(x[i * ORC_QK + j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = f2h(d);
        int sum = 0;
        for (int j = 0; j < ORC_QK; ++j) {
            y[i].qs[j] = (int8_t)roundf(x[i * ORC_QK + j] * id);
            sum += y[i].qs[j];
        }
        y[i].s = f2h((float)sum * d);
    }
}

/* AVX2 quantize_row_q8_1: x86 q8_0 rounding plus s = fp16(d * hsum(q)). */
void orc_quantize_row_q8_1_x86(const float* x, void* vy, int64_t k) {
    blk_q8_1* y = (blk_q8_1*)vy;
    const int64_t nb = k / ORC_QK;
    for (int64_t i = 0; i < nb; ++i) {
        float amax = 0.0f;
        for (int j = 0; j < ORC_QK; ++j) amax = fmaxf(amax, fabsf(x[i * ORC_QK + j]));
        const float d = amax / 127.0f;
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        y[i].d = f2h(d);
        int sum = 0;
        for (int j = 0; j < ORC_QK; ++j) {
            y[i].qs[j] = (int8_t)rintf(x[i * ORC_QK + j] * id);
            sum += y[i].qs[j];
        }
        y[i].s = f2h(d * (float)sum);
    }
}

/* quantize_row_q4_0_ref: max = the x of largest |x| (first one wins),
 * d = max/-8, id = d ? 1/d : 0, q = min(15, (int8)(x*id + 8.5)),
 * qs[j] = q[j] | q[j+16] << 4. */
void orc_quantize_row_q4_0_ref(const float* x, void* vy, int64_t k) {
    blk_q4_0* y = (blk_q4_0*)vy;
    const int64_t nb = k / ORC_QK;
    for (int64_t i = 0; i < nb; ++i) {
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < ORC_QK; ++j) {
            const float v = x[i * ORC_QK + j];
            if (amax < fabsf(v)) { amax = fabsf(v); max = v; }
        }
        const float d = max / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = f2h(d);
        for (int j = 0; j < ORC_QK / 2; ++j) {
            const float x0 = x[i * ORC_QK + j] * id;
            const float x1 = x[i * ORC_QK + ORC_QK / 2 + j] * id;
            int q0 = (int8_t)(x0 + 8.5f); if (q0 > 15) q0 = 15;
            int q1 = (int8_t)(x1 + 8.5f); if (q1 > 15) q1 = 15;
            y[i].qs[j] = (uint8_t)((uint8_t)q0 | ((uint8_t)q1 << 4));
        }
    }
}

/* quantize_row_q4_1_ref: d = (max-min)/15, m = min, id = d ? 1/d : 0,
 * q = min(15, (int8)((x-min)*id + 0.5)). */
void orc_quantize_row_q4_1_ref(const float* x, void* vy, int64_t k) {
    blk_q4_1* y = (blk_q4_1*)vy;
    const int64_t nb = k / ORC_QK;
    for (int64_t i = 0; i < nb; ++i) {
        float min = FLT_MAX, max = -FLT_MAX;
        for (int j = 0; j < ORC_QK; ++j) {
            const float v = x[i * ORC_QK + j];
            if (v < min) min = v;
            if (v > max) max = v;
        }
        const float d = (max - min) / 15.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = f2h(d);
        y[i].m = f2h(min);
        for (int j = 0; j < ORC_QK / 2; ++j) {
            const float x0 = (x[i * ORC_QK + j] - min) * id;
            const float x1 = (x[i * ORC_QK + ORC_QK / 2 + j] - min) * id;
            int q0 = (int8_t)(x0 + 0.5f); if (q0 > 15) q0 = 15;
            int q1 = (int8_t)(x1 + 0.5f); if (q1 > 15) q1 = 15;
            y[i].qs[j] = (uint8_t)((uint8_t)q0 | ((uint8_t)q1 << 4));
        }
    }
}

int64_t orc_quantize_chunk(int type, const float* src, void* dst, int64_t start,
                           int64_t nrows, int64_t n_per_row) {
    const int64_t row_size = orc_row_size(type, n_per_row);
    const int64_t r0 = start / n_per_row;
    uint8_t* out = (uint8_t*)dst + r0 * row_size;
    for (int64_t r = 0; r < nrows; ++r) {
        const float* x = src + start + r * n_per_row;
        void* y = out + r * row_size;
        switch (type) {
            case ORC_TYPE_Q8_0: orc_quantize_row_q8_0_ref(x, y, n_per_row); break;
            case ORC_TYPE_Q8_1: orc_quantize_row_q8_1_ref(x, y, n_per_row); break;
            case ORC_TYPE_Q4_0: orc_quantize_row_q4_0_ref(x, y, n_per_row); break;
            case ORC_TYPE_Q4_1: orc_quantize_row_q4_1_ref(x, y, n_per_row); break;
            case ORC_TYPE_F16: orc_fp32_to_fp16_row(x, (uint16_t*)y, n_per_row); break;
            case ORC_TYPE_F32: memcpy(y, x, (size_t)n_per_row * 4); break;
            default: return -1;
        }
    }
    return nrows * row_size;
}

int orc_from_float(int type, int act_variant, const float* x, void* y, int64_t k) {
    switch (type) {
        case ORC_TYPE_Q8_0:
            if (act_variant == ORC_ACT_REF) orc_quantize_row_q8_0_ref(x, y, k);
            else orc_quantize_row_q8_0_x86(x, y, k);
            return 0;
        case ORC_TYPE_Q8_1:
            if (act_variant == ORC_ACT_REF) orc_quantize_row_q8_1_ref(x, y, k);
            else orc_quantize_row_q8_1_x86(x, y, k);
            return 0;
        case ORC_TYPE_F16: orc_fp32_to_fp16_row(x, (uint16_t*)y, k); return 0;
        case ORC_TYPE_F32: memcpy(y, x, (size_t)k * 4); return 0;
        default: return -1;
    }
}

int orc_dequantize_row(int type, const void* vx, float* y, int64_t k) {
    const int64_t nb = k / ORC_QK;
    switch (type) {
        case ORC_TYPE_Q8_0: {
            const blk_q8_0* x = (const blk_q8_0*)vx;
            for (int64_t i = 0; i < nb; ++i) {
                const float d = h2f(x[i].d);
                for (int j = 0; j < ORC_QK; ++j) y[i * ORC_QK + j] = x[i].qs[j] * d;
            }
            return 0;
        }
        case ORC_TYPE_Q8_1: {
            const blk_q8_1* x = (const blk_q8_1*)vx;
            for (int64_t i = 0; i < nb; ++i) {
                const float d = h2f(x[i].d);
                for (int j = 0; j < ORC_QK; ++j) y[i * ORC_QK + j] = x[i].qs[j] * d;
            }
            return 0;
        }
        case ORC_TYPE_Q4_0: {
            const blk_q4_0* x = (const blk_q4_0*)vx;
            for (int64_t i = 0; i < nb; ++i) {
                const float d = h2f(x[i].d);
                for (int j = 0; j < ORC_QK / 2; ++j) {
                    y[i * ORC_QK + j] = (float)((x[i].qs[j] & 0x0f) - 8) * d;
                    y[i * ORC_QK + j + 16] = (float)((x[i].qs[j] >> 4) - 8) * d;
                }
            }
            return 0;
        }
        case ORC_TYPE_Q4_1: {
            const blk_q4_1* x = (const blk_q4_1*)vx;
            for (int64_t i = 0; i < nb; ++i) {
                const float d = h2f(x[i].d), m = h2f(x[i].m);
                for (int j = 0; j < ORC_QK / 2; ++j) {
                    y[i * ORC_QK + j] = (float)(x[i].qs[j] & 0x0f) * d + m;
                    y[i * ORC_QK + j + 16] = (float)(x[i].qs[j] >> 4) * d + m;
                }
            }
            return 0;
        }
        case ORC_TYPE_F16: orc_fp16_to_fp32_row((const uint16_t*)vx, y, k); return 0;
        case ORC_TYPE_F32: memcpy(y, vx, (size_t)k * 4); return 0;
        default: return -1;
    }
}

/* ------------------------------------------------------------------ */
/* dot products                                                          */
/* ------------------------------------------------------------------ */

/* hsum_float_8 of ggml x86: r_i = a[i+4] + a[i]; (r0 + r2) + (r1 + r3). */
static inline float hsum8(const float a[8]) {
    const float r0 = a[4] + a[0], r1 = a[5] + a[1], r2 = a[6] + a[2], r3 = a[7] + a[3];
    return (r0 + r2) + (r1 + r3);
}

/* Unpacked signed weights of one block, element order 0..31. */
static inline void unpack_q4_0(const blk_q4_0* b, int8_t q[32]) {
    for (int j = 0; j < 16; ++j) {
        q[j] = (int8_t)((b->qs[j] & 0x0f) - 8);
        q[j + 16] = (int8_t)((b->qs[j] >> 4) - 8);
    }
}
static inline void unpack_q4_1(const blk_q4_1* b, int8_t q[32]) {
    for (int j = 0; j < 16; ++j) {
        q[j] = (int8_t)(b->qs[j] & 0x0f);
        q[j + 16] = (int8_t)(b->qs[j] >> 4);
    }
}

/* Scalar dots.  X86 order: eight fp32 lanes, lane l holds the int sum of
 * elements 4l..4l+3 of each block times fp32(d_x)*fp32(d_y), fused with
 * fmaf into its accumulator (mul_sum_i8_pairs_float + _mm256_fmadd_ps of
 * vec_dot_q8_0_q8_0 / tinyBLAS_Q0_AVX); then hsum_float_8.  SEQ order: the
 * generic C loop, sumf += (float)isum * (d_x*d_y). */
static float dot_q8_scalar(int type, int64_t nb, const void* vx, const void* vy, int order) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float sumf = 0.0f, summs = 0.0f;
    for (int64_t b = 0; b < nb; ++b) {
        int8_t qx[32];
        const int8_t* qy;
        float dx, dy, mx = 0.0f, sy = 0.0f;
        if (type == ORC_TYPE_Q8_0) {
            const blk_q8_0* x = (const blk_q8_0*)vx + b;
            memcpy(qx, x->qs, 32);
            dx = h2f(x->d);
        } else if (type == ORC_TYPE_Q4_0) {
            const blk_q4_0* x = (const blk_q4_0*)vx + b;
            unpack_q4_0(x, qx);
            dx = h2f(x->d);
        } else { /* Q4_1 */
            const blk_q4_1* x = (const blk_q4_1*)vx + b;
            unpack_q4_1(x, qx);
            dx = h2f(x->d);
            mx = h2f(x->m);
        }
        if (type == ORC_TYPE_Q4_1) {
            const blk_q8_1* y = (const blk_q8_1*)vy + b;
            qy = y->qs;
            dy = h2f(y->d);
            sy = h2f(y->s);
        } else {
            const blk_q8_0* y = (const blk_q8_0*)vy + b;
            qy = y->qs;
            dy = h2f(y->d);
        }
        const float d = dx * dy; /* exact: two 11-bit significands */
        if (order == ORC_ORDER_X86) {
            for (int l = 0; l < 8; ++l) {
                int s = 0;
                for (int j = 4 * l; j < 4 * l + 4; ++j) s += qx[j] * qy[j];
                acc[l] = fmaf(d, (float)s, acc[l]);
            }
            if (type == ORC_TYPE_Q4_1) {
                const float t = mx * sy;
                summs = summs + t;
            }
        } else {
            int s = 0;
            for (int j = 0; j < 32; ++j) s += qx[j] * qy[j];
            const float t = (float)s * d;
            sumf = sumf + t;
            if (type == ORC_TYPE_Q4_1) {
                const float u = mx * sy;
                sumf = sumf + u;
            }
        }
    }
    if (order == ORC_ORDER_X86) return hsum8(acc) + summs;
    return sumf;
}

/* F16 . F16 with fp32 products.  X86 order: tinyBLAS<8,__m256> (the path
 * ggml-cpu takes for F16 weights once src1 is converted to F16): lane l
 * accumulates elements k = l (mod 8) with fmaf, then hsum_float_8; k%8 tail
 * (not used by the configs) falls back to the SEQ loop.  SEQ order: a plain
 * fp32 running sum of rounded products. */
static float dot_f16_scalar(int64_t n, const uint16_t* x, const uint16_t* y, int order) {
    if (order == ORC_ORDER_X86 && n % 8 == 0) {
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int64_t i = 0; i < n; i += 8)
            for (int l = 0; l < 8; ++l) acc[l] = fmaf(h2f(x[i + l]), h2f(y[i + l]), acc[l]);
        return hsum8(acc);
    }
    float s = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        const float p = h2f(x[i]) * h2f(y[i]);
        s = s + p;
    }
    return s;
}

/* ggml_vec_dot_f32 / ggml_vec_dot_f16 (AVX): four 8-lane accumulators over
 * steps of 32, GGML_F32x8_REDUCE, tail in double.  Used for the K.Q dot of
 * flash_attn_ext. */
static float dot_vec_f32_like(int64_t n, const float* x, const float* y) {
    float a[4][8];
    memset(a, 0, sizeof(a));
    const int64_t np = n & ~(int64_t)31;
    for (int64_t i = 0; i < np; i += 32)
        for (int j = 0; j < 4; ++j)
            for (int l = 0; l < 8; ++l) a[j][l] = fmaf(x[i + 8 * j + l], y[i + 8 * j + l], a[j][l]);
    for (int l = 0; l < 8; ++l) { a[0][l] = a[0][l] + a[2][l]; a[1][l] = a[1][l] + a[3][l]; }
    for (int l = 0; l < 8; ++l) a[0][l] = a[0][l] + a[1][l];
    float t[4];
    for (int l = 0; l < 4; ++l) t[l] = a[0][l] + a[0][l + 4];
    /* _mm_hadd_ps twice: ((t0+t1) + (t2+t3)) */
    const float h0 = t[0] + t[1], h1 = t[2] + t[3];
    double sumf = (double)(h0 + h1);
    for (int64_t i = np; i < n; ++i) sumf += (double)(x[i] * y[i]);
    return (float)sumf;
}

#if defined(__x86_64__)
/* AVX2 versions of the X86-order dots: identical arithmetic, vectorised. */
__attribute__((target("avx2,fma,f16c")))
static float dot_q8_avx2(int type, int64_t nb, const void* vx, const void* vy) {
    __m256 acc = _mm256_setzero_ps();
    float summs = 0.0f;
    const __m256i ones16 = _mm256_set1_epi16(1);
    for (int64_t b = 0; b < nb; ++b) {
        __m256i qx, qy;
        float dx, dy;
        if (type == ORC_TYPE_Q8_0) {
            const blk_q8_0* x = (const blk_q8_0*)vx + b;
            qx = _mm256_loadu_si256((const __m256i*)x->qs);
            dx = h2f(x->d);
        } else {
            const uint8_t* qs;
            if (type == ORC_TYPE_Q4_0) {
                const blk_q4_0* x = (const blk_q4_0*)vx + b;
                qs = x->qs; dx = h2f(x->d);
            } else {
                const blk_q4_1* x = (const blk_q4_1*)vx + b;
                qs = x->qs; dx = h2f(x->d);
            }
            const __m128i t = _mm_loadu_si128((const __m128i*)qs);
            const __m256i both = _mm256_insertf128_si256(_mm256_castsi128_si256(t), _mm_srli_epi16(t, 4), 1);
            qx = _mm256_and_si256(both, _mm256_set1_epi8(0x0f));
            if (type == ORC_TYPE_Q4_0) qx = _mm256_sub_epi8(qx, _mm256_set1_epi8(8));
        }
        if (type == ORC_TYPE_Q4_1) {
            const blk_q8_1* y = (const blk_q8_1*)vy + b;
            qy = _mm256_loadu_si256((const __m256i*)y->qs);
            dy = h2f(y->d);
            const float t = h2f(((const blk_q4_1*)vx + b)->m) * h2f(y->s);
            summs = summs + t;
        } else {
            const blk_q8_0* y = (const blk_q8_0*)vy + b;
            qy = _mm256_loadu_si256((const __m256i*)y->qs);
            dy = h2f(y->d);
        }
        /* |x| * sign(y, x): exact pairwise products, no i16 saturation for |q|<=127 */
        const __m256i ax = _mm256_sign_epi8(qx, qx);
        const __m256i sy = _mm256_sign_epi8(qy, qx);
        const __m256i p16 = _mm256_maddubs_epi16(ax, sy);
        const __m256i p32 = _mm256_madd_epi16(p16, ones16);
        acc = _mm256_fmadd_ps(_mm256_set1_ps(dx * dy), _mm256_cvtepi32_ps(p32), acc);
    }
    float a[8];
    _mm256_storeu_ps(a, acc);
    return hsum8(a) + summs;
}

/* The same dot with AVX512-VNNI: ggml's mul_sum_us8_pairs_float takes _mm256_dpbusd_epi32
 * when __AVX512VNNI__ and __AVX512VL__ are defined, which sums the four u8 x s8 products of
 * each 32-bit lane into int32 exactly as maddubs + madd(ones) do for |q| <= 127 (no 16-bit
 * saturation is reachable), so the eight lanes, their float conversion and the fmadd
 * order are those of dot_q8_avx2 and the result is bit-identical. */
__attribute__((target("avx2,fma,f16c,avx512f,avx512vl,avx512vnni")))
static float dot_q8_vnni(int type, int64_t nb, const void* vx, const void* vy) {
    __m256 acc = _mm256_setzero_ps();
    float summs = 0.0f;
    const __m256i zero = _mm256_setzero_si256();
    for (int64_t b = 0; b < nb; ++b) {
        __m256i qx, qy;
        float dx, dy;
        if (type == ORC_TYPE_Q8_0) {
            const blk_q8_0* x = (const blk_q8_0*)vx + b;
            qx = _mm256_loadu_si256((const __m256i*)x->qs);
            dx = h2f(x->d);
        } else {
            const uint8_t* qs;
            if (type == ORC_TYPE_Q4_0) {
                const blk_q4_0* x = (const blk_q4_0*)vx + b;
                qs = x->qs; dx = h2f(x->d);
            } else {
                const blk_q4_1* x = (const blk_q4_1*)vx + b;
                qs = x->qs; dx = h2f(x->d);
            }
            const __m128i t = _mm_loadu_si128((const __m128i*)qs);
            const __m256i both = _mm256_insertf128_si256(_mm256_castsi128_si256(t), _mm_srli_epi16(t, 4), 1);
            qx = _mm256_and_si256(both, _mm256_set1_epi8(0x0f));
            if (type == ORC_TYPE_Q4_0) qx = _mm256_sub_epi8(qx, _mm256_set1_epi8(8));
        }
        if (type == ORC_TYPE_Q4_1) {
            const blk_q8_1* y = (const blk_q8_1*)vy + b;
            qy = _mm256_loadu_si256((const __m256i*)y->qs);
            dy = h2f(y->d);
            const float t = h2f(((const blk_q4_1*)vx + b)->m) * h2f(y->s);
            summs = summs + t;
        } else {
            const blk_q8_0* y = (const blk_q8_0*)vy + b;
            qy = _mm256_loadu_si256((const __m256i*)y->qs);
            dy = h2f(y->d);
        }
        const __m256i ax = _mm256_sign_epi8(qx, qx);
        const __m256i sy = _mm256_sign_epi8(qy, qx);
        const __m256i p32 = _mm256_dpbusd_epi32(zero, ax, sy);
        acc = _mm256_fmadd_ps(_mm256_set1_ps(dx * dy), _mm256_cvtepi32_ps(p32), acc);
    }
    float a[8];
    _mm256_storeu_ps(a, acc);
    return hsum8(a) + summs;
}

__attribute__((target("avx2,fma,f16c")))
static float dot_f16_avx2(int64_t n, const uint16_t* x, const uint16_t* y) {
    __m256 acc = _mm256_setzero_ps();
    for (int64_t i = 0; i < n; i += 8) {
        const __m256 ax = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(x + i)));
        const __m256 ay = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(y + i)));
        acc = _mm256_fmadd_ps(ax, ay, acc);
    }
    float a[8];
    _mm256_storeu_ps(a, acc);
    return hsum8(a);
}
#endif

/* 0 scalar, 1 AVX2 + FMA, 2 AVX2 + FMA with AVX512-VNNI/VL for the quantized dots (the
 * F16 and F32 dots keep their AVX2 / scalar forms on path 2). */
static int g_isa = -1;
static int isa_detect(void) {
#if defined(__x86_64__)
    __builtin_cpu_init();
    if (!(__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma"))) return 0;
    if (__builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512vl") &&
        __builtin_cpu_supports("avx512vnni"))
        return 2;
    return 1;
#else
    return 0;
#endif
}
int orc_isa_path(void) {
    if (g_isa < 0) g_isa = isa_detect();
    return g_isa;
}
/* path < 0 re-detects; otherwise the requested path, or the best supported one below it. */
void orc_set_isa(int path) {
    const int have = isa_detect();
    g_isa = path < 0 ? have : (path < have ? path : have);
}

float orc_vec_dot(int type, int64_t n, const void* x, const void* y, int order) {
    switch (type) {
        case ORC_TYPE_Q8_0: case ORC_TYPE_Q4_0: case ORC_TYPE_Q4_1:
#if defined(__x86_64__)
            if (order == ORC_ORDER_X86 && orc_isa_path() == 2) return dot_q8_vnni(type, n / ORC_QK, x, y);
            if (order == ORC_ORDER_X86 && orc_isa_path() == 1) return dot_q8_avx2(type, n / ORC_QK, x, y);
#endif
            return dot_q8_scalar(type, n / ORC_QK, x, y, order);
        case ORC_TYPE_F16:
#if defined(__x86_64__)
            if (order == ORC_ORDER_X86 && n % 8 == 0 && orc_isa_path() >= 1)
                return dot_f16_avx2(n, (const uint16_t*)x, (const uint16_t*)y);
#endif
            return dot_f16_scalar(n, (const uint16_t*)x, (const uint16_t*)y, order);
        case ORC_TYPE_F32:
            return dot_vec_f32_like(n, (const float*)x, (const float*)y);
        default:
            return NAN;
    }
}

int orc_block_isums(int type, int64_t n, const void* vx, const void* vy, int32_t* out) {
    const int64_t nb = n / ORC_QK;
    for (int64_t b = 0; b < nb; ++b) {
        int8_t qx[32];
        const int8_t* qy;
        if (type == ORC_TYPE_Q8_0) memcpy(qx, ((const blk_q8_0*)vx)[b].qs, 32);
        else if (type == ORC_TYPE_Q4_0) unpack_q4_0((const blk_q4_0*)vx + b, qx);
        else if (type == ORC_TYPE_Q4_1) unpack_q4_1((const blk_q4_1*)vx + b, qx);
        else return -1;
        qy = (type == ORC_TYPE_Q4_1) ? ((const blk_q8_1*)vy)[b].qs : ((const blk_q8_0*)vy)[b].qs;
        int32_t s = 0;
        for (int j = 0; j < 32; ++j) s += (int32_t)qx[j] * (int32_t)qy[j];
        out[b] = s;
    }
    return 0;
}

/* ggml's block formula, summed in long double: sum_b dx*dy*isum_b (+ mx*sy).
 * absterm = sum_b |dx*dy| * sum_j |qx_j*qy_j| (+ |mx*sy|): the sum of absolute
 * elementwise terms, which bounds the rounding error of any summation order
 * (|fl(sum) - sum| <= gamma_n * absterm). */
static long double dot_exact_ld(int type, int64_t n, const void* vx, const void* vy, long double* absterm) {
    long double s = 0.0L, a = 0.0L;
    if (type == ORC_TYPE_F16) {
        const uint16_t* x = (const uint16_t*)vx;
        const uint16_t* y = (const uint16_t*)vy;
        for (int64_t i = 0; i < n; ++i) {
            const long double p = (long double)h2f(x[i]) * (long double)h2f(y[i]);
            s += p; a += fabsl(p);
        }
    } else if (type == ORC_TYPE_F32) {
        const float* x = (const float*)vx;
        const float* y = (const float*)vy;
        for (int64_t i = 0; i < n; ++i) {
            const long double p = (long double)x[i] * (long double)y[i];
            s += p; a += fabsl(p);
        }
    } else {
        const int64_t nb = n / ORC_QK;
        for (int64_t b = 0; b < nb; ++b) {
            int8_t qx[32];
            const int8_t* qy;
            long double dx, dy, mx = 0.0L, sy = 0.0L;
            if (type == ORC_TYPE_Q8_0) {
                const blk_q8_0* x = (const blk_q8_0*)vx + b;
                memcpy(qx, x->qs, 32); dx = h2f(x->d);
            } else if (type == ORC_TYPE_Q4_0) {
                const blk_q4_0* x = (const blk_q4_0*)vx + b;
                unpack_q4_0(x, qx); dx = h2f(x->d);
            } else {
                const blk_q4_1* x = (const blk_q4_1*)vx + b;
                unpack_q4_1(x, qx); dx = h2f(x->d); mx = h2f(x->m);
            }
            if (type == ORC_TYPE_Q4_1) {
                const blk_q8_1* y = (const blk_q8_1*)vy + b;
                qy = y->qs; dy = h2f(y->d); sy = h2f(y->s);
            } else {
                const blk_q8_0* y = (const blk_q8_0*)vy + b;
                qy = y->qs; dy = h2f(y->d);
            }
            int32_t is = 0, ia = 0;
            for (int j = 0; j < 32; ++j) {
                const int32_t p = (int32_t)qx[j] * (int32_t)qy[j];
                is += p; ia += p < 0 ? -p : p;
            }
            s += dx * dy * (long double)is;
            a += fabsl(dx * dy) * (long double)ia;
            if (type == ORC_TYPE_Q4_1) { s += mx * sy; a += fabsl(mx * sy); }
        }
    }
    if (absterm) *absterm = a;
    return s;
}

double orc_vec_dot_exact(int type, int64_t n, const void* x, const void* y) {
    return (double)dot_exact_ld(type, n, x, y, NULL);
}
double orc_vec_dot_absterm(int type, int64_t n, const void* x, const void* y) {
    long double a;
    (void)dot_exact_ld(type, n, x, y, &a);
    return (double)a;
}

/* ------------------------------------------------------------------ */
/* threading helper                                                      */
/* ------------------------------------------------------------------ */
typedef void (*range_fn)(void* ctx, int64_t begin, int64_t end);
typedef struct { range_fn fn; void* ctx; int64_t b, e; } range_job;
static void* range_thread(void* p) { range_job* j = (range_job*)p; j->fn(j->ctx, j->b, j->e); return NULL; }

static void parallel_for(int64_t n, int n_threads, range_fn fn, void* ctx) {
    if (n_threads <= 1 || n < 2) { fn(ctx, 0, n); return; }
    if (n_threads > 256) n_threads = 256;
    if (n_threads > n) n_threads = (int)n;
    pthread_t th[256];
    range_job jobs[256];
    for (int t = 0; t < n_threads; ++t) {
        jobs[t].fn = fn; jobs[t].ctx = ctx;
        jobs[t].b = n * t / n_threads; jobs[t].e = n * (t + 1) / n_threads;
        if (t > 0) pthread_create(&th[t], NULL, range_thread, &jobs[t]);
    }
    range_thread(&jobs[0]);
    for (int t = 1; t < n_threads; ++t) pthread_join(th[t], NULL);
}

/* ------------------------------------------------------------------ */
/* mul_mat                                                               */
/* ------------------------------------------------------------------ */
typedef struct {
    const orc_tensor *src0, *src1, *dst;
    int vdt, act_variant, order;
    uint8_t* wdata;
    int64_t wrow;
    float* absterm;
    int exact;
} mm_ctx;

static void mm_convert(void* vctx, int64_t b, int64_t e) {
    mm_ctx* c = (mm_ctx*)vctx;
    const orc_tensor* s1 = c->src1;
    const int64_t K = s1->ne[0];
    float* tmp = (float*)malloc((size_t)K * 4);
    for (int64_t r = b; r < e; ++r) {
        const int64_t i11 = r % s1->ne[1];
        const int64_t i12 = (r / s1->ne[1]) % s1->ne[2];
        const int64_t i13 = r / (s1->ne[1] * s1->ne[2]);
        const uint8_t* row = (const uint8_t*)s1->data + i11 * s1->nb[1] + i12 * s1->nb[2] + i13 * s1->nb[3];
        uint8_t* out = c->wdata + r * c->wrow;
        if (s1->type == c->vdt && s1->nb[0] == orc_type_size(s1->type)) {
            memcpy(out, row, (size_t)c->wrow);
            continue;
        }
        for (int64_t k = 0; k < K; ++k) {
            const uint8_t* p = row + k * s1->nb[0];
            tmp[k] = s1->type == ORC_TYPE_F32 ? *(const float*)p : h2f(*(const uint16_t*)p);
        }
        orc_from_float(c->vdt, c->act_variant, tmp, out, K);
    }
    free(tmp);
}

static void mm_compute(void* vctx, int64_t b, int64_t e) {
    mm_ctx* c = (mm_ctx*)vctx;
    const orc_tensor *s0 = c->src0, *s1 = c->src1, *d = c->dst;
    const int64_t K = s0->ne[0], N = s0->ne[1];
    const int64_t r2 = s1->ne[2] / s0->ne[2], r3 = s1->ne[3] / s0->ne[3];
    for (int64_t r = b; r < e; ++r) {
        const int64_t i11 = r % s1->ne[1];
        const int64_t i12 = (r / s1->ne[1]) % s1->ne[2];
        const int64_t i13 = r / (s1->ne[1] * s1->ne[2]);
        const int64_t i02 = i12 / r2, i03 = i13 / r3;
        const uint8_t* y = c->wdata + r * c->wrow;
        uint8_t* drow = (uint8_t*)d->data + i11 * d->nb[1] + i12 * d->nb[2] + i13 * d->nb[3];
        for (int64_t n = 0; n < N; ++n) {
            const uint8_t* x = (const uint8_t*)s0->data + n * s0->nb[1] + i02 * s0->nb[2] + i03 * s0->nb[3];
            float v;
            if (c->exact) {
                long double a;
                v = (float)dot_exact_ld(s0->type, K, x, y, &a);
                if (c->absterm) c->absterm[r * N + n] = (float)a;
            } else {
                v = orc_vec_dot(s0->type, K, x, y, c->order);
            }
            *(float*)(drow + n * d->nb[0]) = v;
        }
    }
}

static int mm_run(const orc_tensor* src0, const orc_tensor* src1, const orc_tensor* dst,
                  int act_variant, int order, int n_threads, int exact, float* absterm) {
    const int vdt = orc_vec_dot_type(src0->type);
    if (vdt < 0) return -3;
    if (src1->type != ORC_TYPE_F32 && !(src1->type == ORC_TYPE_F16 && vdt == ORC_TYPE_F16)) return -3;
    if (dst->type != ORC_TYPE_F32) return -3;
    if (src1->ne[0] != src0->ne[0]) return -4;
    if (src0->ne[0] % orc_blck_size(src0->type) != 0) return -4;
    if (dst->ne[0] != src0->ne[1] || dst->ne[1] != src1->ne[1] || dst->ne[2] != src1->ne[2] ||
        dst->ne[3] != src1->ne[3]) return -4;
    if (src1->ne[2] % src0->ne[2] != 0 || src1->ne[3] % src0->ne[3] != 0) return -4;
    if (src0->nb[0] != orc_type_size(src0->type)) return -4;
    mm_ctx c;
    memset(&c, 0, sizeof(c));
    c.src0 = src0; c.src1 = src1; c.dst = dst; c.vdt = vdt; c.act_variant = act_variant; c.order = order;
    c.exact = exact; c.absterm = absterm;
    c.wrow = orc_row_size(vdt, src1->ne[0]);
    const int64_t rows = src1->ne[1] * src1->ne[2] * src1->ne[3];
    c.wdata = (uint8_t*)malloc((size_t)(rows * c.wrow));
    if (!c.wdata) return -2;
    parallel_for(rows, n_threads, mm_convert, &c);
    parallel_for(rows, n_threads, mm_compute, &c);
    free(c.wdata);
    return 0;
}

int orc_mul_mat(const orc_tensor* src0, const orc_tensor* src1, const orc_tensor* dst,
                int act_variant, int order, int n_threads) {
    return mm_run(src0, src1, dst, act_variant, order, n_threads, 0, NULL);
}

int orc_mul_mat_exact(const orc_tensor* src0, const orc_tensor* src1, const orc_tensor* dst,
                      float* absterm, int act_variant, int n_threads) {
    return mm_run(src0, src1, dst, act_variant, ORC_ORDER_SEQ, n_threads, 1, absterm);
}

/* ------------------------------------------------------------------ */
/* soft_max_ext (no mask, max_bias 0): wp = x*scale; m = max(wp);        */
/* e_i = expf(wp_i - m); sum in double; y = e_i * (float)(1/sum).        */
/* ------------------------------------------------------------------ */
typedef struct { const orc_tensor *src, *dst; float scale; } sm_ctx;

static void sm_rows(void* vctx, int64_t b, int64_t e) {
    sm_ctx* c = (sm_ctx*)vctx;
    const orc_tensor *s = c->src, *d = c->dst;
    const int64_t nc = s->ne[0];
    float* wp = (float*)malloc((size_t)nc * 4);
    for (int64_t r = b; r < e; ++r) {
        const int64_t i1 = r % s->ne[1], i2 = (r / s->ne[1]) % s->ne[2], i3 = r / (s->ne[1] * s->ne[2]);
        const uint8_t* sp = (const uint8_t*)s->data + i1 * s->nb[1] + i2 * s->nb[2] + i3 * s->nb[3];
        uint8_t* dp = (uint8_t*)d->data + i1 * d->nb[1] + i2 * d->nb[2] + i3 * d->nb[3];
        float mx = -INFINITY;
        for (int64_t i = 0; i < nc; ++i) {
            wp[i] = *(const float*)(sp + i * s->nb[0]) * c->scale;
            if (wp[i] > mx) mx = wp[i];
        }
        double sum = 0.0;
        for (int64_t i = 0; i < nc; ++i) {
            const float v = expf(wp[i] - mx);
            sum += (double)v;
            wp[i] = v;
        }
        const float inv = (float)(1.0 / sum);
        for (int64_t i = 0; i < nc; ++i) *(float*)(dp + i * d->nb[0]) = wp[i] * inv;
    }
    free(wp);
}

int orc_soft_max_ext(const orc_tensor* src, const orc_tensor* dst, float scale, int n_threads) {
    if (src->type != ORC_TYPE_F32 || dst->type != ORC_TYPE_F32) return -3;
    for (int i = 0; i < 4; ++i) if (src->ne[i] != dst->ne[i]) return -4;
    sm_ctx c = {src, dst, scale};
    parallel_for(src->ne[1] * src->ne[2] * src->ne[3], n_threads, sm_rows, &c);
    return 0;
}

/* ------------------------------------------------------------------ */
/* flash_attn_ext (ggml-cpu one-chunk loop, mask = NULL, max_bias = 0):  */
/*   Q row converted to K's vec_dot_type; s = dot(K_j, Q)*scale          */
/*   (softcap: s = softcap*tanhf(s)); online softmax with M, S:          */
/*     s > M: ms = expf(Mold - M), V acc *= ms; else vs = expf(s - M)    */
/*     V acc += V_j * vs;  S = S*ms + vs                                 */
/*   F16 V accumulates in fp16 (VKQ16), F32 V in fp32; out = acc/S,      */
/*   written at dst[:, head, iq, batch] ([Dv, n_head, n_q, batch]).      */
/* ------------------------------------------------------------------ */
typedef struct { const orc_tensor *q, *k, *v, *dst; float scale, softcap; int exact; } fa_ctx;

static inline float load_elem(const orc_tensor* t, const uint8_t* p) {
    return t->type == ORC_TYPE_F32 ? *(const float*)p : h2f(*(const uint16_t*)p);
}

static void fa_rows(void* vctx, int64_t b, int64_t e) {
    fa_ctx* c = (fa_ctx*)vctx;
    const orc_tensor *q = c->q, *k = c->k, *v = c->v, *d = c->dst;
    const int64_t D = q->ne[0], Dv = v->ne[0], nq = q->ne[1], nh = q->ne[2], nkv = k->ne[1];
    const int64_t rk2 = q->ne[2] / k->ne[2], rv2 = q->ne[2] / v->ne[2];
    float* qf = (float*)malloc((size_t)D * 4);
    float* kf = (float*)malloc((size_t)D * 4);
    float* acc = (float*)malloc((size_t)Dv * 4);
    uint16_t* acc16 = (uint16_t*)malloc((size_t)Dv * 2);
    long double* accl = (long double*)malloc((size_t)Dv * sizeof(long double));
    long double* sl = (long double*)malloc((size_t)nkv * sizeof(long double));
    for (int64_t r = b; r < e; ++r) {
        const int64_t iq1 = r % nq, iq2 = (r / nq) % nh, iq3 = r / (nq * nh);
        const int64_t ik2 = iq2 / rk2, iv2 = iq2 / rv2;
        const uint8_t* qp = (const uint8_t*)q->data + iq1 * q->nb[1] + iq2 * q->nb[2] + iq3 * q->nb[3];
        for (int64_t i = 0; i < D; ++i) {
            float x = load_elem(q, qp + i * q->nb[0]);
            if (k->type == ORC_TYPE_F16 && !c->exact) x = h2f(f2h(x)); /* q_to_vec_dot */
            qf[i] = x;
        }
        float* out = (float*)((uint8_t*)d->data + iq2 * d->nb[1] + iq1 * d->nb[2] + iq3 * d->nb[3]);
        if (c->exact) {
            long double mx = -INFINITY, S = 0.0L;
            for (int64_t j = 0; j < nkv; ++j) {
                const uint8_t* kp = (const uint8_t*)k->data + j * k->nb[1] + ik2 * k->nb[2] + iq3 * k->nb[3];
                long double s = 0.0L;
                for (int64_t i = 0; i < D; ++i) s += (long double)qf[i] * (long double)load_elem(k, kp + i * k->nb[0]);
                s *= (long double)c->scale;
                sl[j] = s;
                if (s > mx) mx = s;
            }
            for (int64_t i = 0; i < Dv; ++i) accl[i] = 0.0L;
            for (int64_t j = 0; j < nkv; ++j) {
                const long double p = expl(sl[j] - mx);
                S += p;
                const uint8_t* vp = (const uint8_t*)v->data + j * v->nb[1] + iv2 * v->nb[2] + iq3 * v->nb[3];
                for (int64_t i = 0; i < Dv; ++i) accl[i] += p * (long double)load_elem(v, vp + i * v->nb[0]);
            }
            for (int64_t i = 0; i < Dv; ++i) out[i] = (float)(accl[i] / S);
            continue;
        }
        float M = -INFINITY, S = 0.0f;
        const int v16 = v->type == ORC_TYPE_F16;
        for (int64_t i = 0; i < Dv; ++i) { acc[i] = 0.0f; acc16[i] = 0; }
        for (int64_t j = 0; j < nkv; ++j) {
            const uint8_t* kp = (const uint8_t*)k->data + j * k->nb[1] + ik2 * k->nb[2] + iq3 * k->nb[3];
            for (int64_t i = 0; i < D; ++i) kf[i] = load_elem(k, kp + i * k->nb[0]);
            float s = dot_vec_f32_like(D, kf, qf);
            s = s * c->scale;
            if (c->softcap != 0.0f) s = c->softcap * tanhf(s);
            const float Mold = M;
            float ms = 1.0f, vs = 1.0f;
            const uint8_t* vp = (const uint8_t*)v->data + j * v->nb[1] + iv2 * v->nb[2] + iq3 * v->nb[3];
            if (s > M) {
                M = s;
                ms = expf(Mold - M);
                if (v16) for (int64_t i = 0; i < Dv; ++i) acc16[i] = f2h(h2f(acc16[i]) * ms);
                else for (int64_t i = 0; i < Dv; ++i) acc[i] = acc[i] * ms;
            } else {
                vs = expf(s - M);
            }
            if (v16) for (int64_t i = 0; i < Dv; ++i)
                acc16[i] = f2h(fmaf(h2f(*(const uint16_t*)(vp + i * v->nb[0])), vs, h2f(acc16[i])));
            else for (int64_t i = 0; i < Dv; ++i)
                acc[i] = fmaf(*(const float*)(vp + i * v->nb[0]), vs, acc[i]);
            S = S * ms + vs;
        }
        if (v16) for (int64_t i = 0; i < Dv; ++i) acc[i] = h2f(acc16[i]);
        const float Sinv = S == 0.0f ? 0.0f : 1.0f / S;
        for (int64_t i = 0; i < Dv; ++i) out[i] = acc[i] * Sinv;
    }
    free(qf); free(kf); free(acc); free(acc16); free(accl); free(sl);
}

static int fa_check(const orc_tensor* q, const orc_tensor* k, const orc_tensor* v, const orc_tensor* dst) {
    if (dst->type != ORC_TYPE_F32) return -3;
    if (k->ne[0] != q->ne[0] || v->ne[1] != k->ne[1]) return -4;
    if (q->ne[2] % k->ne[2] != 0 || q->ne[2] % v->ne[2] != 0) return -4;
    if (dst->ne[0] != v->ne[0] || dst->ne[1] != q->ne[2] || dst->ne[2] != q->ne[1] || dst->ne[3] != q->ne[3]) return -4;
    return 0;
}

int orc_flash_attn_ext(const orc_tensor* q, const orc_tensor* k, const orc_tensor* v,
                       const orc_tensor* dst, float scale, float softcap, int n_threads) {
    const int rc = fa_check(q, k, v, dst);
    if (rc) return rc;
    fa_ctx c = {q, k, v, dst, scale, softcap, 0};
    parallel_for(q->ne[1] * q->ne[2] * q->ne[3], n_threads, fa_rows, &c);
    return 0;
}

int orc_attn_exact(const orc_tensor* q, const orc_tensor* k, const orc_tensor* v,
                   const orc_tensor* dst, float scale, int n_threads) {
    const int rc = fa_check(q, k, v, dst);
    if (rc) return rc;
    fa_ctx c = {q, k, v, dst, scale, 0.0f, 1};
    parallel_for(q->ne[1] * q->ne[2] * q->ne[3], n_threads, fa_rows, &c);
    return 0;
}

/* ------------------------------------------------------------------ */
/* ViT glue                                                              */
/* ------------------------------------------------------------------ */

/* ggml_norm: mean and variance accumulated in double, y = (x-mean)*(1/sqrt(var+eps)). */
void orc_norm_rows(const float* x, float* y, int64_t nrows, int64_t ne0, float eps) {
    for (int64_t r = 0; r < nrows; ++r) {
        const float* xr = x + r * ne0;
        float* yr = y + r * ne0;
        double sum = 0.0;
        for (int64_t i = 0; i < ne0; ++i) sum += (double)xr[i];
        const float mean = (float)(sum / (double)ne0);
        double sum2 = 0.0;
        for (int64_t i = 0; i < ne0; ++i) {
            const float v = xr[i] - mean;
            yr[i] = v;
            sum2 += (double)(v * v);
        }
        const float variance = (float)(sum2 / (double)ne0);
        const float scale = 1.0f / sqrtf(variance + eps);
        for (int64_t i = 0; i < ne0; ++i) yr[i] *= scale;
    }
}

/* ggml_gelu_erf: 0.5*x*(1 + erf(x/sqrt(2))). */
void orc_gelu_erf(const float* x, float* y, int64_t n) {
    const float s = 0.70710678118654752440f;
    for (int64_t i = 0; i < n; ++i) {
        const float v = x[i];
        y[i] = 0.5f * v * (1.0f + erff(v * s));
    }
}

/* ggml_gelu (tanh form), as ggml-cpu evaluates it with GGML_GELU_FP16: for
 * x <= -10 the result is 0, for x >= 10 it is x, otherwise the fp16 table
 * entry of f16(x): f16(gelu_f32(f16(x))) with
 *   gelu_f32(v) = 0.5*v*(1 + tanh(sqrt(2/pi)*v*(1 + 0.044715*v*v)))
 * evaluated left to right in fp32 (used by the Hiera MLP, sam3.cpp:4453). */
static float gelu_tanh_f32(float v) {
    const float c = 0.79788456080286535587989211986876f, a = 0.044715f;
    const float inner = c * v * (1.0f + a * v * v);
    return 0.5f * v * (1.0f + tanhf(inner));
}
void orc_gelu_tanh(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        const float v = x[i];
        if (v <= -10.0f) y[i] = 0.0f;
        else if (v >= 10.0f) y[i] = v;
        else y[i] = h2f(f2h(gelu_tanh_f32(h2f(f2h(v)))));
    }
}

/* sam2_window_partition (sam3.cpp:4194-4232): x [H][W][C] (ggml [C, W, H]) zero-padded
 * to Hp, Wp (multiples of ws) -> [nW][ws][ws][C], window n = wh + nW_h * ww (the
 * H-major order the reshape sequence produces), token (lh, lw) at lh*ws + lw. */
void orc_hiera_win_part(const float* x, float* y, int64_t C, int64_t W, int64_t H, int ws) {
    const int64_t Wp = (W + ws - 1) / ws * ws, Hp = (H + ws - 1) / ws * ws;
    const int64_t nwh = Hp / ws, nww = Wp / ws;
    for (int64_t ww = 0; ww < nww; ++ww)
        for (int64_t wh = 0; wh < nwh; ++wh)
            for (int64_t lh = 0; lh < ws; ++lh)
                for (int64_t lw = 0; lw < ws; ++lw) {
                    const int64_t n = wh + nwh * ww;
                    float* o = y + ((n * ws + lh) * ws + lw) * C;
                    const int64_t h = wh * ws + lh, w = ww * ws + lw;
                    if (h < H && w < W) memcpy(o, x + (h * W + w) * C, (size_t)C * 4);
                    else memset(o, 0, (size_t)C * 4);
                }
}

/* sam2_window_unpartition (sam3.cpp:4234-4281): inverse of the above for windows of ws
 * over a padded Hp x Wp grid, cropped to H x W. */
void orc_hiera_win_unpart(const float* x, float* y, int64_t C, int64_t W, int64_t H, int ws) {
    const int64_t Hp = (H + ws - 1) / ws * ws;
    const int64_t nwh = Hp / ws;
    for (int64_t h = 0; h < H; ++h)
        for (int64_t w = 0; w < W; ++w) {
            const int64_t n = h / ws + nwh * (w / ws);
            memcpy(y + (h * W + w) * C, x + ((n * ws + h % ws) * ws + w % ws) * C, (size_t)C * 4);
        }
}

/* sam2_maxpool_2d (sam3.cpp:4286-4296): ggml_pool_2d MAX, kernel 2, stride 2, no
 * padding, over x [B][H][W][C] -> [B][H/2][W/2][C]. */
void orc_maxpool2(const float* x, float* y, int64_t C, int64_t W, int64_t H, int64_t B) {
    const int64_t W2 = W / 2, H2 = H / 2;
    for (int64_t b = 0; b < B; ++b)
        for (int64_t h = 0; h < H2; ++h)
            for (int64_t w = 0; w < W2; ++w)
                for (int64_t c = 0; c < C; ++c) {
                    const float* p = x + ((b * H + 2 * h) * W + 2 * w) * C + c;
                    float m = p[0];
                    const float v1 = p[C], v2 = p[W * C], v3 = p[W * C + C];
                    if (v1 > m) m = v1;
                    if (v2 > m) m = v2;
                    if (v3 > m) m = v3;
                    y[((b * H2 + h) * W2 + w) * C + c] = m;
                }
}

/* sam2_bicubic_interpolate_cpu + sam2_compute_pos_embed (sam3.cpp:4076-4157):
 * Keys cubic convolution (a = -0.75), half-pixel source coordinates
 * fy = (y + 0.5) * H_in / H_out - 0.5, taps clamped to the border, summed
 * val += wy * wx * src in tap order (rows outer), plus the window table tiled
 * modulo ws.  bkg [E][bh][bw] and win [E][ws][ws] are CHW; out is token-major
 * [H*W][E] (ggml [E, W, H]). */
static float keys_cubic(float x) {
    x = fabsf(x);
    if (x < 1.0f) return (1.25f * x - 2.25f) * x * x + 1.0f;
    if (x < 2.0f) return ((-0.75f * x + 3.75f) * x - 6.0f) * x + 3.0f;
    return 0.0f;
}

void orc_sam2_pos_embed(const float* bkg, int E, int bh, int bw, const float* win, int ws, int H, int W, float* out) {
    for (int e = 0; e < E; ++e)
        for (int y = 0; y < H; ++y) {
            const float fy = ((float)y + 0.5f) * (float)bh / (float)H - 0.5f;
            const int iy = (int)floorf(fy);
            const float dy = fy - (float)iy;
            for (int x = 0; x < W; ++x) {
                const float fx = ((float)x + 0.5f) * (float)bw / (float)W - 0.5f;
                const int ix = (int)floorf(fx);
                const float dx = fx - (float)ix;
                float val = 0.0f;
                for (int jj = -1; jj <= 2; ++jj) {
                    const float wy = keys_cubic(dy - (float)jj);
                    int sy = iy + jj;
                    sy = sy < 0 ? 0 : sy > bh - 1 ? bh - 1 : sy;
                    for (int ii = -1; ii <= 2; ++ii) {
                        const float wx = keys_cubic(dx - (float)ii);
                        int sx = ix + ii;
                        sx = sx < 0 ? 0 : sx > bw - 1 ? bw - 1 : sx;
                        val += wy * wx * bkg[((int64_t)e * bh + sy) * bw + sx];
                    }
                }
                const float t = win[((int64_t)e * ws + y % ws) * ws + x % ws];
                out[((int64_t)y * W + x) * E + e] = val + t;
            }
        }
}

/* sam3.cpp:3559-3590: freqs[i] = 1/theta^(4i/dim), i < dim/4; token idx at
 * (x = idx % end_x, y = idx / end_x) * scale_pos; pairs 0..dim/4-1 from x,
 * the next dim/4 pairs from y, each stored (cos, sin). */
void orc_compute_axial_cis(float* out, int dim, int end_x, int end_y, float theta, float scale_pos) {
    const int half_dim = dim / 4;
    float freqs[256];
    for (int i = 0; i < half_dim; ++i) freqs[i] = 1.0f / powf(theta, (float)(i * 4) / (float)dim);
    const int n = end_x * end_y;
    for (int idx = 0; idx < n; ++idx) {
        const float tx = (float)(idx % end_x) * scale_pos;
        const float ty = (float)(idx / end_x) * scale_pos;
        for (int i = 0; i < half_dim; ++i) {
            const float ax = tx * freqs[i];
            out[(int64_t)idx * dim + i * 2 + 0] = cosf(ax);
            out[(int64_t)idx * dim + i * 2 + 1] = sinf(ax);
        }
        for (int i = 0; i < half_dim; ++i) {
            const float ay = ty * freqs[i];
            out[(int64_t)idx * dim + half_dim * 2 + i * 2 + 0] = cosf(ay);
            out[(int64_t)idx * dim + half_dim * 2 + i * 2 + 1] = sinf(ay);
        }
    }
}

/* sam3.cpp:3671-3710: per pair (re, im) = (x[2i], x[2i+1]) and (c, s):
 * out_re = re*c - im*s, out_im = re*s + im*c, each product rounded (separate
 * ggml_mul nodes) before the ggml_sub / ggml_add. */
void orc_apply_rope(float* x, const float* freqs, int64_t hd, int64_t n_tok, int64_t n_rows3) {
    const int64_t half = hd / 2;
    for (int64_t h = 0; h < n_rows3; ++h) {
        for (int64_t t = 0; t < n_tok; ++t) {
            float* row = x + (h * n_tok + t) * hd;
            const float* f = freqs + t * hd;
            for (int64_t i = 0; i < half; ++i) {
                const float re = row[2 * i], im = row[2 * i + 1];
                const float c = f[2 * i], s = f[2 * i + 1];
                const float a = re * c, b2 = im * s, p = re * s, q = im * c;
                row[2 * i] = a - b2;
                row[2 * i + 1] = p + q;
            }
        }
    }
}

/* ggml_win_part on [C, W, H, 1] with window w: output [C, w, w, npx*npy],
 * window index py*npx + px, zero padding outside the image. */
void orc_win_part(const float* src, float* dst, int64_t C, int64_t W, int64_t H, int w) {
    const int64_t npx = (W + w - 1) / w, npy = (H + w - 1) / w;
    for (int64_t py = 0; py < npy; ++py)
        for (int64_t px = 0; px < npx; ++px)
            for (int64_t i2 = 0; i2 < w; ++i2)
                for (int64_t i1 = 0; i1 < w; ++i1) {
                    const int64_t i3 = py * npx + px;
                    float* o = dst + ((i3 * w + i2) * w + i1) * C;
                    const int64_t y = py * w + i2, xx = px * w + i1;
                    if (y >= H || xx >= W) { for (int64_t c = 0; c < C; ++c) o[c] = 0.0f; }
                    else memcpy(o, src + (y * W + xx) * C, (size_t)C * 4);
                }
}

/* ggml_win_unpart: inverse of win_part, cropping the padding. */
void orc_win_unpart(const float* src, float* dst, int64_t C, int64_t W, int64_t H, int w) {
    const int64_t npx = (W + w - 1) / w;
    for (int64_t y = 0; y < H; ++y)
        for (int64_t xx = 0; xx < W; ++xx) {
            const int64_t py = y / w, px = xx / w, i2 = y % w, i1 = xx % w;
            const int64_t i3 = py * npx + px;
            memcpy(dst + (y * W + xx) * C, src + ((i3 * w + i2) * w + i1) * C, (size_t)C * 4);
        }
}
