// Device-side building blocks shared by the gfx950 kernels: ggml block
// formats, fp16 conversion, wavefront reductions and MFMA operand types.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace mi355 {

constexpr int QK = 32;  // elements per quantized block (ggml QK8_0 = QK4_0 = 32)

// ggml-common.h block layouts, little-endian, packed.
struct __attribute__((packed)) blk_q8_0 { uint16_t d; int8_t qs[32]; };
struct __attribute__((packed)) blk_q8_1 { uint16_t d; uint16_t s; int8_t qs[32]; };
struct __attribute__((packed)) blk_q4_0 { uint16_t d; uint8_t qs[16]; };
struct __attribute__((packed)) blk_q4_1 { uint16_t d; uint16_t m; uint8_t qs[16]; };
static_assert(sizeof(blk_q8_0) == 34, "q8_0");
static_assert(sizeof(blk_q8_1) == 36, "q8_1");
static_assert(sizeof(blk_q4_0) == 18, "q4_0");
static_assert(sizeof(blk_q4_1) == 20, "q4_1");

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));

// fp16 <-> fp32.  v_cvt_f16_f32 rounds to nearest even under the default
// MODE; fp16 denormals are kept (HIP's default f16/f64 denormal mode).
__device__ __forceinline__ float h2f(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float)v;
}
// The empty asm makes f an opaque, already-rounded fp32 value: without it the
// backend may fold a producing multiply into the conversion (v_fma_mixlo_f16,
// one rounding of the exact product), while ggml rounds the product to fp32
// first, e.g. the Q8_1 sum s = fp16(d * isum) differs when d * isum in fp32
// lands on an fp16 midpoint.
__device__ __forceinline__ uint16_t f2h(float f) {
    asm volatile("" : "+v"(f));
    _Float16 v = (_Float16)f;
    uint16_t h;
    __builtin_memcpy(&h, &v, 2);
    return h;
}

// Raw buffer resource over [base, base + bytes) (stride 0, gfx9 dword3 =
// 0x00020000): offsets at or past the end read as zero.
__device__ __forceinline__ v4i make_rsrc(const void* base, int64_t bytes) {
    const int32_t n = bytes <= 0 ? 0 : (bytes > 0x7fffffffLL ? 0x7fffffff : (int32_t)bytes);
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    return v4i{(int)(uint32_t)a, (int)((uint32_t)(a >> 32) & 0xffffu), n, 0x00020000};
}

// buffer_load ... lds: lane i's 4 (or 16) bytes at voffset land at LDS byte
// address M0 + 4*i (16*i).  Issued from inline asm so the compiler's wait
// insertion does not track them: it cannot tell one stage buffer from another
// and would otherwise wait for every DMA in flight before the first LDS read.
// The kernel orders them itself (vmcnt waits + barrier).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
__device__ __forceinline__ void dma_b32(v4i rsrc, const void* lds, int voff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(lds_addr(lds))), "v"(voff), "s"(rsrc)
                 : "memory", "m0");
}
__device__ __forceinline__ void dma_b128(v4i rsrc, const void* lds, int voff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(lds_addr(lds))), "v"(voff), "s"(rsrc)
                 : "memory", "m0");
}
// The same with the LDS byte address already computed (m0, wave-uniform) and a
// wave-uniform byte offset soff added in the instruction's SGPR offset field,
// so a loop that walks K moves one SGPR instead of rebuilding descriptors.
// Callers keep voff + soff inside the descriptor's records for every lane that
// must load, and send a voff at or past the records (OOB) for lanes that must
// read zero, so either range-check convention (with or without soff) agrees.
__device__ __forceinline__ void dma_b32_so(v4i rsrc, uint32_t m0, int voff, int soff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, %3 offen lds"
                 :
                 : "s"(m0), "v"(voff), "s"(rsrc), "s"(soff)
                 : "memory", "m0");
}
__device__ __forceinline__ void dma_b128_so(v4i rsrc, uint32_t m0, int voff, int soff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(m0), "v"(voff), "s"(rsrc), "s"(soff)
                 : "memory", "m0");
}

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt[3:0] | vmcnt[5:4] << 14, expcnt and
// lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Lane exchanges without the LDS pipe: step S returns the value of the lane paired with
// this one, S = 1: lane ^ 1 and S = 2: lane ^ 2 (DPP quad_perm), S = 4: lane 7 - lane within
// its eight (DPP row_half_mirror), S = 8: lane 15 - lane within its sixteen (DPP row_mirror),
// S = 16: lane ^ 16 (v_permlane16_swap), S = 32: lane ^ 32 (v_permlane32_swap).  Applied in
// the order 1, 2, 4, 8, 16, 32 they form a butterfly over aligned groups of lanes: after the
// steps below 2^k every lane of a 2^k group holds the same value, so the mirror steps pair
// lanes of different halves.  Every lane of a group must be active.
template <int S>
__device__ __forceinline__ int lane_swap(int v) {
    if constexpr (S == 1) return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);
    else if constexpr (S == 2) return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);
    else if constexpr (S == 4) return __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, false);
    else if constexpr (S == 8) return __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, false);
    else if constexpr (S == 16) {
        // odd 16-lane rows of the first operand swap with even rows of the second
        const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (__lane_id() & 16) ? (int)p[0] : (int)p[1];
    } else {
        static_assert(S == 32, "lane_swap step");
        // lanes 32..63 of the first operand swap with lanes 0..31 of the second
        const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (__lane_id() & 32) ? (int)p[0] : (int)p[1];
    }
}
template <int S>
__device__ __forceinline__ float lane_swap_f(float v) {
    return __int_as_float(lane_swap<S>(__float_as_int(v)));
}
template <int S>
__device__ __forceinline__ double lane_swap_d(double v) {
    const long long b = __double_as_longlong(v);
    const int lo = lane_swap<S>((int)(b & 0xffffffffLL)), hi = lane_swap<S>((int)(b >> 32));
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

// LDS staging of a 32x32 fp32 MFMA tile in 1024 floats: rows 2k and 2k + 1 share the 64
// floats (one line of the 64 4-byte banks) at 64 k, row r in half (r ^ r >> 2) & 1, so a write
// of one accumulator element (lanes 0..31 row R, lanes 32..63 row R + 4) and each 16-lane
// quarter of a float4 row read (rows 2k, 2k + 1) cover all 64 banks.
__device__ __forceinline__ int tile32_row(int r) { return 64 * (r >> 1) + 32 * ((r ^ (r >> 2)) & 1); }

// Butterfly max / integer sum across `width` consecutive aligned lanes (a power of two
// <= 64); exact, so the lane order does not matter.
template <int width>
__device__ __forceinline__ float group_max(float v) {
    if constexpr (width >= 2) v = fmaxf(v, lane_swap_f<1>(v));
    if constexpr (width >= 4) v = fmaxf(v, lane_swap_f<2>(v));
    if constexpr (width >= 8) v = fmaxf(v, lane_swap_f<4>(v));
    if constexpr (width >= 16) v = fmaxf(v, lane_swap_f<8>(v));
    if constexpr (width >= 32) v = fmaxf(v, lane_swap_f<16>(v));
    if constexpr (width >= 64) v = fmaxf(v, lane_swap_f<32>(v));
    return v;
}
template <int width>
__device__ __forceinline__ int group_sum_i(int v) {
    if constexpr (width >= 2) v += lane_swap<1>(v);
    if constexpr (width >= 4) v += lane_swap<2>(v);
    if constexpr (width >= 8) v += lane_swap<4>(v);
    if constexpr (width >= 16) v += lane_swap<8>(v);
    if constexpr (width >= 32) v += lane_swap<16>(v);
    if constexpr (width >= 64) v += lane_swap<32>(v);
    return v;
}
// Double sum over aligned groups of G lanes (G a wavefront-uniform power of two <= 64).
__device__ __forceinline__ double group_sum_d(double v, int G) {
    if (G >= 2) v += lane_swap_d<1>(v);
    if (G >= 4) v += lane_swap_d<2>(v);
    if (G >= 8) v += lane_swap_d<4>(v);
    if (G >= 16) v += lane_swap_d<8>(v);
    if (G >= 32) v += lane_swap_d<16>(v);
    if (G >= 64) v += lane_swap_d<32>(v);
    return v;
}
// Float sum through ds_bpermute in a fixed order (largest distance first).
template <int width>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = width / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, width);
    return v;
}

// ---- activation producers that feed a MUL_MAT (ActOut, kernels.h)
// ggml from_float x86 of 32-value blocks (d = amax/127, id = 127/amax, round
// half to even), or F16 / F32 rows.  A lane holds 4 consecutive values, chunk
// c of the row (elements 4c..4c+3); the 8 lanes holding chunks 8k..8k+7 (lanes
// congruent to them mod 8, all active) hold one block and reduce it together.
// Scale (and Q8_1 sum) of block b of a quantized operand row, with the padding
// slot of the last block: fp16 [row][dp] for the fp16-MFMA operand, the dl / dh
// dword arrays for the int8 one.
__device__ __forceinline__ void act_store_scale(const ActOut& o, int64_t row, int64_t K, int64_t b, float d, int isum) {
    const int64_t nb = K / 32;
    if (o.mode >= ACT_I8) {
        uint32_t* dl = reinterpret_cast<uint32_t*>(o.d);
        const int64_t i = row * (o.dp / 2) + b / 2;
        if ((b & 1) == 0) dl[i] = (uint32_t)f2h(d);
        else o.dh[i] = (uint32_t)f2h(d) << 16;
        if (b == nb - 1 && (nb & 1)) o.dh[i] = 0;  // the missing odd block of an odd count
    } else {
        o.d[row * o.dp + b] = f2h(d);
        if (b == nb - 1 && o.dp > nb) o.d[row * o.dp + b + 1] = 0;  // the even-pitch padding slot
    }
    if (act_has_sums(o.mode)) {
        o.s[row * o.dp + b] = f2h(d * (float)isum);
        if (b == nb - 1 && o.dp > nb) o.s[row * o.dp + b + 1] = 0;
    }
}

// Four consecutive values (chunk c of a row of K) into the operand; for the
// quantized modes the 8 lanes holding chunks 8j .. 8j + 7 are consecutive
// lanes of one group and quantize block j together (ggml from_float, x86).
__device__ __forceinline__ void act_store_chunk(const ActOut& o, int64_t row, int64_t K, int64_t c, v4f x) {
    if (o.mode == ACT_F32) {
        *reinterpret_cast<v4f*>(o.y + row * K + 4 * c) = x;
        return;
    }
    if (o.mode == ACT_F16) {
        const uint32_t h0 = (uint32_t)f2h(x[0]) | ((uint32_t)f2h(x[1]) << 16);
        const uint32_t h1 = (uint32_t)f2h(x[2]) | ((uint32_t)f2h(x[3]) << 16);
        *reinterpret_cast<uint2*>(o.q + row * K + 4 * c) = make_uint2(h0, h1);
        return;
    }
    float amax = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
    amax = group_max<8>(amax);
    const float d = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    const int q0 = (int)rintf(x[0] * id), q1 = (int)rintf(x[1] * id);
    const int q2 = (int)rintf(x[2] * id), q3 = (int)rintf(x[3] * id);
    int isum = 0;
    if (act_has_sums(o.mode)) isum = group_sum_i<8>(q0 + q1 + q2 + q3);
    if ((c & 7) == 0) act_store_scale(o, row, K, c >> 3, d, isum);
    if (o.mode >= ACT_I8) {
        const uint32_t b4 = (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) | ((uint32_t)(q2 & 0xff) << 16) |
                            ((uint32_t)(q3 & 0xff) << 24);
        *reinterpret_cast<uint32_t*>(reinterpret_cast<int8_t*>(o.q) + row * K + 4 * c) = b4;
    } else {
        const uint32_t h0 = (uint32_t)f2h((float)q0) | ((uint32_t)f2h((float)q1) << 16);
        const uint32_t h1 = (uint32_t)f2h((float)q2) | ((uint32_t)f2h((float)q3) << 16);
        *reinterpret_cast<uint2*>(o.q + row * K + 4 * c) = make_uint2(h0, h1);
    }
}

// Sixteen consecutive values (half-block h of a row of K: elements 16h .. 16h + 15) into
// the operand; the lanes holding half-blocks 2k and 2k + 1 are adjacent lanes 2j, 2j + 1 of
// one wavefront, both active, and quantize block k together: one DPP swap gives the block
// max, d, id and the quants are act_store_chunk's (ggml from_float, x86).
__device__ __forceinline__ void act_store_half16(const ActOut& o, int64_t row, int64_t K, int h, const float (&x)[16]) {
    if (o.mode == ACT_F32) {
        float* y = o.y + row * K + 16 * h;
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<v4f*>(y + 4 * i) = v4f{x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]};
        return;
    }
    if (o.mode == ACT_F16) {
        uint32_t hw[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) hw[i] = (uint32_t)f2h(x[2 * i]) | ((uint32_t)f2h(x[2 * i + 1]) << 16);
        uint4* dst = reinterpret_cast<uint4*>(o.q + row * K + 16 * h);
        dst[0] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        dst[1] = make_uint4(hw[4], hw[5], hw[6], hw[7]);
        return;
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(x[i]));
    // quad_perm [1, 0, 3, 2]: the lane holding the other half of this block
    amax = fmaxf(amax, lane_swap_f<1>(amax));
    const float d = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    int q[16], isum = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        q[i] = (int)rintf(x[i] * id);
        isum += q[i];
    }
    if (act_has_sums(o.mode)) isum += lane_swap<1>(isum);
    if (o.mode >= ACT_I8) {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            w[i] = (uint32_t)(q[4 * i] & 0xff) | ((uint32_t)(q[4 * i + 1] & 0xff) << 8) |
                   ((uint32_t)(q[4 * i + 2] & 0xff) << 16) | ((uint32_t)(q[4 * i + 3] & 0xff) << 24);
        *reinterpret_cast<uint4*>(reinterpret_cast<int8_t*>(o.q) + row * K + 16 * h) = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
        uint32_t hw[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) hw[i] = (uint32_t)f2h((float)q[2 * i]) | ((uint32_t)f2h((float)q[2 * i + 1]) << 16);
        uint4* dst = reinterpret_cast<uint4*>(o.q + row * K + 16 * h);
        dst[0] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        dst[1] = make_uint4(hw[4], hw[5], hw[6], hw[7]);
    }
    if ((h & 1) == 0) act_store_scale(o, row, K, h >> 1, d, isum);
}

// ggml_norm -> mul(w) -> add(b) of one row of C held by a group of G lanes
// (G a power of two, aligned), lane l holding chunks v*G + l, v < V (C = 4*G*V),
// or with CONTIG chunks l*V + v (4V consecutive values per lane).
// Sums in double as ggml_float; every step rounds to fp32 (callers compile
// without FMA contraction).
template <int V, bool CONTIG = false>
__device__ __forceinline__ void ln_group(v4f (&x)[V], int l, int G, int C, const float* w, const float* b, float eps) {
    // the affine rows are loaded up front, so their latency overlaps the reductions
    v4f wv[V], bv[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
        const int c = CONTIG ? l * V + v : v * G + l;
        wv[v] = w ? *reinterpret_cast<const v4f*>(w + 4 * c) : v4f{1.0f, 1.0f, 1.0f, 1.0f};
        bv[v] = b ? *reinterpret_cast<const v4f*>(b + 4 * c) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
    double s = 0.0;
#pragma unroll
    for (int v = 0; v < V; ++v)
#pragma unroll
        for (int i = 0; i < 4; ++i) s += (double)x[v][i];
    s = group_sum_d(s, G);
    const float mean = (float)(s / (double)C);
    double s2 = 0.0;
#pragma unroll
    for (int v = 0; v < V; ++v)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float t = x[v][i] - mean;
            x[v][i] = t;
            s2 += (double)(t * t);
        }
    s2 = group_sum_d(s2, G);
    const float var = (float)(s2 / (double)C);
    const float scale = 1.0f / sqrtf(var + eps);
#pragma unroll
    for (int v = 0; v < V; ++v) {
        v4f t = x[v] * scale;
        if (w) t = t * wv[v];
        if (b) t = t + bv[v];
        x[v] = t;
    }
}

// lanes per row G (largest power of two <= 64 dividing C/4) and chunks per
// lane V = C/(4G) for the grouped LayerNorm; V > 8 means the row does not fit
inline void ln_shape(int C, int* G, int* V) {
    int g = 1;
    while (g < 64 && (C / 4) % (2 * g) == 0) g *= 2;
    *G = g;
    *V = C % 4 == 0 ? C / (4 * g) : 1 << 30;
}

// Lane-per-element variant for rows the grouped form does not fit: element
// e = 32*blk + (lane & 31) of the row, the 32 lanes of a wavefront half
// holding one block (all 64 lanes call it; valid = false lanes hold no
// element and contribute 0).
__device__ __forceinline__ void act_store_lane32(const ActOut& o, int64_t row, int64_t K, int e, float v, bool valid) {
    if (o.mode == ACT_F32) {
        if (valid) o.y[row * K + e] = v;
        return;
    }
    if (o.mode == ACT_F16) {
        if (valid) o.q[row * K + e] = f2h(v);
        return;
    }
    const float amax = group_max<32>(valid ? fabsf(v) : 0.0f);
    const float d = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    const int q = valid ? (int)rintf(v * id) : 0;
    int isum = 0;
    if (act_has_sums(o.mode)) isum = group_sum_i<32>(q);
    if (valid) {
        if (o.mode >= ACT_I8) reinterpret_cast<int8_t*>(o.q)[row * K + e] = (int8_t)q;
        else o.q[row * K + e] = f2h((float)q);
        if ((e & 31) == 0) act_store_scale(o, row, K, e / 32, d, isum);
    }
}

// ---- elementwise functions shared by the fused passes and GEMM epilogues
// (each step rounds to fp32 as its ggml node does: no FMA contraction)

// erf for gelu_erf, in two pieces fitted for this kernel set (least squares, float32
// coefficients), a = min(|z|, 4):
//   a < 1:  a * c0 + a * P(a^2)                  c0 = 2/sqrt(pi) in float32, P of degree 6
//                                                (its constant term absorbs c0's rounding)
//   a >= 1: 1 - 2^-(a^2 log2(e) + S(a - 2.5))     S of degree 6 (erfc = 2^-Q, Q - a^2 log2 e
//                                                smooth), so erf(4) rounds to 1
// with the sign of z.  Absolute error below 9e-8 against erf (1.5 ulp of 0.84, where the
// pieces meet) over every float32, also with the hardware exp2 one ulp off either way:
// about 24 VALU operations against the library erff's 45 or so.  A NaN z gives +-1;
// gelu_erf's factor 0.5 z carries the NaN.
__device__ __forceinline__ float erf_gelu(float z) {
    const float a = fminf(fabsf(z), 4.0f);
    const float t = a * a;
    float p = 7.74653236e-05f;
    p = __builtin_fmaf(p, t, -0.000797281682f);
    p = __builtin_fmaf(p, t, 0.00518331816f);
    p = __builtin_fmaf(p, t, -0.0268505849f);
    p = __builtin_fmaf(p, t, 0.112834841f);
    p = __builtin_fmaf(p, t, -0.376126111f);
    p = __builtin_fmaf(p, t, -6.53512657e-08f);
    const float ea = __builtin_fmaf(a, 1.12837923f, a * p);
    const float x = a - 2.5f;
    float s = -0.00026368018f;
    s = __builtin_fmaf(s, x, 0.000243758739f);
    s = __builtin_fmaf(s, x, -0.00351444748f);
    s = __builtin_fmaf(s, x, 0.015484035f);
    s = __builtin_fmaf(s, x, -0.0809532776f);
    s = __builtin_fmaf(s, x, 0.508827448f);
    s = __builtin_fmaf(s, x, 2.24601269f);
    const float q = __builtin_fmaf(t, 1.44269502f, s);
    const float eb = 1.0f - __builtin_amdgcn_exp2f(-q);
    return __builtin_copysignf(a < 1.0f ? ea : eb, z);
}

// ggml_vec_gelu_erf_f32: 0.5*x*(1 + erf(x/sqrt(2))), erf by erf_gelu
__device__ __forceinline__ float gelu_erf(float u) {
#pragma clang fp contract(off)
    const float hx = 0.5f * u;
    return hx * (1.0f + erf_gelu(u * 0.70710678118654752440f));
}

// ggml_gelu with ggml-cpu's fp16-table semantics (GGML_GELU_FP16): 0 for x <= -10, x for
// x >= 10, else f16(gelu_f32(f16(x))), gelu_f32 evaluated left to right in fp32
__device__ __forceinline__ float gelu_tanh_table(float u) {
#pragma clang fp contract(off)
    if (u <= -10.0f) return 0.0f;
    if (u >= 10.0f) return u;
    const float v = h2f(f2h(u));
    const float inner0 = 0.79788456080286535587989211986876f * v;
    const float av = 0.044715f * v;
    const float avv = av * v;
    const float inner = inner0 * (1.0f + avv);
    const float hv = 0.5f * v;
    return h2f(f2h(hv * (1.0f + tanhf(inner))));
}

// sam3_apply_rope on one (x[2i], x[2i+1]) pair: the complex product with
// (cos, sin), each product rounded to fp32 before the add / subtract
__device__ __forceinline__ void rope_pair(float& x0, float& x1, float c, float s) {
#pragma clang fp contract(off)
    const float a = x0 * c, b = x1 * s, cc = x0 * s, d = x1 * c;
    x0 = a - b;
    x1 = cc + d;
}

// SAM2 window order (sam2_window_partition over the zero-padded grid: window
// n = wh + nwh*ww, token lh*ws + lw inside it) row r -> image token h*W + w,
// or -1 for a padding token
__device__ __forceinline__ int64_t hwin_src(int64_t r, int W, int H, int ws, int nwh) {
    const int64_t n = r / (ws * ws);
    const int loc = (int)(r - n * ws * ws);
    const int lh = loc / ws, lw = loc % ws;
    const int wh = (int)(n % nwh), ww = (int)(n / nwh);
    const int h = wh * ws + lh, w = ww * ws + lw;
    return (h < H && w < W) ? (int64_t)h * W + w : -1;
}

// ggml_win_part order over a W x W grid (windows row-major, W % ws == 0) row r
// -> image token y*W + x
__device__ __forceinline__ int64_t win_unpart_row(int64_t r, int W, int ws) {
    const int64_t n = r / (ws * ws);
    const int loc = (int)(r - n * ws * ws);
    const int nwx = W / ws;
    const int y = (int)(n / nwx) * ws + loc / ws, x = (int)(n % nwx) * ws + loc % ws;
    return (int64_t)y * W + x;
}

// a / b, and a % b in rem, for a >= 0, b > 0, a + b < 2^31, given rb = 1.0 / b: the double
// product a * rb lies within 2^-21 of a / b, so its truncation is the quotient or one off
// either way, and one correction step makes it exact.  A handful of instructions against
// the thirty-odd of a 32-bit integer division by a runtime divisor.
__device__ __forceinline__ int div_rcp(int a, int b, double rb, int& rem) {
    int q = (int)((double)a * rb);
    int r = a - q * b;
    if (r < 0) {
        --q;
        r += b;
    } else if (r >= b) {
        ++q;
        r -= b;
    }
    rem = r;
    return q;
}

// The reciprocals map_row32 divides by, computed once per thread
struct RowMapRcp {
    double w2, ws, nw;
};
__device__ __forceinline__ RowMapRcp rowmap_rcp(const RowMap& rm) {
    RowMapRcp c{0.0, 0.0, 0.0};
    if (rm.kind == ROWMAP_IDENTITY) return c;
    c.w2 = 1.0 / (double)(rm.ws * rm.ws);
    c.ws = 1.0 / (double)rm.ws;
    c.nw = 1.0 / (double)(rm.kind == ROWMAP_WIN_UNPART ? rm.W / rm.ws : rm.nwh);
    return c;
}
// map_row32 for rows below 2^30 through div_rcp (the same rows)
__device__ __forceinline__ int map_row32(const RowMap& rm, const RowMapRcp& rc, int r) {
    if (rm.kind == ROWMAP_IDENTITY) return r;
    int loc, lx, sub;
    const int n = div_rcp(r, rm.ws * rm.ws, rc.w2, loc), ly = div_rcp(loc, rm.ws, rc.ws, lx);
    if (rm.kind == ROWMAP_WIN_UNPART) {
        const int wy = div_rcp(n, rm.W / rm.ws, rc.nw, sub);  // sub = wx
        return (wy * rm.ws + ly) * rm.W + sub * rm.ws + lx;
    }
    const int ww = div_rcp(n, rm.nwh, rc.nw, sub);  // sub = wh; SAM2: window n = wh + nwh*ww
    const int h = sub * rm.ws + ly, w = ww * rm.ws + lx;
    return (h < rm.H && w < rm.W) ? h * rm.W + w : -1;
}

// map_row for rows and grids below 2^31 (32-bit index arithmetic)
__device__ __forceinline__ int map_row32(const RowMap& rm, int r) {
    if (rm.kind == ROWMAP_IDENTITY) return r;
    const int w2 = rm.ws * rm.ws, n = r / w2, loc = r - n * w2, ly = loc / rm.ws, lx = loc - ly * rm.ws;
    if (rm.kind == ROWMAP_WIN_UNPART) {
        const int nwx = rm.W / rm.ws, wy = n / nwx, wx = n - wy * nwx;
        return (wy * rm.ws + ly) * rm.W + wx * rm.ws + lx;
    }
    const int ww = n / rm.nwh, wh = n - ww * rm.nwh;  // SAM2: window n = wh + nwh*ww
    const int h = wh * rm.ws + ly, w = ww * rm.ws + lx;
    return (h < rm.H && w < rm.W) ? h * rm.W + w : -1;
}

__device__ __forceinline__ int64_t map_row(const RowMap& rm, int64_t r) {
    if (rm.kind == ROWMAP_WIN_UNPART) return win_unpart_row(r, rm.W, rm.ws);
    if (rm.kind == ROWMAP_SAM2_UNPART) return hwin_src(r, rm.W, rm.H, rm.ws, rm.nwh);
    return r;
}

// Unaligned 2-byte-granular loads of quantized block payloads (ggml blocks
// are 34/18/20 bytes, so qs is only 2-byte aligned in general).
__device__ __forceinline__ uint32_t ld_u32_a2(const uint8_t* p) {
    const uint16_t* q = reinterpret_cast<const uint16_t*>(p);
    return (uint32_t)q[0] | ((uint32_t)q[1] << 16);
}

// Q4 nibbles of 4 consecutive payload bytes -> 4 low-nibble bytes and 4
// high-nibble bytes (element j and j+16 of the block).
__device__ __forceinline__ void nibbles(uint32_t w, uint32_t& lo, uint32_t& hi) {
    lo = w & 0x0f0f0f0fu;
    hi = (w >> 4) & 0x0f0f0f0fu;
}
// Per-byte subtract 8 of values in [0,15] -> int8 in [-8,7] (no borrow across bytes).
__device__ __forceinline__ uint32_t sub8_bytes(uint32_t v) {
    return ((v | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
}

}  // namespace mi355
