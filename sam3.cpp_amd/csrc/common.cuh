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
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

// fp16 <-> fp32.  v_cvt_f16_f32 rounds to nearest even under the default
// MODE; fp16 denormals are kept (HIP's default f16/f64 denormal mode).
__device__ __forceinline__ float h2f(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float)v;
}
__device__ __forceinline__ uint16_t f2h(float f) {
    _Float16 v = (_Float16)f;
    uint16_t h;
    __builtin_memcpy(&h, &v, 2);
    return h;
}

// Butterfly reductions across `width` consecutive lanes (width a power of
// two <= 64) through ds_swizzle/ds_bpermute.
template <int width>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int o = width / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, width));
    return v;
}
template <int width>
__device__ __forceinline__ int group_sum_i(int v) {
#pragma unroll
    for (int o = width / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, width);
    return v;
}
template <int width>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = width / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, width);
    return v;
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
