// ggml_soft_max_ext(a, mask = NULL, scale, max_bias = 0): per row of ne0
// elements y = exp(s*x - max) / sum.  One workgroup per row; the row is
// read once into registers (up to 64 values per lane), reduced for max and
// sum with wavefront butterflies plus an LDS stage, then written.
#include "common.cuh"
#include "kernels.h"

namespace mi355 {

namespace {
constexpr int NT = 256;
constexpr int PER = 32;  // values per thread held in registers (rows up to 8192)
}  // namespace

__device__ __forceinline__ float block_reduce_max(float v, float* red) {
    v = group_max<64>(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) r = fmaxf(r, red[w]);
    __syncthreads();
    return r;
}
__device__ __forceinline__ float block_reduce_sum(float v, float* red) {
    v = group_sum<64>(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = 0.0f;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) r += red[w];
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(NT) void soft_max_kernel(const char* __restrict__ src, int64_t ne0, int64_t ne1,
                                                      int64_t ne2, int64_t snb0, int64_t snb1, int64_t snb2,
                                                      int64_t snb3, char* __restrict__ dst, int64_t dnb0,
                                                      int64_t dnb1, int64_t dnb2, int64_t dnb3, float scale) {
    __shared__ float red[NT / 64];
    const int64_t r = blockIdx.x;
    const int64_t i1 = r % ne1, i2 = (r / ne1) % ne2, i3 = r / (ne1 * ne2);
    const char* sp = src + i1 * snb1 + i2 * snb2 + i3 * snb3;
    char* dp = dst + i1 * dnb1 + i2 * dnb2 + i3 * dnb3;
    float v[PER];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int64_t i = threadIdx.x + (int64_t)j * NT;
        v[j] = i < ne0 ? *reinterpret_cast<const float*>(sp + i * snb0) * scale : -INFINITY;
        mx = fmaxf(mx, v[j]);
    }
    mx = block_reduce_max(mx, red);
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int64_t i = threadIdx.x + (int64_t)j * NT;
        v[j] = i < ne0 ? expf(v[j] - mx) : 0.0f;
        sum += v[j];
    }
    sum = block_reduce_sum(sum, red);
    const float inv = 1.0f / sum;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int64_t i = threadIdx.x + (int64_t)j * NT;
        if (i < ne0) *reinterpret_cast<float*>(dp + i * dnb0) = v[j] * inv;
    }
}

hipError_t launch_soft_max(const SrcView& s, float scale, char* dst, const int64_t dnb[4], hipStream_t st) {
    const int64_t rows = s.ne[1] * s.ne[2] * s.ne[3];
    if (rows == 0) return hipSuccess;
    if (s.ne[0] > (int64_t)NT * PER) return hipErrorInvalidValue;
    soft_max_kernel<<<dim3((unsigned)rows), NT, 0, st>>>(s.data, s.ne[0], s.ne[1], s.ne[2], s.nb[0], s.nb[1],
                                                          s.nb[2], s.nb[3], dst, dnb[0], dnb[1], dnb[2], dnb[3],
                                                          scale);
    return hipGetLastError();
}

}  // namespace mi355
