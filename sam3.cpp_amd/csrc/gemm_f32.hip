// ggml MUL_MAT with F32 src0 and F32 src1 (ggml_vec_dot_f32 semantics:
// fp32 products summed in fp32) on gfx950 fp32 MFMA.  Used by the patch
// embedding (ggml_conv_2d_sk_p0 -> im2col + mul_mat with the F32 patch
// weight, sam3.cpp:3815; the weight stays F32 under quantized weight types,
// sam3.cpp:2479-2481, since its rows of 14 are not a multiple of 32).
//
// Workgroup tile 64(m) x 64(n), four wavefronts of 32 x 32, K staged through
// LDS 32 at a time (rows padded to 33 floats: the 32-row fragment reads of a
// column hit 32 distinct banks); v_mfma_f32_32x32x2f32 takes one element of
// A and one of B per lane (lane l: row/column l % 32, k = l / 32).
#include "common.cuh"
#include "kernels.h"

namespace mi355 {

namespace {
constexpr int GT = 64, GK = 32;
}

__global__ __launch_bounds__(256) void gemm_f32_kernel(const GemmF32Args p) {
    __shared__ float sA[GT][GK + 1];
    __shared__ float sB[GT][GK + 1];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = w & 1, wn = w >> 1;
    const int lr = lane & 31, g = lane >> 5;
    const int m0 = blockIdx.x * GT, n0 = blockIdx.y * GT;
    const int z = blockIdx.z, i12 = z % p.ne12, i13 = z / p.ne12;
    const char* W = reinterpret_cast<const char*>(p.W) + (int64_t)(i12 / p.r2) * p.w_nb2 + (int64_t)(i13 / p.r3) * p.w_nb3;
    const char* X = reinterpret_cast<const char*>(p.X) + (int64_t)i12 * p.x_nb2 + (int64_t)i13 * p.x_nb3;
    v16f acc = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    for (int k0 = 0; k0 < p.K; k0 += GK) {
        for (int idx = tid; idx < GT * GK; idx += 256) {
            const int r = idx / GK, kk = idx % GK, k = k0 + kk;
            sA[r][kk] = (m0 + r < p.M && k < p.K) ? *reinterpret_cast<const float*>(X + (int64_t)(m0 + r) * p.x_nb1 + 4LL * k)
                                                   : 0.0f;
            sB[r][kk] = (n0 + r < p.N && k < p.K) ? *reinterpret_cast<const float*>(W + (int64_t)(n0 + r) * p.w_nb1 + 4LL * k)
                                                   : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int s = 0; s < GK / 2; ++s)
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(sA[wm * 32 + lr][2 * s + g], sB[wn * 32 + lr][2 * s + g], acc, 0, 0,
                                                      0);
        __syncthreads();
    }
    char* D = reinterpret_cast<char*>(p.D) + (int64_t)i12 * p.d_nb2 + (int64_t)i13 * p.d_nb3;
    const int n = n0 + wn * 32 + lr;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int m = m0 + wm * 32 + 8 * (i >> 2) + 4 * g + (i & 3);
        if (m < p.M && n < p.N) *reinterpret_cast<float*>(D + (int64_t)m * p.d_nb1 + 4LL * n) = acc[i];
    }
}

hipError_t launch_gemm_f32(const GemmF32Args& a, int Z, hipStream_t st) {
    if (a.M <= 0 || a.N <= 0 || Z <= 0) return hipSuccess;
    const dim3 grid((unsigned)((a.M + GT - 1) / GT), (unsigned)((a.N + GT - 1) / GT), (unsigned)Z);
    gemm_f32_kernel<<<grid, 256, 0, st>>>(a);
    return hipGetLastError();
}

}  // namespace mi355
