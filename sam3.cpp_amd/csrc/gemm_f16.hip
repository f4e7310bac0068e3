// F16 mul_mat (ggml MUL_MAT with F16 weights, activations converted to F16)
// on gfx950 fp16 MFMA with fp32 accumulation.
//
// dst[m][n] = sum_k f16(w[n][k]) * f16(a[m][k]) (products exact in fp32).
//
// Tiling: workgroup 128(m) x 128(n), 4 wavefronts in 2x2, each 64x64 =
// 2x2 tiles of v_mfma_f32_32x32x16_f16.  K is staged 64 halves (128 B) per
// step.  MFMA operand (lane l): row l%32, halves k = 8*(l/32)..+7 of the
// 16-wide k slice; the same k mapping on both operands, so the sum is the
// plain dot product.
#include "common.cuh"
#include "kernels.h"

namespace mi355 {

namespace {
constexpr int BM = 128, BN = 128, BKH = 64;  // BKH halves per k-step
constexpr int LDT = BKH * 2 + 16;           // LDS row pitch in bytes
constexpr int NT = 256;
}  // namespace

__global__ __launch_bounds__(NT, 2) void gemm_f16_kernel(const uint8_t* __restrict__ W, int64_t w_nb1,
                                                         int64_t w_nb2, int64_t w_nb3,
                                                         const uint16_t* __restrict__ A, int64_t a_s1,
                                                         int64_t a_s2, int64_t a_s3, float* __restrict__ D,
                                                         int64_t d_nb1, int64_t d_nb2, int64_t d_nb3, int M, int N,
                                                         int K, int ne12, int r2, int r3) {
    __shared__ __attribute__((aligned(16))) uint8_t sA[BM * LDT];
    __shared__ __attribute__((aligned(16))) uint8_t sB[BN * LDT];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
    const int z = blockIdx.z, i12 = z % ne12, i13 = z / ne12;
    const uint8_t* Wz = W + (int64_t)(i12 / r2) * w_nb2 + (int64_t)(i13 / r3) * w_nb3;
    const uint16_t* Az = A + (int64_t)i12 * a_s2 + (int64_t)i13 * a_s3;

    v16f acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.0f;

    for (int k0 = 0; k0 < K; k0 += BKH) {
#pragma unroll
        for (int it = 0; it < (BM * BKH * 2 / 16) / NT; ++it) {
            const int c = tid + it * NT;
            const int row = c / (BKH / 8), col = (c % (BKH / 8)) * 8;  // col in halves
            const int k = k0 + col;
            v4i va = {0, 0, 0, 0}, vb = {0, 0, 0, 0};
            const int m = m0 + row, n = n0 + row;
            if (m < M && k < K) va = *reinterpret_cast<const v4i*>(Az + (int64_t)m * a_s1 + k);
            if (n < N && k < K) vb = *reinterpret_cast<const v4i*>(Wz + (int64_t)n * w_nb1 + (int64_t)k * 2);
            *reinterpret_cast<v4i*>(sA + row * LDT + col * 2) = va;
            *reinterpret_cast<v4i*>(sB + row * LDT + col * 2) = vb;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < BKH / 16; ++kk) {
            v8h af[2], bf[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                af[t] = *reinterpret_cast<const v8h*>(sA + (wm * 64 + t * 32 + (lane & 31)) * LDT + kk * 32 +
                                                      (lane >> 5) * 16);
                bf[t] = *reinterpret_cast<const v8h*>(sB + (wn * 64 + t * 32 + (lane & 31)) * LDT + kk * 32 +
                                                      (lane >> 5) * 16);
            }
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[mt], bf[nt], acc[mt][nt], 0, 0, 0);
        }
        __syncthreads();
    }

    char* Dz = reinterpret_cast<char*>(D) + (int64_t)i12 * d_nb2 + (int64_t)i13 * d_nb3;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const int n = n0 + wn * 64 + nt * 32 + (lane & 31);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int m = m0 + wm * 64 + mt * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
                if (m < M && n < N) *reinterpret_cast<float*>(Dz + (int64_t)m * d_nb1 + (int64_t)n * 4) = acc[mt][nt][i];
            }
        }
}

hipError_t launch_gemm_f16(const MatW& w, const uint16_t* a, int64_t a_s1, int64_t a_s2, int64_t a_s3,
                           const MatD& d, int64_t M, int64_t N, int64_t K, int64_t ne12, int64_t ne13,
                           hipStream_t st) {
    const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM), (unsigned)(ne12 * ne13));
    gemm_f16_kernel<<<grid, NT, 0, st>>>(w.data, w.nb1, w.nb2, w.nb3, a, a_s1, a_s2, a_s3, d.data, d.nb1, d.nb2,
                                         d.nb3, (int)M, (int)N, (int)K, (int)ne12, (int)(ne12 / w.ne2),
                                         (int)(ne13 / w.ne3));
    return hipGetLastError();
}

}  // namespace mi355
