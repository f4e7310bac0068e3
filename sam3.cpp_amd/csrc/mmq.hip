// Quantized mul_mat (ggml MUL_MAT with Q8_0 / Q4_0 / Q4_1 weights) on
// gfx950 int8 MFMA.
//
// dst[m][n] = sum_b fp32(d_w[n][b]) * fp32(d_a[m][b]) * isum[m][n][b]
//             (+ fp32(m_w[n][b]) * fp32(s_a[m][b]) for Q4_1)
// isum[m][n][b] = sum_{j<32} q_w[n][32b+j] * q_a[m][32b+j]  (exact int32)
//
// One v_mfma_i32_32x32x32_i8 covers exactly one 32-element block of a
// 32x32 output tile, so its int32 result *is* the ggml block dot; the
// per-block scale is applied in fp32 right after (fma into the accumulator).
//
// Tiling: workgroup 128(m) x 128(n), 4 wavefronts in 2x2, each owning a
// 64x64 sub-tile = 2x2 MFMA tiles.  Per k-step of 4 blocks (128 bytes of K)
// the workgroup stages the activation tile (int8, from the MMQ layout) and
// the weight tile (ggml blocks unpacked to int8 in registers) in LDS, with
// the scales in separate fp32 arrays.  MFMA operand (lane l): row l%32 of
// the tile, the 16 consecutive k-bytes 16*(l/32)..+15 of the block.
#include "common.cuh"
#include "kernels.h"

namespace mi355 {

namespace {
constexpr int BM = 128, BN = 128, BKB = 4, BK = BKB * QK;
constexpr int LDT = BK + 16;  // LDS row pitch in bytes (16 B pad against bank conflicts)
constexpr int NT = 256;
}  // namespace

// Unpacks one weight block into 8 dwords of int8 (element order 0..31) and
// returns its scale (and min for Q4_1).
template <int WT>
__device__ __forceinline__ void load_wblock(const uint8_t* blk, uint32_t w[8], float& dv, float& mv) {
    if (WT == T_Q8_0) {
        dv = h2f(*reinterpret_cast<const uint16_t*>(blk));
#pragma unroll
        for (int j = 0; j < 8; ++j) w[j] = ld_u32_a2(blk + 2 + 4 * j);
    } else if (WT == T_Q4_0) {
        dv = h2f(*reinterpret_cast<const uint16_t*>(blk));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t lo, hi;
            nibbles(ld_u32_a2(blk + 2 + 4 * j), lo, hi);
            w[j] = sub8_bytes(lo);
            w[4 + j] = sub8_bytes(hi);
        }
    } else {  // Q4_1: raw nibbles in [0,15]
        dv = h2f(reinterpret_cast<const uint16_t*>(blk)[0]);
        mv = h2f(reinterpret_cast<const uint16_t*>(blk)[1]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t lo, hi;
            nibbles(ld_u32_a2(blk + 4 + 4 * j), lo, hi);
            w[j] = lo;
            w[4 + j] = hi;
        }
    }
}

template <int WT> constexpr int wblock_bytes() {
    return WT == T_Q8_0 ? (int)sizeof(blk_q8_0) : WT == T_Q4_0 ? (int)sizeof(blk_q4_0) : (int)sizeof(blk_q4_1);
}

template <int WT, bool DOTS>
__global__ __launch_bounds__(NT, 2) void mmq_kernel(const uint8_t* __restrict__ W, int64_t w_nb1, int64_t w_nb2,
                                                    int64_t w_nb3, const int8_t* __restrict__ aq,
                                                    const float* __restrict__ ad, const float* __restrict__ as,
                                                    float* __restrict__ D, int64_t d_nb1, int64_t d_nb2,
                                                    int64_t d_nb3, int32_t* __restrict__ dots, int M, int N, int K,
                                                    int ne12, int r2, int r3) {
    __shared__ __attribute__((aligned(16))) int8_t sA[BM * LDT];
    __shared__ __attribute__((aligned(16))) int8_t sB[BN * LDT];
    __shared__ __attribute__((aligned(16))) float sAd[BKB][BM];
    __shared__ __attribute__((aligned(16))) float sBd[BKB][BN];
    __shared__ __attribute__((aligned(16))) float sAs[WT == T_Q4_1 ? BKB : 1][BM];
    __shared__ __attribute__((aligned(16))) float sBm[WT == T_Q4_1 ? BKB : 1][BN];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
    const int z = blockIdx.z, i12 = z % ne12, i13 = z / ne12;
    const uint8_t* Wz = W + (int64_t)(i12 / r2) * w_nb2 + (int64_t)(i13 / r3) * w_nb3;
    const int nb = K / QK;
    const int8_t* aqz = aq + (int64_t)z * M * K;
    const float* adz = ad + (int64_t)z * nb * M;
    const float* asz = WT == T_Q4_1 ? as + (int64_t)z * nb * M : nullptr;
    constexpr int WB = wblock_bytes<WT>();

    v16f acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.0f;
    const v16i zero16 = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

    for (int kb0 = 0; kb0 < nb; kb0 += BKB) {
        // activation tile: BM rows x BK bytes, 16 B per thread-chunk
#pragma unroll
        for (int it = 0; it < (BM * BK / 16) / NT; ++it) {
            const int c = tid + it * NT;
            const int row = c / (BK / 16), col = (c % (BK / 16)) * 16;
            const int m = m0 + row, kb = kb0 + col / QK;
            v4i v = {0, 0, 0, 0};
            if (m < M && kb < nb) v = *reinterpret_cast<const v4i*>(aqz + (int64_t)m * K + (int64_t)kb0 * QK + col);
            *reinterpret_cast<v4i*>(sA + row * LDT + col) = v;
        }
#pragma unroll
        for (int it = 0; it < (BKB * BM) / NT; ++it) {
            const int c = tid + it * NT;
            const int b = c / BM, row = c % BM;
            const int m = m0 + row, kb = kb0 + b;
            const bool ok = m < M && kb < nb;
            sAd[b][row] = ok ? adz[(int64_t)kb * M + m] : 0.0f;
            if (WT == T_Q4_1) sAs[b][row] = ok ? asz[(int64_t)kb * M + m] : 0.0f;
        }
        // weight tile: BN rows x BKB blocks, unpacked to int8
#pragma unroll
        for (int it = 0; it < (BN * BKB) / NT; ++it) {
            const int c = tid + it * NT;
            const int row = c / BKB, b = c % BKB;
            const int n = n0 + row, kb = kb0 + b;
            uint32_t w[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            float dv = 0.0f, mv = 0.0f;
            if (n < N && kb < nb) load_wblock<WT>(Wz + (int64_t)n * w_nb1 + (int64_t)kb * WB, w, dv, mv);
            v4i* dp = reinterpret_cast<v4i*>(sB + row * LDT + b * QK);
            dp[0] = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
            dp[1] = v4i{(int)w[4], (int)w[5], (int)w[6], (int)w[7]};
            sBd[b][row] = dv;
            if (WT == T_Q4_1) sBm[b][row] = mv;
        }
        __syncthreads();

#pragma unroll
        for (int b = 0; b < BKB; ++b) {
            if (kb0 + b >= nb) break;
            v4i af[2], bf[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                af[t] = *reinterpret_cast<const v4i*>(sA + (wm * 64 + t * 32 + (lane & 31)) * LDT + b * QK +
                                                      (lane >> 5) * 16);
                bf[t] = *reinterpret_cast<const v4i*>(sB + (wn * 64 + t * 32 + (lane & 31)) * LDT + b * QK +
                                                      (lane >> 5) * 16);
            }
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) {
                    const v16i is = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[mt], bf[nt], zero16, 0, 0, 0);
                    const int ncol = wn * 64 + nt * 32 + (lane & 31);
                    const int mrow = wm * 64 + mt * 32 + 4 * (lane >> 5);
                    if (DOTS) {
                        const int n = n0 + ncol;
#pragma unroll
                        for (int i = 0; i < 16; ++i) {
                            const int m = m0 + mrow + 8 * (i >> 2) + (i & 3);
                            if (m < M && n < N)
                                dots[(((int64_t)z * M + m) * N + n) * nb + kb0 + b] = is[i];
                        }
                        continue;
                    }
                    const float dw = sBd[b][ncol];
                    float mw = 0.0f;
                    if (WT == T_Q4_1) mw = sBm[b][ncol];
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const v4f da = *reinterpret_cast<const v4f*>(&sAd[b][mrow + 8 * g]);
                        v4f sa = {0.f, 0.f, 0.f, 0.f};
                        if (WT == T_Q4_1) sa = *reinterpret_cast<const v4f*>(&sAs[b][mrow + 8 * g]);
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int i = 4 * g + r;
                            float a = __builtin_fmaf((float)is[i], da[r] * dw, acc[mt][nt][i]);
                            if (WT == T_Q4_1) a = __builtin_fmaf(sa[r], mw, a);
                            acc[mt][nt][i] = a;
                        }
                    }
                }
            }
        }
        __syncthreads();
    }
    if (DOTS) return;

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

template <int WT>
static hipError_t launch_t(const MatW& w, const ActQ8& a, const MatD& d, int64_t N, int64_t ne12, int64_t ne13,
                           int32_t* dots, hipStream_t st) {
    const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((a.M + BM - 1) / BM), (unsigned)(ne12 * ne13));
    const int r2 = (int)(ne12 / w.ne2), r3 = (int)(ne13 / w.ne3);
    if (dots)
        mmq_kernel<WT, true><<<grid, NT, 0, st>>>(w.data, w.nb1, w.nb2, w.nb3, a.qs, a.d, a.s, d.data, d.nb1, d.nb2,
                                                  d.nb3, dots, (int)a.M, (int)N, (int)a.K, (int)ne12, r2, r3);
    else
        mmq_kernel<WT, false><<<grid, NT, 0, st>>>(w.data, w.nb1, w.nb2, w.nb3, a.qs, a.d, a.s, d.data, d.nb1, d.nb2,
                                                   d.nb3, nullptr, (int)a.M, (int)N, (int)a.K, (int)ne12, r2, r3);
    return hipGetLastError();
}

hipError_t launch_mmq(const MatW& w, const ActQ8& a, const MatD& d, int64_t N, int64_t ne12, int64_t ne13,
                      int32_t* dots, hipStream_t st) {
    switch (w.type) {
        case T_Q8_0: return launch_t<T_Q8_0>(w, a, d, N, ne12, ne13, dots, st);
        case T_Q4_0: return launch_t<T_Q4_0>(w, a, d, N, ne12, ne13, dots, st);
        case T_Q4_1: return launch_t<T_Q4_1>(w, a, d, N, ne12, ne13, dots, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace mi355
