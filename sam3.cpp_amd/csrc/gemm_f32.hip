// ggml MUL_MAT with F32 src0 and F32 src1 (ggml_vec_dot_f32 semantics:
// fp32 products summed in fp32) on gfx950 fp32 MFMA.  Used by the patch
// embeddings (ggml_conv_2d -> im2col + mul_mat with the F32 patch weight,
// sam3.cpp:3815, 4473; the weight stays F32 under quantized weight types,
// sam3.cpp:2479-2481, since its rows of 7 or 14 are not a multiple of 32) and
// by the SimpleFPN neck's F32 convolutions.
//
// Tiled kernel (rows 16-byte aligned, K % 4 == 0): workgroup 128(m) x 128(n),
// four wavefronts of 64 x 64 (2 x 2 v_mfma_f32_32x32x2f32 tiles), K staged 32
// at a time, double-buffered through LDS by float4 loads held in registers
// across the current stage's MFMAs.  The MFMA takes one A and one B element
// per lane (lane l: row l % 32, k-slot l / 32 of a 2-wide k step), so a tile
// row is stored parity-split, [row][k % 2][k / 2]: each lane's sixteen operand
// values of a stage are four contiguous ds_read_b128.  Row pitch 36 floats:
// the 16 rows one read pass touches land on distinct 4-bank groups.  Tiles
// are walked XCD-aware (each XCD a contiguous band), so the n-tiles of one
// m-tile read their activation rows through one L2.
//
// The same kernel runs a 3x3 / stride-1 / pad-1 convolution as an implicit
// GEMM over a token-major [H*W][C] map (C % 32 == 0): a stage of 32 K values
// lies within one tap, so each A row is one 128-byte segment of the pixel the
// tap reaches, or zeros outside the image.  No im2col buffer exists.
//
// gemm_f32_dma_kernel is the same GEMM with both operands staged by LDS DMA
// (two 32 KB stage buffers, no staging registers); it serves every operand its
// 32-bit buffer offsets reach, the register-staged kernel the rest.  Grids of
// fewer than two tiles per CU may split K (gemm_ksplit): fp32 partial sums per
// range into caller scratch, added in split order with the bias by
// gemm_f32_split_reduce_kernel.
//
// The 64 x 64 scalar-load kernel remains for rows that are not 16-byte
// aligned or K not a multiple of 4.
#include "common.cuh"
#include "kernels.h"

namespace mi355 {

namespace {
constexpr int GT = 64, GK = 32;
constexpr int TM = 128, TN = 128, TK = 32, TP = 36;  // tile, K stage, LDS row pitch (floats)
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
    const float bn = p.bias && n < p.N ? p.bias[n] : 0.0f;
    float ad[16];  // the addend, loaded before the first store (as the tiled kernels)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int m = m0 + wm * 32 + 8 * (i >> 2) + 4 * g + (i & 3);
        ad[i] = p.add && m < p.M && n < p.N ? p.add[(int64_t)m * p.N + n] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int m = m0 + wm * 32 + 8 * (i >> 2) + 4 * g + (i & 3);
        if (m < p.M && n < p.N) {
            float v = acc[i] + bn;
            if (p.add) v = v + ad[i];
            *reinterpret_cast<float*>(D + (int64_t)m * p.d_nb1 + 4LL * n) = v;
        }
    }
}

template <bool CONV>
__global__ __launch_bounds__(256, 2) void gemm_f32_tiled_kernel(const GemmF32Args p, int ksplit, int sps) {
    __shared__ __attribute__((aligned(16))) float sA[2][TM * TP];
    __shared__ __attribute__((aligned(16))) float sB[2][TN * TP];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = w & 1, wn = w >> 1;  // this wavefront's 64 x 64 quadrant
    const int lr = lane & 31, g = lane >> 5;
    // XCD-aware order: workgroups are dispatched round-robin over the 8 XCDs, so
    // workgroup b works tile (b % 8) * per_xcd + b / 8 and each XCD walks a contiguous
    // band of tiles (the n-tiles of one m-tile share its activation rows in one L2)
    // band of tiles. With a K split, the split is the slowest index: workgroup slot
    // (split, tile), its K range stages [split * sps, (split + 1) * sps)
    const int tiles_n = (p.N + TN - 1) / TN, tiles = ((p.M + TM - 1) / TM) * tiles_n;
    const int TT = tiles * ksplit, per_xcd = (TT + 7) / 8;
    const int tls = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (tls >= TT) return;
    const int split = tls / tiles, tl = tls - split * tiles;
    const int m0 = (tl / tiles_n) * TM, n0 = (tl % tiles_n) * TN;
    const int z = blockIdx.y, i12 = z % p.ne12, i13 = z / p.ne12;
    const char* Wb = reinterpret_cast<const char*>(p.W) + (int64_t)(i12 / p.r2) * p.w_nb2 + (int64_t)(i13 / p.r3) * p.w_nb3;
    const char* Xb = reinterpret_cast<const char*>(p.X) + (int64_t)i12 * p.x_nb2 + (int64_t)i13 * p.x_nb3;

    // loader: thread t fills row t/2 of both tiles, K values 16*(t%2) .. +15 of the stage
    const int lrow = tid >> 1, lk = 16 * (tid & 1);
    const int am = m0 + lrow, bn_ = n0 + lrow;
    int oy = 0, ox = 0;
    if (CONV) {
        oy = am / p.Wd;
        ox = am - oy * p.Wd;
    }
    v4f ra[4], rb[4];
    auto load = [&](int k0) {
        const v4f zero = {0, 0, 0, 0};
        if (CONV) {  // the 32 K values of a stage lie within one tap (C % 32 == 0)
            const int tap = k0 / p.C, c0 = k0 - tap * p.C;
            const int iy = oy + tap / 3 - 1, ix = ox + tap % 3 - 1;
            const bool in = am < p.M && iy >= 0 && iy < p.H && ix >= 0 && ix < p.Wd;
            const float* src = reinterpret_cast<const float*>(Xb) + ((int64_t)iy * p.Wd + ix) * p.C + c0 + lk;
#pragma unroll
            for (int h = 0; h < 4; ++h) ra[h] = in ? *reinterpret_cast<const v4f*>(src + 4 * h) : zero;
        } else {
            const float* src = reinterpret_cast<const float*>(Xb + (int64_t)am * p.x_nb1) + k0 + lk;
#pragma unroll
            for (int h = 0; h < 4; ++h)
                ra[h] = am < p.M && k0 + lk + 4 * h < p.K ? *reinterpret_cast<const v4f*>(src + 4 * h) : zero;
        }
        const float* wsrc = reinterpret_cast<const float*>(Wb + (int64_t)bn_ * p.w_nb1) + k0 + lk;
#pragma unroll
        for (int h = 0; h < 4; ++h)
            rb[h] = bn_ < p.N && k0 + lk + 4 * h < p.K ? *reinterpret_cast<const v4f*>(wsrc + 4 * h) : zero;
    };
    // k = lk + 4h + j -> parity j & 1 at [row][16 * (j & 1) + k / 2]
    auto park = [&](int buf) {
        float* a = &sA[buf][lrow * TP];
        float* b = &sB[buf][lrow * TP];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const int kk = (lk >> 1) + 2 * h;
            *reinterpret_cast<v2f*>(&a[kk]) = v2f{ra[h][0], ra[h][2]};
            *reinterpret_cast<v2f*>(&a[16 + kk]) = v2f{ra[h][1], ra[h][3]};
            *reinterpret_cast<v2f*>(&b[kk]) = v2f{rb[h][0], rb[h][2]};
            *reinterpret_cast<v2f*>(&b[16 + kk]) = v2f{rb[h][1], rb[h][3]};
        }
    };

    v16f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int kb = split * sps * TK;
    const int nst = min((p.K - kb + TK - 1) / TK, sps);
    load(kb);
    park(0);
    __syncthreads();
    for (int s = 0; s < nst; ++s) {
        const int buf = s & 1;
        if (s + 1 < nst) load(kb + (s + 1) * TK);
        v4f av[2][4], bv[2][4];  // this lane's 16 k values of its row (k-slot g), per tile
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const float* a = &sA[buf][(wm * 64 + i * 32 + lr) * TP + 16 * g];
            const float* b = &sB[buf][(wn * 64 + i * 32 + lr) * TP + 16 * g];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                av[i][q] = *reinterpret_cast<const v4f*>(a + 4 * q);
                bv[i][q] = *reinterpret_cast<const v4f*>(b + 4 * q);
            }
        }
#pragma unroll
        for (int kk = 0; kk < TK / 2; ++kk)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][kk >> 2][kk & 3], bv[j][kk >> 2][kk & 3],
                                                                    acc[i][j], 0, 0, 0);
        if (s + 1 < nst) park(buf ^ 1);
        __syncthreads();
    }

    if (ksplit > 1) {  // this split's partial sums, no bias: part [split][M][N]
        float* P = p.part + (int64_t)split * p.M * p.N;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + wn * 64 + j * 32 + lr;
            if (n >= p.N) continue;
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                    if (m < p.M) P[(int64_t)m * p.N + n] = acc[i][j][r];
                }
        }
        return;
    }
    char* D = reinterpret_cast<char*>(p.D) + (int64_t)i12 * p.d_nb2 + (int64_t)i13 * p.d_nb3;
    // the addend's values, all loaded before the first store (D may alias it, so loads
    // interleaved with the stores would each wait for the one before)
    float ad[2][2][16];
    if (p.add) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int n = n0 + wn * 64 + j * 32 + lr;
                    const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                    ad[j][i][r] = m < p.M && n < p.N ? p.add[(int64_t)m * p.N + n] : 0.0f;
                }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn * 64 + j * 32 + lr;
        if (n >= p.N) continue;
        const float bn = p.bias ? p.bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                if (m < p.M) {
                    float v = acc[i][j][r] + bn;
                    if (p.add) v = v + ad[j][i][r];
                    *reinterpret_cast<float*>(D + (int64_t)m * p.d_nb1 + 4LL * n) = v;
                }
            }
    }
}

// The tiled kernel with its operands staged by LDS DMA (buffer_load ... lds) into NB stage
// buffers of 32 K values (A and B rows of 128 bytes, 32 KB per stage), filled NB - 1 stages
// ahead, so no registers stage anything and no branch guards a load: rows past M or N,
// taps outside the image and the chunks of a last partial stage past K get an offset past
// the buffer's records, which reads zero. Rows hold chunk c (k values 4c .. 4c + 3) in slot
// c ^ fswz(r), so the 16 rows of a ds_read_b128 quarter (two parities of eight rows) cover
// the 64 banks. Lane group g of a fragment read takes chunks 2q + g (q < 4), and MFMA step
// (q, e) pairs k = 8q + e (lanes 0..31) with 8q + 4 + e (lanes 32..63) in A and B alike:
// every k of the stage once, in fp32 products and fp32 accumulation as before (the k order
// inside a stage differs from the tiled kernel's, so sums may differ in the last bits).
namespace {
constexpr int F32_OOB = 0x7ffffff0;  // a buffer offset past every operand the launcher admits
// LDS slot of chunk c of tile row r (16-byte chunks, KD / 4 to a row): c ^ fswz<KD>(r). At KD = 32
// two 128-byte rows share a 256-byte bank line, at KD = 16 four 64-byte rows: the 16 rows of
// a ds_read_b128 quarter then cover the 64 banks
template <int KD>
__device__ __forceinline__ int fswz(int r) { return KD == 32 ? (r >> 1) & 7 : (r >> 2) & 3; }
template <int KD>
struct F32Stage {
    float A[TM * KD];
    float B[TN * KD];
};
}  // namespace

// KD: K values per stage (32 or 16); NB stage buffers, up to NB - 1 stages in flight past the
// one computed. sps counts 32-deep stages (the launcher's unit) whatever KD.
template <bool CONV, int KD, int NB>
__global__ __launch_bounds__(256, NB * KD * 2 * 128 * 4 <= 54 * 1024 ? 3 : (NB * KD * 2 * 128 * 4 <= 80 * 1024 ? 2 : 1))
void gemm_f32_dma_kernel(const GemmF32Args p, int ksplit, int sps) {
    using Stage = F32Stage<KD>;
    constexpr int CH = KD / 4;        // 16-byte chunks per tile row
    constexpr int RPI = 64 / CH;      // tile rows per DMA instruction (1 KB)
    constexpr int NI = TM / RPI / 4;  // DMA instructions per wavefront and operand
    constexpr int NL = 2 * NI;        // per wavefront and stage
    __shared__ __attribute__((aligned(16))) Stage sb[NB];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wv & 1, wn = wv >> 1;
    const int lr = lane & 31, g = lane >> 5;
    // XCD-aware order with the K split as the slowest index, as the tiled kernel
    const int M = p.M, N = p.N, K = p.K;
    const int tiles_n = (N + TN - 1) / TN, tiles = ((M + TM - 1) / TM) * tiles_n;
    const int TT = tiles * ksplit, per_xcd = (TT + 7) / 8;
    const int tls = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (tls >= TT) return;
    const int split = tls / tiles, tl = tls - split * tiles;
    const int m0 = (tl / tiles_n) * TM, n0 = (tl % tiles_n) * TN;
    const int z = blockIdx.y, i12 = z % p.ne12, i13 = z / p.ne12;
    const char* Wb = reinterpret_cast<const char*>(p.W) + (int64_t)(i12 / p.r2) * p.w_nb2 + (int64_t)(i13 / p.r3) * p.w_nb3;
    const char* Xb = reinterpret_cast<const char*>(p.X) + (int64_t)i12 * p.x_nb2 + (int64_t)i13 * p.x_nb3;
    const int kb = split * sps * TK;
    const int nst = min((K - kb + KD - 1) / KD, sps * (TK / KD));

    // DMA instruction j (< NI) of wavefront wv: tile rows RPI (NI wv + j) + lane / CH of A and of
    // B, LDS slot lane % CH, global chunk slot ^ fswz(row)
    const v4i xr = make_rsrc(Xb, CONV ? (int64_t)M * p.C * 4 : (int64_t)(M - 1) * p.x_nb1 + 4LL * K);
    const v4i wr = make_rsrc(Wb, (int64_t)(N - 1) * p.w_nb1 + 4LL * K);
    int ach[NI], aoff[NI], boff[NI], py[NI], px[NI];
#pragma unroll
    for (int j = 0; j < NI; ++j) {
        const int row = RPI * (NI * wv + j) + lane / CH, m = m0 + row, n = n0 + row;
        ach[j] = (lane % CH) ^ fswz<KD>(row);  // the chunk this lane loads
        py[j] = px[j] = 0;
        if (CONV) {
            py[j] = m < M ? m / p.Wd : -(1 << 20);  // past M: every tap lands outside the image
            px[j] = m < M ? m - (m / p.Wd) * p.Wd : 0;
        }
        aoff[j] = m < M ? (int)((int64_t)m * p.x_nb1) + 16 * ach[j] : F32_OOB;
        boff[j] = n < N ? (int)((int64_t)n * p.w_nb1) + 16 * ach[j] : F32_OOB;
    }
    uint32_t lb[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) lb[i] = (uint32_t)__builtin_amdgcn_readfirstlane(lds_addr(&sb[i]));
    auto dma = [&](int s, uint32_t base) __attribute__((always_inline)) {
        const int k0 = kb + s * KD;
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const bool kin = k0 + 4 * ach[j] < K;  // false only in a last partial stage
            int off;
            if (CONV) {
                const int tap = k0 / p.C, c0 = k0 - tap * p.C;
                const int iy = py[j] + tap / 3 - 1, ix = px[j] + tap % 3 - 1;
                const bool in = iy >= 0 && iy < p.H && ix >= 0 && ix < p.Wd;
                off = in ? ((iy * p.Wd + ix) * p.C + c0) * 4 + 16 * ach[j] : F32_OOB;
            } else {
                off = aoff[j] != F32_OOB && kin ? aoff[j] + 4 * k0 : F32_OOB;
            }
            dma_b128_so(xr, base + (uint32_t)offsetof(Stage, A) + 1024u * (NI * wv + j), off, 0);
        }
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const bool kin = k0 + 4 * ach[j] < K;
            const int off = boff[j] != F32_OOB && kin ? boff[j] + 4 * k0 : F32_OOB;
            dma_b128_so(wr, base + (uint32_t)offsetof(Stage, B) + 1024u * (NI * wv + j), off, 0);
        }
    };
    // wait until this wavefront's DMA of all but the last `later` stages issued has landed
    auto wait_stages = [&](int later) __attribute__((always_inline)) {
        if (later >= 3) wait_vmcnt<3 * NL>();
        else if (later == 2) wait_vmcnt<2 * NL>();
        else if (later == 1) wait_vmcnt<NL>();
        else wait_vmcnt<0>();
    };

    const v16f zf = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    v16f acc[2][2] = {{zf, zf}, {zf, zf}};
    auto compute = [&](const Stage& b) __attribute__((always_inline)) {
        v4f av[CH / 2][2], bv[CH / 2][2];
#pragma unroll
        for (int q = 0; q < CH / 2; ++q)
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int ra = wm * 64 + i * 32 + lr, rb = wn * 64 + i * 32 + lr, c = 2 * q + g;
                av[q][i] = *reinterpret_cast<const v4f*>(&b.A[ra * KD + ((c ^ fswz<KD>(ra)) << 2)]);
                bv[q][i] = *reinterpret_cast<const v4f*>(&b.B[rb * KD + ((c ^ fswz<KD>(rb)) << 2)]);
            }
#pragma unroll
        for (int q = 0; q < CH / 2; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[q][i][e], bv[q][j][e], acc[i][j], 0, 0, 0);
    };

    // all NB buffers filled up front; stage s + NB refills stage s's buffer once it is read
#pragma unroll
    for (int i = 0; i < NB; ++i)
        if (i < nst) dma(i, lb[i]);
    wait_stages(min(nst, NB) - 1);
    __syncthreads();
    for (int s = 0; s < nst; ++s) {
        const int cb = s % NB;
        compute(sb[cb]);
        if (s + 1 < nst) {
            wait_stages(min(nst - 1, s + NB - 1) - (s + 1));  // stage s + 1 has landed
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // and stage s's buffer is read
            if (s + NB < nst) dma(s + NB, lb[cb]);
        }
    }

    if (ksplit > 1) {  // this split's partial sums, no bias: part [split][M][N]
        float* P = p.part + (int64_t)split * M * N;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + wn * 64 + j * 32 + lr;
            if (n >= N) continue;
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                    if (m < M) P[(int64_t)m * N + n] = acc[i][j][r];
                }
        }
        return;
    }
    char* D = reinterpret_cast<char*>(p.D) + (int64_t)i12 * p.d_nb2 + (int64_t)i13 * p.d_nb3;
    // the addend's values, all loaded before the first store (D may alias it, so loads
    // interleaved with the stores would each wait for the one before)
    float ad[2][2][16];
    if (p.add) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int n = n0 + wn * 64 + j * 32 + lr;
                    const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                    ad[j][i][r] = m < M && n < N ? p.add[(int64_t)m * N + n] : 0.0f;
                }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn * 64 + j * 32 + lr;
        if (n >= N) continue;
        const float bn = p.bias ? p.bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                if (m < M) {
                    float v = acc[i][j][r] + bn;
                    if (p.add) v = v + ad[j][i][r];
                    *reinterpret_cast<float*>(D + (int64_t)m * p.d_nb1 + 4LL * n) = v;
                }
            }
    }
}

// D = bias + part[0] + part[1] + ... (in split order) over an M x N tile set, float4 columns
// (f16out: D holds fp16, the sums rounded RNE)
__global__ __launch_bounds__(256) void gemm_f32_split_reduce_kernel(const float* __restrict__ part, int S, int M, int N,
                                                                    const float* __restrict__ bias, float* D,
                                                                    int64_t d_nb1, int f16out) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int n4 = N / 4;
    if (t >= (int64_t)M * n4) return;
    const int64_t m = t / n4;
    const int c = (int)(t - m * n4) * 4;
    const int64_t plane = (int64_t)M * N;
    v4f v = *reinterpret_cast<const v4f*>(part + m * N + c);
    for (int s = 1; s < S; ++s) v = v + *reinterpret_cast<const v4f*>(part + s * plane + m * N + c);
    if (bias) v = v + *reinterpret_cast<const v4f*>(bias + c);
    if (f16out) {
        const uint32_t h0 = (uint32_t)f2h(v[0]) | ((uint32_t)f2h(v[1]) << 16);
        const uint32_t h1 = (uint32_t)f2h(v[2]) | ((uint32_t)f2h(v[3]) << 16);
        *reinterpret_cast<uint2*>(reinterpret_cast<char*>(D) + m * d_nb1 + 2LL * c) = make_uint2(h0, h1);
    } else {
        *reinterpret_cast<v4f*>(reinterpret_cast<char*>(D) + m * d_nb1 + 4LL * c) = v;
    }
}

namespace {
// operand extents (bytes) the DMA kernel's 32-bit buffer offsets reach, with room for the
// out-of-range offset
bool dma_ok(int64_t x_bytes, int64_t w_bytes) { return x_bytes < F32_OOB - 4096 && w_bytes < F32_OOB - 4096; }
constexpr int F32_KD = 32, F32_NB = 2;  // K per stage and stage buffers of the DMA kernel
// the fp32 MFMA kernels split grids below two tiles per CU; one 32-deep stage of a
// 128 x 128 tile takes about 2.5 us alone on a CU
int f32_ksplit(int64_t M, int64_t N, int64_t K) {
    const int64_t tiles = ((M + TM - 1) / TM) * ((N + TN - 1) / TN);
    return gemm_ksplit(tiles, 512, M, N, (K + TK - 1) / TK, 2.5);
}
}  // namespace

size_t gemm_f32_part_bytes(int64_t M, int64_t N, int64_t K) {
    const int S = f32_ksplit(M, N, K);
    return S > 1 ? (size_t)S * (size_t)M * (size_t)N * 4 : 0;
}

hipError_t launch_split_reduce(const float* part, int S, int M, int N, const float* bias, float* D, int64_t d_nb1,
                               hipStream_t st, bool f16out) {
    if (N % 4 != 0 || S < 1 || ((reinterpret_cast<uintptr_t>(part) | reinterpret_cast<uintptr_t>(bias) |
                                 reinterpret_cast<uintptr_t>(D) | (uintptr_t)d_nb1) & 15))
        return hipErrorInvalidValue;
    const int64_t n = (int64_t)M * (N / 4);
    if (n > 0)
        gemm_f32_split_reduce_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(part, S, M, N, bias, D, d_nb1, f16out ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_gemm_f32(const GemmF32Args& a, int Z, hipStream_t st) {
    if (a.M <= 0 || a.N <= 0 || Z <= 0) return hipSuccess;
    if (a.add && Z != 1) return hipErrorInvalidValue;
    const int tiles = ((a.M + TM - 1) / TM) * ((a.N + TN - 1) / TN);
    // the K split (partials in a.part, then the reduce pass), when the caller gave room for it
    int S = 1, sps = (a.K + TK - 1) / TK;
    // (the reduce stores float4 rows: D and its row pitch on 16 bytes, N % 4 == 0)
    const bool d16 = ((reinterpret_cast<uintptr_t>(a.D) | (uintptr_t)a.d_nb1 | reinterpret_cast<uintptr_t>(a.part) |
                       reinterpret_cast<uintptr_t>(a.bias)) & 15) == 0;
    if (a.part && Z == 1 && !a.add && d16) {
        const int s = f32_ksplit(a.M, a.N, a.K);
        if (s > 1 && (size_t)s * (size_t)a.M * (size_t)a.N * 4 <= a.part_bytes) {
            S = s;
            sps = (sps + S - 1) / S;
        }
    }
    auto reduce = [&]() -> hipError_t {
        const hipError_t e = hipGetLastError();
        if (S == 1 || e != hipSuccess) return e;
        return launch_split_reduce(a.part, S, a.M, a.N, a.bias, a.D, a.d_nb1, st);
    };
    if (a.conv) {
        if (a.C % TK != 0 || a.K != 9 * a.C || (int64_t)a.H * a.Wd != a.M || Z != 1 ||
            (reinterpret_cast<uintptr_t>(a.X) & 15) || (reinterpret_cast<uintptr_t>(a.W) & 15) || (a.w_nb1 & 15))
            return hipErrorInvalidValue;
        if (dma_ok((int64_t)a.M * a.C * 4, (int64_t)(a.N - 1) * a.w_nb1 + 4LL * a.K))
            gemm_f32_dma_kernel<true, F32_KD, F32_NB><<<dim3((unsigned)((tiles * S + 7) / 8 * 8), 1), 256, 0, st>>>(a, S, sps);
        else
            gemm_f32_tiled_kernel<true><<<dim3((unsigned)((tiles * S + 7) / 8 * 8), 1), 256, 0, st>>>(a, S, sps);
        return reduce();
    }
    const bool tiled = a.K % 4 == 0 &&
                       ((reinterpret_cast<uintptr_t>(a.X) | reinterpret_cast<uintptr_t>(a.W) | (uintptr_t)a.x_nb1 |
                         (uintptr_t)a.x_nb2 | (uintptr_t)a.x_nb3 | (uintptr_t)a.w_nb1 | (uintptr_t)a.w_nb2 |
                         (uintptr_t)a.w_nb3) & 15) == 0;
    if (tiled) {
        // the DMA kernel's 32-bit buffer offsets must reach every operand of every batch
        if (dma_ok((int64_t)(a.M - 1) * a.x_nb1 + 4LL * a.K, (int64_t)(a.N - 1) * a.w_nb1 + 4LL * a.K))
            gemm_f32_dma_kernel<false, F32_KD, F32_NB><<<dim3((unsigned)((tiles * S + 7) / 8 * 8), (unsigned)Z), 256, 0, st>>>(a, S, sps);
        else
            gemm_f32_tiled_kernel<false><<<dim3((unsigned)((tiles * S + 7) / 8 * 8), (unsigned)Z), 256, 0, st>>>(a, S, sps);
        return reduce();
    }
    const dim3 grid((unsigned)((a.M + GT - 1) / GT), (unsigned)((a.N + GT - 1) / GT), (unsigned)Z);
    gemm_f32_kernel<<<grid, 256, 0, st>>>(a);
    return hipGetLastError();
}

}  // namespace mi355
