// SAM3 SimpleFPN neck kernels (sam3_build_neck_graph, sam3.cpp:3867-3925) on
// token-major activations [H*W][C] (ggml [C, W, H]).  conv_f16_dma_kernel (and
// conv_f16_kernel, its register-staged form for operands beyond 32-bit buffer
// offsets) is the fp16-MFMA implicit GEMM of the F16-kernel convolutions (3x3,
// 1x1 and the 2x2 / stride-2 conv-transpose with its scatter, bias and GELU in
// the epilogue; the 3x3 and 1x1 split K on grids smaller than the CU count, the
// partial sums added by gemm_f32.hip's reduce); F32-kernel convolutions run on
// gemm_f32.hip.  The rest are
// HBM-bound passes: the conv-transpose kernel repack + F16 cast, the 3x3
// kernel repacks for the implicit GEMMs, and, for maps the implicit GEMMs do
// not take, im2col, the conv-transpose scatter and bias adds; the 2x2
// max-pool.
#include "common.cuh"
#include "kernels.h"

namespace mi355 {

namespace {
unsigned nblk(int64_t n) { return (unsigned)((n + 255) / 256); }
}

// ggml conv-transpose kernel [kW=2, kH=2, Cout, Cin] (memory [ci][co][kh][kw]),
// F32 or F16, -> F16 MUL_MAT weight rows [4*Cout][Cin], row n = (kh*2 + kw)*Cout + co.
// The F32 -> F16 cast rounds to nearest even, as ggml_cast does
// (sam3_conv_transpose_weight, sam3.cpp:1087-1090).
__global__ __launch_bounds__(256) void deconv_pack_kernel(const void* __restrict__ w, int wtype, int Cin, int Cout,
                                                          uint16_t* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= 4LL * Cout * Cin) return;
    const int ci = (int)(i % Cin);
    const int n = (int)(i / Cin), t = n / Cout, co = n % Cout;
    const int64_t src = (((int64_t)ci * Cout + co) * 2 + (t >> 1)) * 2 + (t & 1);
    out[i] = wtype == T_F16 ? static_cast<const uint16_t*>(w)[src] : f2h(static_cast<const float*>(w)[src]);
}

// y[(2py + kh)(2W) + 2px + kw][co] = D[py*W + px][(kh*2 + kw)*Cout + co] + b[co]
// (then GELU-erf, or not).  Four channels per thread; Cout % 4 == 0.
__global__ __launch_bounds__(256) void deconv_scatter_kernel(const float* __restrict__ D, const float* __restrict__ b,
                                                             int H, int W, int Cout, int gelu, float* __restrict__ y) {
    const int c4 = Cout / 4;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= 4LL * H * W * c4) return;
    const int co = (int)(i % c4) * 4;
    const int64_t pix = i / c4;
    const int W2 = 2 * W;
    const int oy = (int)(pix / W2), ox = (int)(pix % W2);
    const int64_t p = (int64_t)(oy >> 1) * W + (ox >> 1);
    const int t = (oy & 1) * 2 + (ox & 1);
    v4f v = *reinterpret_cast<const v4f*>(&D[p * 4 * Cout + (int64_t)t * Cout + co]);
    const v4f bb = *reinterpret_cast<const v4f*>(&b[co]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float s = v[j] + bb[j];
        v[j] = gelu ? gelu_erf(s) : s;
    }
    *reinterpret_cast<v4f*>(&y[pix * Cout + co]) = v;
}

// ggml_im2col for a 3x3 / stride 1 / pad 1 convolution on token-major input:
// cols[p][(ic*3 + kh)*3 + kw] = x[(oy + kh - 1)*W + ox + kw - 1][ic], zero
// outside the image; F32, or F16 rounded to nearest even (im2col in the
// kernel's type).
template <bool F16>
__global__ __launch_bounds__(256) void im2col3x3_kernel(const float* __restrict__ x, int H, int W, int C,
                                                        void* __restrict__ cols) {
    const int64_t K = 9LL * C;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)H * W * K) return;
    const int64_t p = i / K;
    const int k = (int)(i - p * K);
    const int ic = k / 9, tap = k - ic * 9;
    const int oy = (int)(p / W) + tap / 3 - 1, ox = (int)(p % W) + tap % 3 - 1;
    const float v = oy >= 0 && oy < H && ox >= 0 && ox < W ? x[((int64_t)oy * W + ox) * C + ic] : 0.0f;
    if (F16) static_cast<uint16_t*>(cols)[i] = f2h(v);
    else static_cast<float*>(cols)[i] = v;
}

// F32 3x3 kernel [Cout][Cin][3][3] (ggml [3, 3, Cin, Cout]) -> rows [Cout][tap][Cin],
// tap = kh*3 + kw: the K order of the implicit-GEMM convolution
__global__ __launch_bounds__(256) void conv3x3_pack_kernel(const float* __restrict__ w, int Cin, int Cout,
                                                           float* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= 9LL * Cin * Cout) return;
    const int ci = (int)(i % Cin);
    const int64_t r = i / Cin;
    const int tap = (int)(r % 9), co = (int)(r / 9);
    out[i] = w[((int64_t)co * Cin + ci) * 9 + tap];
}

// F16 3x3 kernel [Cout][Cin][3][3] -> rows [Cout][tap][Cin] (the implicit GEMM's K order)
__global__ __launch_bounds__(256) void conv3x3_pack_f16_kernel(const uint16_t* __restrict__ w, int Cin, int Cout,
                                                               uint16_t* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= 9LL * Cin * Cout) return;
    const int ci = (int)(i % Cin);
    const int64_t r = i / Cin;
    const int tap = (int)(r % 9), co = (int)(r / 9);
    out[i] = w[((int64_t)co * Cin + ci) * 9 + tap];
}

// ggml_conv_2d_s1_ph (TAPS = 9) or ggml_conv_2d_sk_p0 1x1 (TAPS = 1) with an F16
// kernel as an implicit GEMM: y[p][n] = bias[n] + sum_{tap, c} f16(x[p + tap
// offset][c]) * w[n][tap][c] over a token-major map (C % 32 == 0), zero outside
// the image.  TAPS = 4 is conv_transpose_2d_p0 (kernel 2, stride 2): the GEMM
// of the map with the deconv_pack rows [4*Cout][C], each column n = t*Cout + co
// stored to pixel (2py + t/2, 2px + t%2) of the 2x map as bias[co] + sum (then
// GELU-erf if gelu), the scatter of deconv_scatter_kernel done in registers.  The activations are rounded to fp16
// (RNE) as they are loaded, exactly as ggml's F16 im2col rounds them, so the
// products are those of im2col + F16 MUL_MAT; fp32 accumulation.
// Workgroup 128(m) x 128(n), four wavefronts of 64 x 64 (2 x 2
// v_mfma_f32_32x32x16_f16 tiles), K staged KST = 32 at a time (one tap's
// channel slice) through two LDS buffers.  The next
// stage's map values are held raw (fp32) in registers and rounded to fp16 as
// they are parked in LDS after the current stage's MFMAs, so their global
// latency overlaps the MFMAs.  Tile rows are KST halves (KST / 8 16-byte
// chunks), unpadded; chunk c of row r sits in slot c ^ csw(r), which spreads
// the rows of one ds_read_b128 pass over all 64 banks.
namespace {
constexpr int CT = 128;
template <int CH>
__device__ __forceinline__ int csw(int r) {
    return CH == 8 ? ((r & 7) ^ ((r >> 3) & 1)) : (((r >> 1) & 3) ^ ((r >> 3) & 1));
}
}
template <int TAPS, int KST>
__global__ __launch_bounds__(256, 2) void conv_f16_kernel(const float* __restrict__ x, const uint16_t* __restrict__ w,
                                                          const float* __restrict__ bias, int H, int W, int C, int N,
                                                          int gelu, float* __restrict__ y) {
    constexpr int CH = KST / 8, HC = CH / 2;  // chunks per row; chunks per loading thread
    __shared__ __attribute__((aligned(16))) _Float16 sA[2][CT * KST];
    __shared__ __attribute__((aligned(16))) _Float16 sB[2][CT * KST];
    const int M = H * W, K = TAPS == 9 ? 9 * C : C;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wv & 1, wn = wv >> 1;
    const int lr = lane & 31, g = lane >> 5;
    // XCD-aware tile order (each XCD a contiguous band of tiles)
    const int tiles_n = (N + CT - 1) / CT, tiles = ((M + CT - 1) / CT) * tiles_n;
    const int per_xcd = (tiles + 7) / 8;
    const int tl = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (tl >= tiles) return;
    const int m0 = (tl / tiles_n) * CT, n0 = (tl % tiles_n) * CT;
    // loader: thread t fills row t/2 of both tiles, chunks HC*(t%2) .. +HC-1 of the stage
    const int lrow = tid >> 1, lc = HC * (tid & 1);
    const int am = m0 + lrow, bn = n0 + lrow;
    const int oy = am / W, ox = am - (am / W) * W;
    v4f ra[2 * HC];
    uint4 rb[HC];
    auto load = [&](int k0) {
        const int tap = TAPS == 9 ? k0 / C : 0, c0 = k0 - tap * C;
        const int iy = TAPS == 9 ? oy + tap / 3 - 1 : oy, ix = TAPS == 9 ? ox + tap % 3 - 1 : ox;
        const bool in = am < M && iy >= 0 && iy < H && ix >= 0 && ix < W;
        const float* src = x + ((int64_t)iy * W + ix) * C + c0 + 8 * lc;
#pragma unroll
        for (int h = 0; h < 2 * HC; ++h) ra[h] = in ? *reinterpret_cast<const v4f*>(src + 4 * h) : v4f{0, 0, 0, 0};
        const uint4* ws = reinterpret_cast<const uint4*>(w + (int64_t)bn * K + k0 + 8 * lc);
#pragma unroll
        for (int h = 0; h < HC; ++h) rb[h] = bn < N ? ws[h] : uint4{0, 0, 0, 0};
    };
    auto park = [&](int buf) {
#pragma unroll
        for (int h = 0; h < HC; ++h) {
            const int slot = ((lc + h) ^ csw<CH>(lrow)) << 3;
            const v4f a = ra[2 * h], b = ra[2 * h + 1];
            const uint4 q = {(uint32_t)f2h(a[0]) | ((uint32_t)f2h(a[1]) << 16), (uint32_t)f2h(a[2]) | ((uint32_t)f2h(a[3]) << 16),
                             (uint32_t)f2h(b[0]) | ((uint32_t)f2h(b[1]) << 16), (uint32_t)f2h(b[2]) | ((uint32_t)f2h(b[3]) << 16)};
            *reinterpret_cast<uint4*>(&sA[buf][lrow * KST + slot]) = q;
            *reinterpret_cast<uint4*>(&sB[buf][lrow * KST + slot]) = rb[h];
        }
    };
    const v16f zf = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    v16f acc[2][2] = {{zf, zf}, {zf, zf}};
    const int nst = K / KST;
    load(0);
    park(0);
    __syncthreads();
    for (int s = 0; s < nst; ++s) {
        const int buf = s & 1;
        if (s + 1 < nst) load((s + 1) * KST);
#pragma unroll
        for (int kk = 0; kk < KST / 16; ++kk) {
            v8h a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int ra_ = wm * 64 + i * 32 + lr, rb_ = wn * 64 + i * 32 + lr, c = 2 * kk + g;
                a[i] = *reinterpret_cast<const v8h*>(&sA[buf][ra_ * KST + ((c ^ csw<CH>(ra_)) << 3)]);
                b[i] = *reinterpret_cast<const v8h*>(&sB[buf][rb_ * KST + ((c ^ csw<CH>(rb_)) << 3)]);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (s + 1 < nst) park(buf ^ 1);
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn * 64 + j * 32 + lr;
        if (n >= N) continue;
        if (TAPS == 4) {
            const int Cout = N >> 2, t = n / Cout, co = n - t * Cout;
            const float bv = bias[co];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                    if (m >= M) continue;
                    const int py = m / W, px = m - (m / W) * W;
                    const int64_t pix = (int64_t)(2 * py + (t >> 1)) * (2 * W) + 2 * px + (t & 1);
                    const float s = acc[i][j][r] + bv;
                    y[pix * Cout + co] = gelu ? gelu_erf(s) : s;
                }
        } else {
            const float bv = bias[n];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                    if (m < M) y[(int64_t)m * N + n] = acc[i][j][r] + bv;
                }
        }
    }
}

// conv_f16_kernel's implicit GEMM with its operands staged by LDS DMA (buffer_load ... lds):
// per 32-deep K step the fp32 map rows (128 bytes of one tap's channel slice per output
// pixel, zero by the buffer's range check outside the image or past M) and the fp16 weight
// rows (64 bytes), two stage buffers (48 KB: three workgroups per CU; three buffers filled
// two stages ahead left two per CU and measured slower), no staging registers.  The
// map is rounded to fp16 (RNE, f2h) as the MFMA fragments are read from LDS: the operands,
// products and accumulation order of conv_f16_kernel, so the same bits.
// LDS rows: map rows of 8 chunks of 16 bytes, chunk c of row r in slot c ^ ((r >> 1) & 7),
// so the 16 rows of a ds_read_b128 quarter (rows of two parities) cover all 64 banks;
// weight rows as conv_f16_kernel's (csw<4>).
namespace {
struct ConvDmaStage {
    float A[CT * 32];     // 128 map rows x 32 channels, fp32
    uint16_t B[CT * 32];  // 128 weight rows x 32 K, fp16
};
constexpr int CONV_OOB = 0x7ffffff0;
constexpr int CONV_NB = 2;  // stage buffers  // a buffer offset past every operand the launcher admits
__device__ __forceinline__ int aswz(int r) { return (r >> 1) & 7; }
}  // namespace

// AH: the map is fp16 already (a producer of this file rounded it, RNE): its rows are 64 bytes
// per stage, staged and read as the weights are, with no conversion. OH: the output is fp16
// (the f32 result rounded, RNE), for a map only another of these kernels reads.
template <int TAPS, int NB, bool AH = false, bool OH = false>
__global__ __launch_bounds__(256, NB == 3 ? 2 : 3) void conv_f16_dma_kernel(const void* __restrict__ xv, const uint16_t* __restrict__ w,
                                                              const float* __restrict__ bias, int H, int W, int C, int N,
                                                              int gelu, void* __restrict__ yv, int ksplit, int sps,
                                                              float* __restrict__ part) {
    constexpr int NL = AH ? 4 : 6;  // DMA instructions per wavefront and stage: 4 (fp16: 2) map, 2 weight
    constexpr int NA = AH ? 2 : 4;  // map DMA instructions per wavefront and stage
    __shared__ __attribute__((aligned(16))) ConvDmaStage sb[NB];
    const int M = H * W, K = TAPS == 9 ? 9 * C : C, cps = C / 32;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wv & 1, wn = wv >> 1;
    const int lr = lane & 31, g = lane >> 5;
    // XCD-aware tile order (each XCD a contiguous band of tiles); with a K split (taps 1 and
    // 9) the split is the slowest index: slot (split, tile) runs stages [split * sps, + sps)
    const int tiles_n = (N + CT - 1) / CT, tiles = ((M + CT - 1) / CT) * tiles_n;
    const int TT = tiles * ksplit, per_xcd = (TT + 7) / 8;
    const int tls = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (tls >= TT) return;
    const int split = tls / tiles, tl = tls - split * tiles;
    const int m0 = (tl / tiles_n) * CT, n0 = (tl % tiles_n) * CT;

    // map DMA instruction j of wavefront wv: tile rows 8 (4 wv + j) + lane / 8, LDS slot lane % 8,
    // global chunk slot ^ aswz(row) (fp16 map: rows 16 (2 wv + j) + lane / 4, slot lane % 4, as
    // the weights); weight instruction j: rows 16 (2 wv + j) + lane / 4, slot lane % 4
    constexpr int XES = AH ? 2 : 4;  // map element bytes
    const v4i xr = make_rsrc(xv, (int64_t)M * C * XES), wr = make_rsrc(w, (int64_t)N * K * 2);
    int py[NA], px[NA], ach[NA];
#pragma unroll
    for (int j = 0; j < NA; ++j) {
        const int row = AH ? 16 * (2 * wv + j) + (lane >> 2) : 8 * (4 * wv + j) + (lane >> 3), p = m0 + row;
        py[j] = p < M ? p / W : -(1 << 20);  // past M: every tap lands outside the image
        px[j] = p < M ? p - (p / W) * W : 0;
        ach[j] = AH ? (((lane & 3) ^ csw<4>(row)) << 4) : (((lane & 7) ^ aswz(row)) << 4);
    }
    int woff[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int row = 16 * (2 * wv + j) + (lane >> 2), n = n0 + row;
        woff[j] = n < N ? n * K * 2 + (((lane & 3) ^ csw<4>(row)) << 4) : CONV_OOB;
    }
    uint32_t lb[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) lb[i] = (uint32_t)__builtin_amdgcn_readfirstlane(lds_addr(&sb[i]));
    auto dma = [&](int s, uint32_t base) __attribute__((always_inline)) {
        const int tap = TAPS == 9 ? s / cps : 0, c0 = (s - tap * cps) * 32;
        const int dy = TAPS == 9 ? tap / 3 - 1 : 0, dx = TAPS == 9 ? tap % 3 - 1 : 0;
#pragma unroll
        for (int j = 0; j < NA; ++j) {
            const int iy = py[j] + dy, ix = px[j] + dx;
            const bool in = iy >= 0 && iy < H && ix >= 0 && ix < W;
            const int off = in ? ((iy * W + ix) * C + c0) * XES + ach[j] : CONV_OOB;
            dma_b128_so(xr, base + (uint32_t)offsetof(ConvDmaStage, A) + 1024u * (NA * wv + j), off, 0);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j)
            dma_b128_so(wr, base + (uint32_t)offsetof(ConvDmaStage, B) + 1024u * (2 * wv + j), woff[j], s * 64);
    };

    const v16f zf = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    v16f acc[2][2] = {{zf, zf}, {zf, zf}};
    auto compute = [&](const ConvDmaStage& b) __attribute__((always_inline)) {
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            v8h a[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int ra = wm * 64 + i * 32 + lr, rb = wn * 64 + i * 32 + lr;
                if (AH) {
                    const uint16_t* ah = reinterpret_cast<const uint16_t*>(b.A);
                    a[i] = *reinterpret_cast<const v8h*>(&ah[ra * 32 + (((2 * kk + g) ^ csw<4>(ra)) << 3)]);
                } else {
                    const int c = 4 * kk + 2 * g;  // the lane's 8 channels: chunks c, c + 1 of its map row
                    const v4f lo = *reinterpret_cast<const v4f*>(&b.A[ra * 32 + ((c ^ aswz(ra)) << 2)]);
                    const v4f hi = *reinterpret_cast<const v4f*>(&b.A[ra * 32 + (((c + 1) ^ aswz(ra)) << 2)]);
                    const uint4 q = {(uint32_t)f2h(lo[0]) | ((uint32_t)f2h(lo[1]) << 16), (uint32_t)f2h(lo[2]) | ((uint32_t)f2h(lo[3]) << 16),
                                     (uint32_t)f2h(hi[0]) | ((uint32_t)f2h(hi[1]) << 16), (uint32_t)f2h(hi[2]) | ((uint32_t)f2h(hi[3]) << 16)};
                    a[i] = __builtin_bit_cast(v8h, q);
                }
                bf[i] = *reinterpret_cast<const v8h*>(&b.B[rb * 32 + (((2 * kk + g) ^ csw<4>(rb)) << 3)]);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], bf[j], acc[i][j], 0, 0, 0);
        }
    };

    const int s0 = split * sps, nst = min(K / 32 - s0, sps);  // this split's first stage and stage count
    // NB buffers filled NB - 1 stages ahead
    dma(s0, lb[0]);
    if (nst > 1) dma(s0 + 1, lb[1]);
    if (NB == 3 && nst > 2) dma(s0 + 2, lb[NB - 1]);
    if (NB == 3 && nst > 2) wait_vmcnt<2 * NL>();
    else if (nst > 1) wait_vmcnt<NL>();
    else wait_vmcnt<0>();
    __syncthreads();
    for (int s = 0; s < nst; ++s) {
        const int cb = s % NB;
        compute(sb[cb]);
        if (s + 1 < nst) {
            if (NB == 3 && s + 2 < nst) wait_vmcnt<NL>();  // stage s + 1 has landed (s + 2 may be in flight)
            else wait_vmcnt<0>();
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // and stage s's buffer is read
            if (s + NB < nst) dma(s0 + s + NB, lb[cb]);
        }
    }
    if (TAPS != 4 && ksplit > 1) {  // this split's partial sums, no bias: part [split][M][N]
        float* P = part + (int64_t)split * M * N;
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
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn * 64 + j * 32 + lr;
        if (n >= N) continue;
        if (TAPS == 4) {
            const int Cout = N >> 2, t = n / Cout, co = n - t * Cout;
            const float bv = bias[co];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                    if (m >= M) continue;
                    const int qy = m / W, qx = m - (m / W) * W;
                    const int64_t pix = (int64_t)(2 * qy + (t >> 1)) * (2 * W) + 2 * qx + (t & 1);
                    const float sv = acc[i][j][r] + bv;
                    const float o = gelu ? gelu_erf(sv) : sv;
                    if (OH) static_cast<uint16_t*>(yv)[pix * Cout + co] = f2h(o);
                    else static_cast<float*>(yv)[pix * Cout + co] = o;
                }
        } else {
            const float bv = bias[n];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                    if (m >= M) continue;
                    const float o = acc[i][j][r] + bv;
                    if (OH) static_cast<uint16_t*>(yv)[(int64_t)m * N + n] = f2h(o);
                    else static_cast<float*>(yv)[(int64_t)m * N + n] = o;
                }
        }
    }
}

// y[r][c] += b[c], four channels per thread (C % 4 == 0)
__global__ __launch_bounds__(256) void bias_rows_kernel(float* __restrict__ y, const float* __restrict__ b, int64_t rows,
                                                        int C) {
    const int c4 = C / 4;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * c4) return;
    const int c = (int)(i % c4) * 4;
    v4f v = *reinterpret_cast<const v4f*>(&y[i * 4]);
    const v4f bb = *reinterpret_cast<const v4f*>(&b[c]);
    *reinterpret_cast<v4f*>(&y[i * 4]) = v + bb;
}

// ggml_pool_2d MAX, 2x2 window, stride 2, no padding: four channels per thread
__global__ __launch_bounds__(256) void maxpool2_kernel(const float* __restrict__ x, int H, int W, int C,
                                                       float* __restrict__ y) {
    const int c4 = C / 4, H2 = H / 2, W2 = W / 2;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)H2 * W2 * c4) return;
    const int c = (int)(i % c4) * 4;
    const int64_t q = i / c4;
    const int py = (int)(q / W2), px = (int)(q % W2);
    const float* s = x + ((int64_t)(2 * py) * W + 2 * px) * C + c;
    const v4f a = *reinterpret_cast<const v4f*>(s), b = *reinterpret_cast<const v4f*>(s + C);
    const v4f d = *reinterpret_cast<const v4f*>(s + (int64_t)W * C), e = *reinterpret_cast<const v4f*>(s + (int64_t)W * C + C);
    v4f m;
#pragma unroll
    for (int j = 0; j < 4; ++j) m[j] = fmaxf(fmaxf(a[j], b[j]), fmaxf(d[j], e[j]));
    *reinterpret_cast<v4f*>(&y[q * C + c]) = m;
}

hipError_t launch_deconv_pack(const void* w, int wtype, int Cin, int Cout, uint16_t* out, hipStream_t st) {
    const int64_t n = 4LL * Cout * Cin;
    if (n > 0) deconv_pack_kernel<<<nblk(n), 256, 0, st>>>(w, wtype, Cin, Cout, out);
    return hipGetLastError();
}

hipError_t launch_deconv_scatter(const float* D, const float* b, int H, int W, int Cout, bool gelu, float* y,
                                 hipStream_t st) {
    if (Cout % 4 != 0) return hipErrorInvalidValue;
    const int64_t n = 4LL * H * W * (Cout / 4);
    if (n > 0) deconv_scatter_kernel<<<nblk(n), 256, 0, st>>>(D, b, H, W, Cout, gelu ? 1 : 0, y);
    return hipGetLastError();
}

hipError_t launch_im2col3x3(const float* x, int H, int W, int C, bool f16, void* cols, hipStream_t st) {
    const int64_t n = (int64_t)H * W * 9 * C;
    if (n <= 0) return hipSuccess;
    if (f16) im2col3x3_kernel<true><<<nblk(n), 256, 0, st>>>(x, H, W, C, cols);
    else im2col3x3_kernel<false><<<nblk(n), 256, 0, st>>>(x, H, W, C, cols);
    return hipGetLastError();
}

hipError_t launch_conv3x3_pack(const float* w, int Cin, int Cout, float* out, hipStream_t st) {
    const int64_t n = 9LL * Cin * Cout;
    if (n > 0) conv3x3_pack_kernel<<<nblk(n), 256, 0, st>>>(w, Cin, Cout, out);
    return hipGetLastError();
}

hipError_t launch_conv3x3_pack_f16(const uint16_t* w, int Cin, int Cout, uint16_t* out, hipStream_t st) {
    const int64_t n = 9LL * Cin * Cout;
    if (n > 0) conv3x3_pack_f16_kernel<<<nblk(n), 256, 0, st>>>(w, Cin, Cout, out);
    return hipGetLastError();
}

namespace {
// operands the DMA kernel's 32-bit buffer offsets reach (with the out-of-range offset above)
bool conv_dma_ok(int taps, int64_t M, int64_t C, int64_t N) {
    return M * C * 4 < CONV_OOB - 4096 && N * (taps == 9 ? 9 : 1) * C * 2 < CONV_OOB - 4096;
}
// K split of the DMA kernel (taps 1 and 9): grids below one tile per CU; one 32-deep stage of
// a tile takes about 0.9 us alone on a CU
int conv_f16_ksplit(int taps, int64_t M, int64_t C, int64_t N) {
    if (taps == 4 || !conv_dma_ok(taps, M, C, N)) return 1;
    const int64_t tiles = ((M + CT - 1) / CT) * ((N + CT - 1) / CT);
    return gemm_ksplit(tiles, 256, M, N, (taps == 9 ? 9 : 1) * C / 32, 0.9);
}
}  // namespace

size_t conv_f16_part_bytes(int taps, int64_t M, int64_t C, int64_t N) {
    const int S = conv_f16_ksplit(taps, M, C, N);
    return S > 1 ? (size_t)S * (size_t)M * (size_t)N * 4 : 0;
}

hipError_t launch_conv_f16(int taps, const void* x, bool x16, const uint16_t* w, const float* bias, int H, int W, int C,
                           int N, bool gelu, void* y, bool y16, hipStream_t st, float* part, size_t part_bytes) {
    if ((taps != 1 && taps != 4 && taps != 9) || C % 32 != 0 || (reinterpret_cast<uintptr_t>(x) & 15) ||
        (reinterpret_cast<uintptr_t>(w) & 15) || (taps == 4 && N % 4 != 0))
        return hipErrorInvalidValue;
    const int64_t M = (int64_t)H * W;
    if (M <= 0 || N <= 0) return hipSuccess;
    const int tiles = (int)(((M + CT - 1) / CT) * ((N + CT - 1) / CT));
    const unsigned grid = (unsigned)((tiles + 7) / 8 * 8);
    const int gl = gelu ? 1 : 0;
    if (conv_dma_ok(taps, M, C, N)) {
        // the K split, when the caller gave room for its partial sums
        // (the reduce stores float4 rows: y and part on 16 bytes; N % 4 == 0 in the split choice)
        const bool a16 = ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(part) |
                           reinterpret_cast<uintptr_t>(bias)) & 15) == 0;
        int S = part && a16 ? conv_f16_ksplit(taps, M, C, N) : 1;
        if ((size_t)S * (size_t)M * (size_t)N * 4 > part_bytes) S = 1;
        const int nst = (taps == 9 ? 9 : 1) * C / 32, sps = (nst + S - 1) / S;
        const unsigned gs = (unsigned)((tiles * S + 7) / 8 * 8);
        // the map formats the neck uses: F32 in and out (the per-op entry points), and in the
        // fused neck fp16 intermediates (a 3x3 reads one and writes a neck output; a
        // conv-transpose or 1x1 reads the ViT output, the pool output or one, and writes one;
        // with F32 convolution kernels scale 0's second conv-transpose reads one, writes F32)
        const int f = (x16 ? 2 : 0) + (y16 ? 1 : 0);
        if (taps == 9 && f == 0) conv_f16_dma_kernel<9, CONV_NB><<<gs, 256, 0, st>>>(x, w, bias, H, W, C, N, gl, y, S, sps, part);
        else if (taps == 9 && f == 2) conv_f16_dma_kernel<9, CONV_NB, true, false><<<gs, 256, 0, st>>>(x, w, bias, H, W, C, N, gl, y, S, sps, part);
        else if (taps == 4 && f == 0) conv_f16_dma_kernel<4, CONV_NB><<<grid, 256, 0, st>>>(x, w, bias, H, W, C, N, gl, y, 1, nst, nullptr);
        else if (taps == 4 && f == 1) conv_f16_dma_kernel<4, CONV_NB, false, true><<<grid, 256, 0, st>>>(x, w, bias, H, W, C, N, gl, y, 1, nst, nullptr);
        else if (taps == 4 && f == 3) conv_f16_dma_kernel<4, CONV_NB, true, true><<<grid, 256, 0, st>>>(x, w, bias, H, W, C, N, gl, y, 1, nst, nullptr);
        else if (taps == 4 && f == 2) conv_f16_dma_kernel<4, CONV_NB, true, false><<<grid, 256, 0, st>>>(x, w, bias, H, W, C, N, gl, y, 1, nst, nullptr);
        else if (taps == 1 && f == 0) conv_f16_dma_kernel<1, CONV_NB><<<gs, 256, 0, st>>>(x, w, bias, H, W, C, N, gl, y, S, sps, part);
        else if (taps == 1 && f == 1) conv_f16_dma_kernel<1, CONV_NB, false, true><<<gs, 256, 0, st>>>(x, w, bias, H, W, C, N, gl, y, S, sps, part);
        else if (taps == 1 && f == 3) conv_f16_dma_kernel<1, CONV_NB, true, true><<<gs, 256, 0, st>>>(x, w, bias, H, W, C, N, gl, y, S, sps, part);
        else return hipErrorInvalidValue;
        const hipError_t e = hipGetLastError();
        if (S == 1 || e != hipSuccess) return e;
        return launch_split_reduce(part, S, (int)M, N, bias, static_cast<float*>(y), (y16 ? 2LL : 4LL) * N, st, y16);
    }
    // K step 32: a 64-deep step (64 KB of LDS, two workgroups per CU) measured slower
    if (x16 || y16) return hipErrorInvalidValue;  // fp16 maps: the DMA kernel only
    const float* xf = static_cast<const float*>(x);
    float* yf = static_cast<float*>(y);
    if (taps == 9)
        conv_f16_kernel<9, 32><<<grid, 256, 0, st>>>(xf, w, bias, H, W, C, N, gl, yf);
    else if (taps == 4)
        conv_f16_kernel<4, 32><<<grid, 256, 0, st>>>(xf, w, bias, H, W, C, N, gl, yf);
    else
        conv_f16_kernel<1, 32><<<grid, 256, 0, st>>>(xf, w, bias, H, W, C, N, gl, yf);
    return hipGetLastError();
}

hipError_t launch_bias_rows(float* y, const float* b, int64_t rows, int C, hipStream_t st) {
    if (C % 4 != 0) return hipErrorInvalidValue;
    const int64_t n = rows * (C / 4);
    if (n > 0) bias_rows_kernel<<<nblk(n), 256, 0, st>>>(y, b, rows, C);
    return hipGetLastError();
}

hipError_t launch_maxpool2(const float* x, int H, int W, int C, float* y, hipStream_t st) {
    if (C % 4 != 0) return hipErrorInvalidValue;
    const int64_t n = (int64_t)(H / 2) * (W / 2) * (C / 4);
    if (n > 0) maxpool2_kernel<<<nblk(n), 256, 0, st>>>(x, H, W, C, y);
    return hipGetLastError();
}

}  // namespace mi355
