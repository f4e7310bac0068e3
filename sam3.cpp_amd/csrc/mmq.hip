// ggml MUL_MAT on gfx950 MFMA for Q8_0 / Q4_0 / Q4_1 / F16 weights.
//
// Quantized weights:
//   dst[m][n] = sum_b fp32(d_w[n][b]) * fp32(d_a[m][b]) * isum[m][n][b]
//               (+ sum_b fp32(m_w[n][b]) * fp32(s_a[m][b]) for Q4_1)
//   isum[m][n][b] = sum_{j<32} q_w[n][32b+j] * q_a[m][32b+j]
// Both operands' quants are staged as fp16 (integers up to |127| are exact),
// so two chained v_mfma_f32_32x32x16_f16 give isum exactly (every partial
// sum is an integer below 2^24).  The scale product d_a (x) d_w of a 32x32
// tile is one more MFMA (outer product in k-slot 0; fp16 x fp16 is exact in
// fp32), which leaves one fp32 FMA per output element and block on the VALU:
// acc = fma(isum, S, acc).  The Q4_1 offset term sum_b m_w s_a is a plain
// fp16 GEMM over blocks, accumulated straight into acc by MFMA.
//
// F16 weights: the same tiles, acc = MFMA(a, w, acc) over k.
//
// Tiling: workgroup 128(m) x 128(n), four wavefronts; wavefront w owns all
// 128 rows and the 32 columns n0+32w..+31 (4 MFMA tiles along m).  K
// advances two blocks (64 elements) per stage with one barrier per stage:
// the next stage's global loads are issued into registers before the
// current stage's MFMAs and written to the other LDS buffer after them.
// All global traffic uses buffer loads: every per-thread offset is computed
// once, a stage advances only the (scalar) base of the buffer resource, and
// rows past M/N read as zeros through the resource's range check.  Weight
// stage segments (2 blocks = 68/36/40 bytes per row) are fetched as
// consecutive dwords across lanes (~4 rows per load instruction) and parked
// raw in LDS; each wavefront decodes its own MFMA weight fragments from
// them (byte -> 0x64XX half -> packed f16 subtract).  Workgroups are
// numbered so each XCD (round-robin dispatch) walks n-tiles of its own band
// of m-tiles.
#include "common.cuh"
#include "kernels.h"

namespace mi355 {

namespace {
constexpr int BM = 128, BN = 128, BKB = 2, BKH = BKB * QK;
constexpr int NT = 256;
constexpr int OOB = 0x40000000;  // voffset past any range: buffer loads return 0
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
}  // namespace

template <int WT> struct WInfo;
template <> struct WInfo<T_Q8_0> { static constexpr int bytes = 34, hdr = 2; };
template <> struct WInfo<T_Q4_0> { static constexpr int bytes = 18, hdr = 2; };
template <> struct WInfo<T_Q4_1> { static constexpr int bytes = 20, hdr = 4; };

// Raw buffer resource over [base, base + bytes): gfx9 dword3 = 0x00020000.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
    const int32_t n = bytes <= 0 ? 0 : (bytes > 0x7fffffffLL ? 0x7fffffff : (int32_t)bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}

__device__ __forceinline__ uint32_t h2_sub(uint32_t v, _Float16 c) {
    h2 x = __builtin_bit_cast(h2, v);
    x = x - h2{c, c};
    return __builtin_bit_cast(uint32_t, x);
}
// 4 bytes (offset-binary or nibble values 0..255) -> 4 halves (1024 + byte) - bias.
__device__ __forceinline__ void bytes_to_h4(uint32_t u, _Float16 bias, uint32_t& h01, uint32_t& h23) {
    h01 = h2_sub(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u), bias);
    h23 = h2_sub(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u), bias);
}

struct MmqArgs {
    const uint8_t* W;
    int64_t w_nb1, w_nb2, w_nb3;
    int64_t w_extent;          // bytes of one src0 slice ((N-1)*nb1 + row size)
    const _Float16* A;         // activations (fp16 values), row stride a_s1 halves
    int64_t a_s1, a_s2, a_s3;
    int64_t a_extent;          // bytes of one activation slice ((M-1)*s1 + K halves)
    const _Float16* Ad;        // [Z][nb][M] activation scales (quantized path)
    const _Float16* As;        // [Z][nb][M] Q8_1 sums (Q4_1 path)
    float* D;
    int64_t d_nb1, d_nb2, d_nb3;
    int32_t* dots;             // block-dot inspection output (or null)
    int M, Mp, N, K, ne12, r2, r3, tiles_m, tiles_n;  // Mp: padded row count of the scale arrays
};

// 8 consecutive int8 quants (two dwords) -> 8 fp16 (one MFMA k-chunk).
__device__ __forceinline__ v8h i8x8_to_h8(uint32_t w0, uint32_t w1) {
    uint32_t h[4];
    bytes_to_h4(w0 ^ 0x80808080u, (_Float16)1152.0f, h[0], h[1]);
    bytes_to_h4(w1 ^ 0x80808080u, (_Float16)1152.0f, h[2], h[3]);
    return __builtin_bit_cast(v8h, v4i{(int)h[0], (int)h[1], (int)h[2], (int)h[3]});
}
// 8 nibble values (one per byte, 0..15) -> 8 fp16 of (value - bias).
__device__ __forceinline__ v8h n8_to_h8(uint32_t w0, uint32_t w1, _Float16 bias) {
    uint32_t h[4];
    bytes_to_h4(w0, bias, h[0], h[1]);
    bytes_to_h4(w1, bias, h[2], h[3]);
    return __builtin_bit_cast(v8h, v4i{(int)h[0], (int)h[1], (int)h[2], (int)h[3]});
}
// Two dwords starting at byte offset o of an LDS row; sh = o % 4 is 0 or 2 and
// known at compile time after unrolling.
__device__ __forceinline__ void lds_dw2(const uint32_t* row, int o, int sh, uint32_t& w0, uint32_t& w1) {
    const uint32_t* q = row + (o >> 2);
    if (sh == 0) {
        w0 = q[0];
        w1 = q[1];
    } else {
        const uint32_t r0 = q[0], r1 = q[1], r2 = q[2];
        w0 = __builtin_amdgcn_alignbyte(r1, r0, 2);
        w1 = __builtin_amdgcn_alignbyte(r2, r1, 2);
    }
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Workgroup 128(m) x 128(n); wavefront w owns all 128 rows of m and the 32
// columns n0 + 32w .. +31 (4 MFMA tiles stacked along m).  Every stage's
// operands are DMA'd from global memory straight into LDS (buffer_load ...
// lds): no staging registers, no LDS store instructions.  Per stage each
// wavefront issues its share of the next stage's DMA into the other buffer
// right after the barrier and then runs the current stage's MFMAs; one
// vmcnt(0) + barrier per stage.
//   activation tile: 128 rows x 64 halves, unpadded; 16-byte chunk c of row r
//     sits in slot c ^ (r & 7), so a 32-row MFMA fragment read hits 8
//     distinct slots (no bank conflicts) while each DMA lane still writes
//     16 contiguous bytes;
//   raw weight segments: lane-linear dwords (row j / RD, dword j % RD);
//     each wavefront decodes its own 32 weight rows' fragments on the fly;
//   activation scales (and Q8_1 sums): 128 fp16 per block, one dword per lane.
template <int WT, bool DOTS>
__global__ __launch_bounds__(NT, 2) void mmq_kernel(const MmqArgs p) {
    constexpr bool QUANT = WT != T_F16;
    constexpr int QT = WT == T_F16 ? T_Q8_0 : WT;
    constexpr int WB = WInfo<QT>::bytes, HDR = WInfo<QT>::hdr;
    constexpr int RD = (2 * WB) / 4;             // dwords of a row's 2-block stage segment
    constexpr int RLD = (BN * RD + NT - 1) / NT; // raw dword DMA instructions per wavefront
    constexpr int MT = BM / 32;                  // m tiles per wavefront
    constexpr int TH = BM * BKH;                 // halves per activation tile
    __shared__ __attribute__((aligned(16))) _Float16 sA[2][TH];
    __shared__ __attribute__((aligned(16))) _Float16 sBf[QUANT ? 1 : 2][QUANT ? 8 : BN * BKH];
    __shared__ __attribute__((aligned(16))) uint32_t sW[QUANT ? 2 : 1][QUANT ? RLD * NT : 4];
    __shared__ __attribute__((aligned(16))) _Float16 sAd[2][BKB][BM];
    __shared__ __attribute__((aligned(16))) _Float16 sAs[WT == T_Q4_1 ? 2 : 1][BKB][BM];
    __shared__ __attribute__((aligned(16))) _Float16 sZero[2 * BKB * BM];  // S-operand lanes 32..63

    // XCD-aware tile order: workgroup id -> (xcd, slot) -> contiguous tile band per XCD
    const int T = p.tiles_m * p.tiles_n;
    const int per_xcd = (T + 7) / 8;
    const int t = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (t >= T) return;
    const int m0 = (t / p.tiles_n) * BM, n0 = (t % p.tiles_n) * BN;

    const int tid = threadIdx.x, lane = tid & 63, wn = tid >> 6;
    const int z = blockIdx.y, i12 = z % p.ne12, i13 = z / p.ne12;
    const int M = p.M, N = p.N, K = p.K;
    const int nb = K / QK;
    const int nstage = QUANT ? (nb + BKB - 1) / BKB : (K + BKH - 1) / BKH;
    const uint8_t* Wz = p.W + (int64_t)(i12 / p.r2) * p.w_nb2 + (int64_t)(i13 / p.r3) * p.w_nb3;
    const _Float16* Az = p.A + (int64_t)i12 * p.a_s2 + (int64_t)i13 * p.a_s3;
    const int Mp = p.Mp;
    const _Float16* Adz = QUANT ? p.Ad + (int64_t)z * nb * Mp : nullptr;
    const _Float16* Asz = WT == T_Q4_1 ? p.As + (int64_t)z * nb * Mp : nullptr;

    // ---- DMA offsets, fixed for the whole K loop
    // activation / F16-weight tile, instruction i of wavefront w: rows (4w+i)*8 + lane/8,
    // slot lane%8 <- chunk (lane%8) ^ (lane/8)
    const int trow = lane >> 3, tchunk = (lane & 7) ^ (lane >> 3);
    int aoff[4], foff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = (wn * 4 + i) * 8 + trow;
        aoff[i] = m0 + row < M ? ((m0 + row) * (int)p.a_s1 + tchunk * 8) * 2 : OOB;
        foff[i] = !QUANT && n0 + row < N ? (n0 + row) * (int)p.w_nb1 + tchunk * 16 : OOB;
    }
    int woff[QUANT ? RLD : 1];  // raw weight dword j = NT*i + 64w + lane -> (row j / RD, dword j % RD)
#pragma unroll
    for (int i = 0; i < (QUANT ? RLD : 1); ++i) {
        const int j = tid + NT * i, row = j / RD, c = j - row * RD;
        woff[i] = QUANT && j < BN * RD && n0 + row < N ? (n0 + row) * (int)p.w_nb1 + 4 * c : OOB;
    }

    auto dma_stage = [&](int s, int buf) {
        const int k0 = s * BKH;
        const bool tail = k0 + BKH > K;  // chunks past K must read zeros (rows continue in memory)
        const bool cvalid = k0 + tchunk * 8 < K;
        const auto ar = make_rsrc(Az + k0, p.a_extent - 2LL * k0);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ar, (lds_ptr_t)&sA[buf][(wn * 4 + i) * 8 * BKH], 16,
                                                     tail && !cvalid ? OOB : aoff[i], 0, 0, 0);
        if (QUANT) {
            const int64_t seg = (int64_t)s * BKB * WB;
            const auto wrs = make_rsrc(Wz + seg, p.w_extent - seg);
#pragma unroll
            for (int i = 0; i < RLD; ++i)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (lds_ptr_t)&sW[buf][NT * i + 64 * wn], 4, woff[i], 0, 0, 0);
            // scales of blocks 2s, 2s+1: wavefronts 0, 1 (d) and, for Q8_1, 2, 3 (s)
            const int b = wn & 1;
            const int64_t so = (int64_t)(s * BKB + b) * Mp + m0;  // halves
            if (wn < 2) {
                const auto dr = make_rsrc(Adz + so, 2LL * ((int64_t)nb * Mp - so));
                __builtin_amdgcn_raw_ptr_buffer_load_lds(dr, (lds_ptr_t)&sAd[buf][b][0], 4, lane * 4, 0, 0, 0);
            } else if (WT == T_Q4_1) {
                const auto sr = make_rsrc(Asz + so, 2LL * ((int64_t)nb * Mp - so));
                __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (lds_ptr_t)&sAs[buf][b][0], 4, lane * 4, 0, 0, 0);
            }
        } else {
            const auto fr = make_rsrc(Wz + 2LL * k0, p.w_extent - 2LL * k0);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(fr, (lds_ptr_t)&sBf[buf][(wn * 4 + i) * 8 * BKH], 16,
                                                         tail && !cvalid ? OOB : foff[i], 0, 0, 0);
        }
    };

    v16f acc[MT];
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[a][i] = 0.0f;
    const v16f zf = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    const int lr = lane & 31, g = lane >> 5;  // fragment row, lane group
    const int wrow = wn * 32 + lr;           // this lane's weight row in the tile
    const uint16_t* zero16 = reinterpret_cast<const uint16_t*>(&sZero[0]);
    // S-operand activation scales: lanes 0..31 read sAd, lanes 32..63 the zero mirror
    const uint16_t* da_src = lane < 32 ? reinterpret_cast<const uint16_t*>(&sAd[0][0][0]) : zero16;
    const uint16_t* sa_src = lane < 32 ? reinterpret_cast<const uint16_t*>(&sAs[0][0][0]) : zero16;
    if (QUANT) {
        for (int i = tid; i < 2 * BKB * BM; i += NT) sZero[i] = (_Float16)0.0f;
    }
    // fragment of row r, 8-half chunk c in a swizzled tile
    auto frag = [&](const _Float16* tile, int r, int c) -> v8h {
        return *reinterpret_cast<const v8h*>(&tile[r * BKH + ((c ^ (r & 7)) << 3)]);
    };

    dma_stage(0, 0);
    for (int s = 0; s < nstage; ++s) {
        const int cur = s & 1;
        __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0): this wavefront's DMA for stage s landed
        __syncthreads();                     // ... and everyone's; stage s-1 buffers are free
        if (s + 1 < nstage) dma_stage(s + 1, cur ^ 1);
        if (QUANT) {
            const uint32_t* rowp = &sW[cur][wrow * RD];
            const uint16_t* hsrc = lane < 32 ? reinterpret_cast<const uint16_t*>(rowp) : zero16;
#pragma unroll
            for (int b = 0; b < BKB; ++b) {
                if (DOTS && s * BKB + b >= nb) break;
                // this lane's weight fragments: row wrow, k-chunk 8g..8g+7 of each 16-wide half.
                // A block past K (odd block count) runs with d_a = 0: S = 0 leaves acc unchanged.
                v8h bf[2];
                if (WT == T_Q8_0) {
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        uint32_t w0, w1;
                        lds_dw2(rowp, b * WB + HDR + 16 * h + 8 * g, (b * WB + HDR) & 3, w0, w1);
                        bf[h] = i8x8_to_h8(w0, w1);
                    }
                } else {
                    uint32_t w0, w1;  // payload bytes 8g..8g+7: low nibbles = half 0, high = half 1
                    lds_dw2(rowp, b * WB + HDR + 8 * g, (b * WB + HDR) & 3, w0, w1);
                    const _Float16 bias = WT == T_Q4_0 ? (_Float16)1032.0f : (_Float16)1024.0f;
                    bf[0] = n8_to_h8(w0 & 0x0f0f0f0fu, w1 & 0x0f0f0f0fu, bias);
                    bf[1] = n8_to_h8((w0 >> 4) & 0x0f0f0f0fu, (w1 >> 4) & 0x0f0f0f0fu, bias);
                }
                const v4i dwf = {(int)(uint32_t)hsrc[b * WB / 2], 0, 0, 0};
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const int ar_ = mt * 32 + lr;
                    const v8h a0 = frag(sA[cur], ar_, 4 * b + g);
                    const v8h a1 = frag(sA[cur], ar_, 4 * b + 2 + g);
                    v16f I = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, bf[0], zf, 0, 0, 0);
                    I = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, bf[1], I, 0, 0, 0);
                    if (DOTS) {
                        const int n = n0 + wrow;
#pragma unroll
                        for (int i = 0; i < 16; ++i) {
                            const int m = m0 + mt * 32 + 8 * (i >> 2) + 4 * g + (i & 3);
                            if (m < M && n < N) p.dots[(((int64_t)z * M + m) * N + n) * nb + s * BKB + b] = (int32_t)I[i];
                        }
                        continue;
                    }
                    const v4i daf = {(int)(uint32_t)da_src[(cur * BKB + b) * BM + ar_], 0, 0, 0};
                    const v16f S = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                        __builtin_bit_cast(v8h, daf), __builtin_bit_cast(v8h, dwf), zf, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 16; ++i) acc[mt][i] = __builtin_fmaf(I[i], S[i], acc[mt][i]);
                }
            }
            if (WT == T_Q4_1 && !DOTS) {
                // acc += sum_b s_a[m][b] * m_w[n][b] over this stage's blocks (k-slots 0, 1)
                const v4i mwf = {(int)((uint32_t)hsrc[1] | ((uint32_t)hsrc[WB / 2 + 1] << 16)), 0, 0, 0};
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const int ar_ = mt * 32 + lr;
                    const v4i saf = {(int)((uint32_t)sa_src[(cur * BKB) * BM + ar_] |
                                           ((uint32_t)sa_src[(cur * BKB + 1) * BM + ar_] << 16)), 0, 0, 0};
                    acc[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, saf),
                                                                     __builtin_bit_cast(v8h, mwf), acc[mt], 0, 0, 0);
                }
            }
        } else {
#pragma unroll
            for (int kk = 0; kk < BKH / 16; ++kk) {
                const v8h bfr = frag(sBf[cur], wrow, 2 * kk + g);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    acc[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(frag(sA[cur], mt * 32 + lr, 2 * kk + g), bfr,
                                                                     acc[mt], 0, 0, 0);
            }
        }
    }
    if (DOTS) return;

    char* Dz = reinterpret_cast<char*>(p.D) + (int64_t)i12 * p.d_nb2 + (int64_t)i13 * p.d_nb3;
    const int n = n0 + wrow;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int m = m0 + mt * 32 + 8 * (i >> 2) + 4 * g + (i & 3);
            if (m < M && n < N) *reinterpret_cast<float*>(Dz + (int64_t)m * p.d_nb1 + (int64_t)n * 4) = acc[mt][i];
        }
}

// Copies rows of row_bytes (2-byte aligned source rows) to a 4-byte pitch so
// the weight DMA can use dword loads.
__global__ __launch_bounds__(256) void align_rows_kernel(const uint8_t* __restrict__ src, int64_t nb1, int64_t nb2,
                                                         int64_t nb3, int64_t ne1, int64_t ne2, int64_t rows,
                                                         int row_halves, int pitch_halves, uint16_t* __restrict__ dst) {
    const int64_t r = blockIdx.x;
    if (r >= rows) return;
    const int64_t i1 = r % ne1, i2 = (r / ne1) % ne2, i3 = r / (ne1 * ne2);
    const uint16_t* s = reinterpret_cast<const uint16_t*>(src + i1 * nb1 + i2 * nb2 + i3 * nb3);
    for (int i = threadIdx.x; i < pitch_halves; i += blockDim.x) dst[r * pitch_halves + i] = i < row_halves ? s[i] : 0;
}

template <int WT>
static void launch_t(const MmqArgs& a, int Z, bool dots, hipStream_t st) {
    const int T = a.tiles_m * a.tiles_n;
    const dim3 grid((unsigned)(((T + 7) / 8) * 8), (unsigned)Z);
    if (dots) mmq_kernel<WT, true><<<grid, NT, 0, st>>>(a);
    else mmq_kernel<WT, false><<<grid, NT, 0, st>>>(a);
}

int64_t mmq_scale_rows(int64_t M) { return (M + BM - 1) / BM * BM; }

// The weight DMA reads whole dwords and the buffer range check zeroes a dword
// that straddles the end, so rows must start 4-byte aligned and span a whole
// number of dwords; other weights are first copied to a zero-padded 4-byte
// pitch.
size_t mmq_align_bytes(const MatW& w, int64_t N, int64_t K) {
    if (w.type == T_F16) return 0;
    const int64_t rowb = (K / QK) * (w.type == T_Q8_0 ? 34 : w.type == T_Q4_0 ? 18 : 20);
    const bool a4 = ((reinterpret_cast<uintptr_t>(w.data) | (uintptr_t)w.nb1 | (uintptr_t)w.nb2 | (uintptr_t)w.nb3 |
                      (uintptr_t)rowb) & 3) == 0;
    return a4 ? 0 : (size_t)(N * w.ne2 * w.ne3) * (size_t)((rowb + 3) & ~3);
}

hipError_t launch_mmq(const MatW& w_in, const ActF16& a, const MatD& d, int64_t N, int64_t ne12, int64_t ne13,
                      int32_t* dots, void* align_buf, hipStream_t st) {
    MatW w = w_in;
    int64_t rowb = w.type == T_F16 ? a.K * 2 : (a.K / QK) * (w.type == T_Q8_0 ? 34 : w.type == T_Q4_0 ? 18 : 20);
    if (mmq_align_bytes(w_in, N, a.K) != 0) {
        // weight rows are only 2-byte aligned: copy them to a 4-byte pitch first
        const int64_t pitch = (rowb + 3) & ~3, rows = N * w.ne2 * w.ne3;
        if (!align_buf) return hipErrorInvalidValue;
        align_rows_kernel<<<dim3((unsigned)rows), 64, 0, st>>>(w.data, w.nb1, w.nb2, w.nb3, N, w.ne2, rows,
                                                              (int)(rowb / 2), (int)(pitch / 2),
                                                              static_cast<uint16_t*>(align_buf));
        w.data = static_cast<const uint8_t*>(align_buf);
        w.nb1 = pitch;
        w.nb2 = pitch * N;
        w.nb3 = pitch * N * w.ne2;
        rowb = pitch;  // the zero padding belongs to the copy
    }
    MmqArgs p;
    p.W = w.data;
    p.w_nb1 = w.nb1;
    p.w_nb2 = w.nb2;
    p.w_nb3 = w.nb3;
    p.w_extent = (N - 1) * w.nb1 + rowb;
    p.A = static_cast<const _Float16*>(a.q);
    p.a_s1 = a.s1;
    p.a_s2 = a.s2;
    p.a_s3 = a.s3;
    p.a_extent = ((a.M - 1) * a.s1 + a.K) * 2;
    p.Ad = static_cast<const _Float16*>(a.d);
    p.As = static_cast<const _Float16*>(a.s);
    p.D = d.data;
    p.d_nb1 = d.nb1;
    p.d_nb2 = d.nb2;
    p.d_nb3 = d.nb3;
    p.dots = dots;
    p.M = (int)a.M;
    p.Mp = (int)mmq_scale_rows(a.M);
    p.N = (int)N;
    p.K = (int)a.K;
    p.ne12 = (int)ne12;
    p.r2 = (int)(ne12 / w.ne2);
    p.r3 = (int)(ne13 / w.ne3);
    p.tiles_m = (int)((a.M + BM - 1) / BM);
    p.tiles_n = (int)((N + BN - 1) / BN);
    // buffer offsets are 32-bit
    if (p.w_extent >= OOB || p.a_extent >= OOB) return hipErrorInvalidValue;
    const int Z = (int)(ne12 * ne13);
    switch (w.type) {
        case T_Q8_0: launch_t<T_Q8_0>(p, Z, dots, st); break;
        case T_Q4_0: launch_t<T_Q4_0>(p, Z, dots, st); break;
        case T_Q4_1: launch_t<T_Q4_1>(p, Z, dots, st); break;
        case T_F16: launch_t<T_F16>(p, Z, false, st); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mi355
