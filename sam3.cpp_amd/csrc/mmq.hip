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
// advances two blocks (64 elements) per stage with one barrier per stage;
// three stage buffers in LDS are filled by LDS DMA (buffer_load ... lds),
// two stages ahead of the one being computed.  Every per-thread offset is
// computed once, a stage advances only the (scalar) base of the buffer
// resource, and rows past M/N read as zeros through the resource's range
// check.  Weight stage segments (2 blocks = 68/36/40 bytes per row) arrive
// as consecutive dwords across lanes (~4 rows per DMA instruction) and stay
// raw in LDS; each wavefront decodes its own MFMA weight fragments from them
// (byte -> 0x64XX half -> packed f16 subtract).  A stage's quantized work is
// eight units (block x m-tile) whose combine FMAs trail their MFMAs by one
// unit.  Workgroups are numbered so each XCD (round-robin dispatch) walks a
// contiguous band of the tile order, which groups a few m-tiles and walks
// n-tiles inside a group (L2 reuse of the resident workgroups' operands).
#include <atomic>
#include <algorithm>
#include <type_traits>

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

// 16-byte slot of chunk c of tile row r is c ^ swz(r): ds_read_b128 serves 16
// lanes per pass from 64 banks, and the 16 consecutive rows an MFMA fragment
// read touches per pass land in 16 distinct slots (8 within every 8 rows).
template <int CH>
__device__ __forceinline__ int swz(int r) {
    return CH == 8 ? ((r & 7) ^ ((r >> 3) & 1)) : (((r >> 1) & 3) ^ ((r >> 3) & 1));
}

struct MmqArgs {
    const uint8_t* W;
    int64_t w_nb1, w_nb2, w_nb3;
    int64_t w_extent;          // bytes of one src0 slice ((N-1)*nb1 + row size)
    const _Float16* A;         // activations (fp16 values), row stride a_s1 halves
    int64_t a_s1, a_s2, a_s3;
    int64_t a_extent;          // bytes of one activation slice ((M-1)*s1 + K halves)
    const _Float16* Ad;        // [Z][M][dp] activation scales (quantized path)
    const _Float16* As;        // [Z][M][dp] Q8_1 sums (Q4_1 path)
    float* D;
    int64_t d_nb1, d_nb2, d_nb3;
    int32_t* dots;             // block-dot inspection output (or null)
    int M, dp, N, K, ne12, r2, r3, tiles_m, tiles_n;  // dp: row pitch (halves) of the scale arrays
    int gm;                    // m-tiles per group of the tile order
    int ksplit, sps;           // K split into ksplit ranges of sps stages; partial sums go to
    int64_t d_split;           // D + split * d_split (bytes), summed by mmq_reduce_kernel
    int d_v4;                  // D rows 16-byte aligned, N % 4 == 0: float4 stores through LDS
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


// Workgroup barrier without a memory fence.  __syncthreads() releases all
// prior memory operations, which waits for every outstanding load, including
// the DMA of later stages still in flight; here each wavefront has already
// waited for the DMA of the stage being published, so only its own LDS reads
// need to be done.  The "memory" clobber keeps the compiler from moving LDS
// accesses across it.
__device__ __forceinline__ void stage_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// One pipeline stage of operands in LDS (two K blocks = 64 halves).  The
// kernel keeps three of these as distinct __shared__ objects so that the
// compiler's LDS-DMA tracking can tell a read of the current stage from the
// DMA still landing in the stage after next.
template <int WT>
struct Stage {
    static constexpr bool QUANT = WT != T_F16;
    static constexpr int SKH = QUANT ? BKH : 32;         // halves of K per stage (F16: 32, keeps 3 stages in LDS)
    static constexpr int CH = SKH / 8;                   // 16-byte chunks per tile row
    static constexpr int WB = WInfo<WT == T_F16 ? T_Q8_0 : WT>::bytes;
    static constexpr int RD = (2 * WB) / 4;              // dwords of a row's 2-block stage segment
    static constexpr int RLD = (BN * RD + NT - 1) / NT;  // raw dword DMA instructions per wavefront
    _Float16 A[BM * SKH];                                // activation tile, swizzled 16-byte chunks
    _Float16 Bf[QUANT ? 8 : BN * SKH];                   // F16 weight tile (same swizzle)
    uint32_t W[QUANT ? RLD * NT : 4];                    // raw weight segments, lane-linear dwords
    _Float16 Ad[BM][BKB];                                // activation scales of the two blocks, per row
    _Float16 As[WT == T_Q4_1 ? BM : 1][BKB];             // Q8_1 sums (Q4_1), per row
};

// Workgroup 128(m) x 128(n); wavefront w owns all 128 rows of m and the 32
// columns n0 + 32w .. +31 (4 MFMA tiles stacked along m).  Every stage's
// operands are DMA'd from global memory straight into LDS (buffer_load ...
// lds): no staging registers, no LDS store instructions.  Three stages are
// in flight: at stage s each wavefront waits for its own DMA of stage s
// (leaving stage s+1's outstanding), one barrier publishes everyone's, and
// the DMA of stage s+2 goes into the buffer stage s-1 used.
//   activation tile: 128 rows x 64 halves, unpadded; 16-byte chunk c of row r
//     sits in slot c ^ swz(r), so the MFMA fragment reads are free of bank
//     conflicts while each DMA lane still writes 16 contiguous bytes;
//   raw weight segments: lane-linear dwords (row j / RD, dword j % RD);
//     each wavefront decodes its own 32 weight rows' fragments on the fly;
//   activation scales (and Q8_1 sums): 128 fp16 per block, one dword per lane.
template <int WT, bool DOTS, int EPI>
__global__ __launch_bounds__(NT, 2) void mmq_kernel(const MmqArgs p, const MmqEpi e) {
    using St = Stage<WT>;
    constexpr bool QUANT = St::QUANT;
    constexpr int WB = St::WB, HDR = WInfo<WT == T_F16 ? T_Q8_0 : WT>::hdr;
    constexpr int RD = St::RD, RLD = St::RLD, SKH = St::SKH, CH = St::CH;
    constexpr int MT = BM / 32;       // m tiles per wavefront
    constexpr int RPI = 64 / CH;      // tile rows per DMA instruction
    constexpr int NI = BM / 4 / RPI;  // tile DMA instructions per wavefront
    // per-wavefront DMA instructions of one stage (plus one scale load on some wavefronts)
    constexpr int NL = QUANT ? NI + RLD : 2 * NI;
    __shared__ __attribute__((aligned(16))) St st0;
    __shared__ __attribute__((aligned(16))) St st1;
    __shared__ __attribute__((aligned(16))) St st2;

    // XCD-aware tile order: workgroup id -> (xcd, slot) -> contiguous tile band per XCD
    // (a K split's ranges of one tile are adjacent, so they share an XCD)
    const int TT = p.tiles_m * p.tiles_n * p.ksplit;
    const int per_xcd = (TT + 7) / 8;
    const int tl = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (tl >= TT) return;
    const int t = tl / p.ksplit, split = tl - t * p.ksplit;
    // grouped order: gm m-tiles per group, n-major inside a group, so the
    // workgroups resident on one XCD at a time share a few weight column
    // tiles and activation row tiles in its L2
    const int gsz = p.gm * p.tiles_n, grp = t / gsz, gr = t - grp * gsz;
    const int gmr = min(p.gm, p.tiles_m - grp * p.gm);
    const int m0 = (grp * p.gm + gr % gmr) * BM, n0 = (gr / gmr) * BN;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wn = __builtin_amdgcn_readfirstlane(tid >> 6);  // wavefront index (uniform)
    const int z = blockIdx.y, i12 = z % p.ne12, i13 = z / p.ne12;
    // a K split computes a plain GEMM over its range k0s .. k0s + K: shifted
    // operand bases, the same kernel code
    const int k0s = split * p.sps * SKH;
    const int M = p.M, N = p.N, K = min(p.K - k0s, p.sps * SKH);
    const int nb = K / QK;
    const int nstage = QUANT ? (nb + BKB - 1) / BKB : (K + SKH - 1) / SKH;
    const int64_t wsh = QUANT ? (int64_t)(k0s / QK) * WB : 2LL * k0s;  // weight bytes skipped per row
    const uint8_t* Wz = p.W + (int64_t)(i12 / p.r2) * p.w_nb2 + (int64_t)(i13 / p.r3) * p.w_nb3 + wsh;
    const int64_t w_extent = p.w_extent - wsh, a_extent = p.a_extent - 2LL * k0s;
    const _Float16* Az = p.A + (int64_t)i12 * p.a_s2 + (int64_t)i13 * p.a_s3 + k0s;
    const int dp = p.dp;
    const int64_t sc_extent = 2LL * M * dp - 2LL * (k0s / QK);
    const _Float16* Adz = QUANT ? p.Ad + (int64_t)z * M * dp + k0s / QK : nullptr;
    const _Float16* Asz = WT == T_Q4_1 ? p.As + (int64_t)z * M * dp + k0s / QK : nullptr;
    // wavefronts 0, 1 load the two blocks' d; for Q4_1, 2 and 3 load the two blocks' s
    const bool xload = QUANT && (wn < 2 || WT == T_Q4_1);

    // ---- DMA offsets, fixed for the whole K loop
    // activation / F16-weight tile, instruction i of wavefront w: rows (NI*w+i)*RPI + lane/CH,
    // slot lane%CH <- chunk (lane%CH) ^ (row%CH)
    const int trow = lane / CH;
    int aoff[NI], foff[NI], tch[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int row = (wn * NI + i) * RPI + trow;
        tch[i] = (lane % CH) ^ swz<CH>(row);
        aoff[i] = m0 + row < M ? ((m0 + row) * (int)p.a_s1 + tch[i] * 8) * 2 : OOB;
        foff[i] = !QUANT && n0 + row < N ? (n0 + row) * (int)p.w_nb1 + tch[i] * 16 : OOB;
    }
    int woff[QUANT ? RLD : 1];  // raw weight dword j = NT*i + 64w + lane -> (row j / RD, dword j % RD)
#pragma unroll
    for (int i = 0; i < (QUANT ? RLD : 1); ++i) {
        const int j = tid + NT * i, row = j / RD, c = j - row * RD;
        woff[i] = QUANT && j < BN * RD && n0 + row < N ? (n0 + row) * (int)p.w_nb1 + 4 * c : OOB;
    }

    auto dma_stage = [&](int s, St& b) {
        const int k0 = s * SKH;
        const bool tail = k0 + SKH > K;  // chunks past K must read zeros (rows continue in memory)
        const auto ar = make_rsrc(Az + k0, a_extent - 2LL * k0);
#pragma unroll
        for (int i = 0; i < NI; ++i)
            dma_b128(ar, &b.A[(wn * NI + i) * RPI * SKH], tail && k0 + tch[i] * 8 >= K ? OOB : aoff[i]);
        if (QUANT) {
            const int64_t seg = (int64_t)s * BKB * WB;
            const auto wrs = make_rsrc(Wz + seg, w_extent - seg);
#pragma unroll
            for (int i = 0; i < RLD; ++i)
                dma_b32(wrs, &b.W[NT * i + 64 * wn], woff[i]);
            // row m0 + 64*(w & 1) + lane: one dword = the row's scales of blocks 2s, 2s+1
            const int sr_ = 64 * (wn & 1) + lane;
            const int soff = m0 + sr_ < M ? ((m0 + sr_) * dp + s * BKB) * 2 : OOB;
            if (wn < 2) {
                dma_b32(make_rsrc(Adz, sc_extent), &b.Ad[64 * (wn & 1)][0], soff);
            } else if (WT == T_Q4_1) {
                dma_b32(make_rsrc(Asz, sc_extent), &b.As[WT == T_Q4_1 ? 64 * (wn & 1) : 0][0], soff);
            }
        } else {
            const auto fr = make_rsrc(Wz + 2LL * k0, w_extent - 2LL * k0);
#pragma unroll
            for (int i = 0; i < NI; ++i)
                dma_b128(fr, &b.Bf[(wn * NI + i) * RPI * SKH], tail && k0 + tch[i] * 8 >= K ? OOB : foff[i]);
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
    const bool lo = lane < 32;
    // fragment of row r, 8-half chunk c in a swizzled tile
    auto frag = [&](const _Float16* tile, int r, int c) -> v8h {
        return *reinterpret_cast<const v8h*>(&tile[r * SKH + ((c ^ swz<CH>(r)) << 3)]);
    };

    auto compute = [&](int s, const St& b) {
        if (QUANT) {
            const uint32_t* rowp = &b.W[wrow * RD];
            const uint16_t* hrow = reinterpret_cast<const uint16_t*>(rowp);
            if (WT == T_Q4_1 && !DOTS) {
                // acc += sum_b s_a[m][b] * m_w[n][b] over this stage's blocks (k-slots 0, 1)
                const uint32_t m1 = s * BKB + 1 < nb ? (uint32_t)hrow[WB / 2 + 1] << 16 : 0u;
                const v4i mwf = {lo ? (int)((uint32_t)hrow[1] | m1) : 0, 0, 0, 0};
                const uint32_t* asw = reinterpret_cast<const uint32_t*>(&b.As[0][0]);  // row: s of blocks 2s, 2s+1
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const int ar_ = mt * 32 + lr;
                    v4i saf = __builtin_bit_cast(v4i, frag(b.A, ar_, g));  // finite filler
                    saf[0] = (int)asw[WT == T_Q4_1 ? ar_ : 0];
                    acc[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, saf),
                                                                     __builtin_bit_cast(v8h, mwf), acc[mt], 0, 0, 0);
                }
            }
#pragma unroll
            for (int bk = 0; bk < BKB; ++bk) {
                if (DOTS && s * BKB + bk >= nb) break;
                // this lane's weight fragments: row wrow, k-chunk 8g..8g+7 of each 16-wide half
                v8h bf[2];
                if (WT == T_Q8_0) {
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        uint32_t w0, w1;
                        lds_dw2(rowp, bk * WB + HDR + 16 * h + 8 * g, (bk * WB + HDR) & 3, w0, w1);
                        bf[h] = i8x8_to_h8(w0, w1);
                    }
                } else {
                    uint32_t w0, w1;  // payload bytes 8g..8g+7: low nibbles = half 0, high = half 1
                    lds_dw2(rowp, bk * WB + HDR + 8 * g, (bk * WB + HDR) & 3, w0, w1);
                    const _Float16 bias = WT == T_Q4_0 ? (_Float16)1032.0f : (_Float16)1024.0f;
                    bf[0] = n8_to_h8(w0 & 0x0f0f0f0fu, w1 & 0x0f0f0f0fu, bias);
                    bf[1] = n8_to_h8((w0 >> 4) & 0x0f0f0f0fu, (w1 >> 4) & 0x0f0f0f0fu, bias);
                }
                // S-MFMA B operand: d_w in k-slot 0 (lanes 0..31), zero in every other k-slot.
                // A block past K (odd block count) gets d_w = 0: its raw bytes belong to the
                // next row (or padding) and its d_a is 0, so S = 0 leaves acc unchanged.
                const bool bvalid = s * BKB + bk < nb;
                const v4i dwf = {lo && bvalid ? (int)(uint32_t)hrow[bk * WB / 2] : 0, 0, 0, 0};
#pragma unroll
                for (int mp = 0; mp < MT; mp += 2) {
                    v16f I[2], S[2];
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const int ar_ = (mp + j) * 32 + lr;
                        const v8h a0 = frag(b.A, ar_, 4 * bk + g);
                        const v8h a1 = frag(b.A, ar_, 4 * bk + 2 + g);
                        I[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, bf[0], zf, 0, 0, 0);
                        I[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, bf[1], I[j], 0, 0, 0);
                        if (!DOTS) {
                            // S-MFMA A operand: d_a in k-slot 0; the other k-slots keep a1's
                            // (finite) quants, which meet B's zeros
                            v4i daf = __builtin_bit_cast(v4i, a1);
                            daf[0] = (int)(uint32_t) reinterpret_cast<const uint16_t*>(&b.Ad[0][0])[ar_ * BKB + bk];
                            S[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, daf),
                                                                          __builtin_bit_cast(v8h, dwf), zf, 0, 0, 0);
                        }
                    }
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        if (DOTS) {
                            const int n = n0 + wrow;
#pragma unroll
                            for (int i = 0; i < 16; ++i) {
                                const int m = m0 + (mp + j) * 32 + 8 * (i >> 2) + 4 * g + (i & 3);
                                if (m < M && n < N)
                                    p.dots[(((int64_t)z * M + m) * N + n) * nb + s * BKB + bk] = (int32_t)I[j][i];
                            }
                        } else {
#pragma unroll
                            for (int i = 0; i < 16; ++i) acc[mp + j][i] = __builtin_fmaf(I[j][i], S[j][i], acc[mp + j][i]);
                        }
                    }
                }
            }
        } else {
#pragma unroll
            for (int kk = 0; kk < SKH / 16; ++kk) {
                const v8h bfr = frag(b.Bf, wrow, 2 * kk + g);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    acc[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(frag(b.A, mt * 32 + lr, 2 * kk + g), bfr,
                                                                     acc[mt], 0, 0, 0);
            }
        }
    };

    // Quantized weights (no block-dot output): each stage is 8 units (block bk,
    // m-tile mt; mt fastest).  Unit u issues its three MFMAs (the isum in two,
    // the scale outer product in one) into product buffer u % 2, then the fp32
    // FMAs of unit u - 1 from the other buffer; the stage ends with unit 7's
    // FMAs.  A wavefront's FMAs thus never wait for the MFMAs it has just
    // issued and run while they execute (FMAs right behind their own MFMAs
    // leave the matrix core idle while both wavefronts of a SIMD apply theirs).
    // Every acc tile still receives its terms in block order (for Q4_1: the
    // stage's offset term, then block 0, block 1).  Products do not live
    // across stages: 16-register tuples carried around the K loop spill.
    static_assert(MT == 4, "unit pipeline assumes four m-tiles per wavefront");
    auto apply = [&](int mt, const v16f& I, const v16f& S) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[mt][i] = __builtin_fmaf(I[i], S[i], acc[mt][i]);
    };
    // Fragments of unit (bk, mt): the two 8-half activation chunks of row
    // mt*32 + lr and the row's activation scale.  Unit u reads unit u + 1's
    // while its MFMAs run, so only a stage's first unit waits on LDS.
    struct Frag {
        v8h a0, a1;
        uint32_t da;
    };
    auto load_frag = [&](const St& b, auto bkc, auto mtc) __attribute__((always_inline)) -> Frag {
        constexpr int bk = decltype(bkc)::value, mt = decltype(mtc)::value;
        const int ar_ = mt * 32 + lr;
        Frag f;
        f.a0 = frag(b.A, ar_, 4 * bk + g);
        f.a1 = frag(b.A, ar_, 4 * bk + 2 + g);
        f.da = reinterpret_cast<const uint16_t*>(&b.Ad[0][0])[ar_ * BKB + bk];
        return f;
    };
    // weight fragments of block bk (row wrow, k-chunk 8g..8g+7 of each 16-wide
    // half) and the S-MFMA B operand: d_w in k-slot 0 (lanes 0..31), zero in
    // every other k-slot.  A block past K (odd block count) gets d_w = 0: its raw
    // bytes belong to the next row (or padding) and its d_a is 0, so S = 0.
    struct WFrag {
        v8h bf[2];
        v4i dwf;
    };
    auto load_wfrag = [&](int s, const St& b, auto bkc) __attribute__((always_inline)) -> WFrag {
        constexpr int bk = decltype(bkc)::value;
        const uint32_t* rowp = &b.W[wrow * RD];
        const uint16_t* hrow = reinterpret_cast<const uint16_t*>(rowp);
        WFrag w;
        if (WT == T_Q8_0) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                uint32_t w0, w1;
                lds_dw2(rowp, bk * WB + HDR + 16 * h + 8 * g, (bk * WB + HDR) & 3, w0, w1);
                w.bf[h] = i8x8_to_h8(w0, w1);
            }
        } else {
            uint32_t w0, w1;  // payload bytes 8g..8g+7: low nibbles = half 0, high = half 1
            lds_dw2(rowp, bk * WB + HDR + 8 * g, (bk * WB + HDR) & 3, w0, w1);
            const _Float16 bias = WT == T_Q4_0 ? (_Float16)1032.0f : (_Float16)1024.0f;
            w.bf[0] = n8_to_h8(w0 & 0x0f0f0f0fu, w1 & 0x0f0f0f0fu, bias);
            w.bf[1] = n8_to_h8((w0 >> 4) & 0x0f0f0f0fu, (w1 >> 4) & 0x0f0f0f0fu, bias);
        }
        const uint32_t dw = hrow[bk * WB / 2];
        w.dwf = v4i{lo && s * BKB + bk < nb ? (int)dw : 0, 0, 0, 0};
        return w;
    };
    // unit (bk, mt): MFMAs of its fragments f into product buffer mt % 2, then the
    // FMAs of the previous unit (m-tile mt - 1) from the other buffer, pinned
    // here (an empty asm reads the updated accumulator) so that they are not
    // sunk past the next units' MFMAs
    auto unit = [&](const St& b, auto bkc, auto mtc, const Frag& f, const WFrag& w, const v4i& mwf, v16f(&PI)[2],
                    v16f(&PS)[2]) __attribute__((always_inline)) {
        constexpr int bk = decltype(bkc)::value, mt = decltype(mtc)::value;
        constexpr int u2 = mt & 1, p2 = u2 ^ 1;
        if (WT == T_Q4_1 && bk == 0) {
            // acc += sum_b s_a[m][b] * m_w[n][b] over this stage's blocks (k-slots 0, 1)
            v4i saf = __builtin_bit_cast(v4i, f.a0);  // finite filler
            saf[0] = (int)reinterpret_cast<const uint32_t*>(&b.As[0][0])[WT == T_Q4_1 ? mt * 32 + lr : 0];
            acc[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, saf), __builtin_bit_cast(v8h, mwf),
                                                             acc[mt], 0, 0, 0);
        }
        // S-MFMA A operand: d_a in k-slot 0; the other k-slots keep a1's (finite)
        // quants, which meet B's zeros
        v4i daf = __builtin_bit_cast(v4i, f.a1);
        daf[0] = (int)f.da;
        PI[u2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a0, w.bf[0], zf, 0, 0, 0);
        PI[u2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a1, w.bf[1], PI[u2], 0, 0, 0);
        PS[u2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, daf), __builtin_bit_cast(v8h, w.dwf), zf,
                                                        0, 0, 0);
        if (bk > 0 || mt > 0) {
            constexpr int pm = (mt + 3) & 3;
            apply(pm, PI[p2], PS[p2]);
            asm volatile("" : "+v"(acc[pm]));
        }
    };
    auto compute_q = [&](int s, const St& b) __attribute__((always_inline)) {
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        using I2 = std::integral_constant<int, 2>;
        using I3 = std::integral_constant<int, 3>;
        static_assert(BKB == 2, "two blocks per stage");
        v16f PI[2], PS[2];
        v4i mwf = {0, 0, 0, 0};
        if (WT == T_Q4_1) {
            const uint16_t* hrow = reinterpret_cast<const uint16_t*>(&b.W[wrow * RD]);
            const uint32_t m1 = s * BKB + 1 < nb ? (uint32_t)hrow[WB / 2 + 1] << 16 : 0u;
            mwf[0] = lo ? (int)((uint32_t)hrow[1] | m1) : 0;
        }
        const WFrag w0 = load_wfrag(s, b, I0{});
        Frag f = load_frag(b, I0{}, I0{});
        Frag n = load_frag(b, I0{}, I1{});
        unit(b, I0{}, I0{}, f, w0, mwf, PI, PS);
        __builtin_amdgcn_sched_barrier(0);
        f = load_frag(b, I0{}, I2{});
        unit(b, I0{}, I1{}, n, w0, mwf, PI, PS);
        __builtin_amdgcn_sched_barrier(0);
        n = load_frag(b, I0{}, I3{});
        unit(b, I0{}, I2{}, f, w0, mwf, PI, PS);
        __builtin_amdgcn_sched_barrier(0);
        const WFrag w1 = load_wfrag(s, b, I1{});
        f = load_frag(b, I1{}, I0{});
        unit(b, I0{}, I3{}, n, w0, mwf, PI, PS);
        __builtin_amdgcn_sched_barrier(0);
        n = load_frag(b, I1{}, I1{});
        unit(b, I1{}, I0{}, f, w1, mwf, PI, PS);
        __builtin_amdgcn_sched_barrier(0);
        f = load_frag(b, I1{}, I2{});
        unit(b, I1{}, I1{}, n, w1, mwf, PI, PS);
        __builtin_amdgcn_sched_barrier(0);
        n = load_frag(b, I1{}, I3{});
        unit(b, I1{}, I2{}, f, w1, mwf, PI, PS);
        __builtin_amdgcn_sched_barrier(0);
        unit(b, I1{}, I3{}, n, w1, mwf, PI, PS);
        apply(3, PI[1], PS[1]);  // unit 7
    };

    // one pipeline step: wait for stage s, publish it, refill the oldest buffer, compute
    auto step = [&](int s, const St& cur, St& refill) __attribute__((always_inline)) {
        if (s + 1 < nstage) {
            if (xload) wait_vmcnt<NL + 1>();
            else wait_vmcnt<NL>();
        } else {
            wait_vmcnt<0>();
        }
        stage_barrier();
        if (s + 2 < nstage) dma_stage(s + 2, refill);
        if (QUANT && !DOTS) {
            compute_q(s, cur);
        } else {
            compute(s, cur);
        }
    };

    // F16 weights, residual epilogue: the thread's sixteen residual float4 (the epilogue's rows
    // and columns below) are loaded before the first stage's DMA, so their latency passes
    // under the K loop instead of being paid per group of rows after it (80 VGPRs, which the
    // quantized types' fragments leave no room for).  Issued ahead of the stage DMAs they
    // complete before stage 0 by the in-order vmcnt, so the K loop's waits are unchanged;
    // each element is read and later written by this thread only (in place is safe).
    constexpr bool PRE = EPI == MMQ_EPI_RESIDUAL && WT == T_F16;
    int rr_pre[PRE ? 16 : 1];
    v4f xs_pre[PRE ? 16 : 1];
    if (PRE) {
        const int nc = n0 + 4 * (tid % (BN / 4));
#pragma unroll
        for (int q = 0; q < (PRE ? 16 : 1); ++q) {
            const int m = m0 + (q >> 3) * 64 + (q & 7) * (NT / (BN / 4)) + tid / (BN / 4);
            rr_pre[q] = m < M && nc < N ? map_row32(e.map, m) : -1;
            xs_pre[q] = rr_pre[q] >= 0 ? *reinterpret_cast<const v4f*>(&e.res[(int64_t)rr_pre[q] * N + nc])
                                       : v4f{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    dma_stage(0, st0);
    if (nstage > 1) dma_stage(1, st1);
    for (int s = 0; s < nstage; s += 3) {
        step(s, st0, st2);
        if (s + 1 < nstage) step(s + 1, st1, st0);
        if (s + 2 < nstage) step(s + 2, st2, st1);
    }
    if (DOTS) return;

    const int n = n0 + wrow;
    if (EPI == MMQ_EPI_STORE) {
        char* Dz = reinterpret_cast<char*>(p.D) + (int64_t)i12 * p.d_nb2 + (int64_t)i13 * p.d_nb3 + split * p.d_split;
        if (p.d_v4) {  // row-major through LDS: float4 stores, whole 512-byte row segments
            // 128-float rows (two lines of the 64 4-byte banks), columns of rows with bit 2 set
            // rotated by 32: a write (lanes 0..31 row R, lanes 32..63 row R + 4) hits 64 banks
            constexpr int TP = BN, CPR = BN / 4, IT = 64 * CPR / NT;
            float* t0 = reinterpret_cast<float*>(&st0);
            float* t1 = reinterpret_cast<float*>(&st1);
            const int c = tid % CPR, nc = n0 + 4 * c;
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                __syncthreads();
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int r = 8 * (i >> 2) + 4 * g + (i & 3);
                    t0[r * TP + ((wrow + 32 * g) & (BN - 1))] = acc[2 * half][i];
                    t1[r * TP + ((wrow + 32 * g) & (BN - 1))] = acc[2 * half + 1][i];
                }
                __syncthreads();
#pragma unroll
                for (int it = 0; it < IT; ++it) {
                    const int r = it * (NT / CPR) + tid / CPR, m = m0 + half * 64 + r;
                    if (m >= M || nc >= N) continue;
                    const v4f v = *reinterpret_cast<const v4f*>(&(it < IT / 2 ? t0 : t1)[(r & 31) * TP + ((4 * c + 32 * ((r >> 2) & 1)) & (BN - 1))]);
                    *reinterpret_cast<v4f*>(Dz + (int64_t)m * p.d_nb1 + (int64_t)nc * 4) = v;
                }
            }
            return;
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int m = m0 + mt * 32 + 8 * (i >> 2) + 4 * g + (i & 3);
                if (m < M && n < N) *reinterpret_cast<float*>(Dz + (int64_t)m * p.d_nb1 + (int64_t)n * 4) = acc[mt][i];
            }
        return;
    }
    // The fused epilogues go through LDS: the 128 x 128 result tile, 64 rows
    // at a time (32 in st0, 32 in st1), is rewritten row-major so that each
    // thread then owns 4 consecutive columns (float4 loads and stores).
    // u = dst + bias, each add rounded to fp32 as ggml's ADD nodes.
    constexpr int TP = BN;                    // row pitch (floats), rows with bit 2 set rotated by 32
    constexpr int CPR = BN / 4;               // float4 chunks per row
    constexpr int IT = 64 * CPR / NT;         // rows per thread per half
    static_assert(32 * TP * 4 <= (int)sizeof(St), "epilogue tile exceeds a stage buffer");
    float* t0 = reinterpret_cast<float*>(&st0);
    float* t1 = reinterpret_cast<float*>(&st1);
    const int c = tid % CPR, nc = n0 + 4 * c;  // this thread's 4 columns, the same in every row
    const bool cv = nc < N;                    // N % 4 == 0
    const v4f bv = cv ? *reinterpret_cast<const v4f*>(&e.bias[nc]) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        __syncthreads();  // every wavefront is done reading the stage buffers / the previous half
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = 8 * (i >> 2) + 4 * g + (i & 3);
            t0[r * TP + ((wrow + 32 * g) & (BN - 1))] = acc[2 * half][i];
            t1[r * TP + ((wrow + 32 * g) & (BN - 1))] = acc[2 * half + 1][i];
        }
        __syncthreads();
        if (EPI == MMQ_EPI_QKV) {
            const int E = e.nh * e.hd, which = nc / E, col = nc - which * E, hh = col / e.hd, d = col - hh * e.hd;
            _Float16* dst = which == 0 ? e.q : which == 1 ? e.k : e.v;
#pragma unroll
            for (int it = 0; it < IT; ++it) {
                const int r = it * (NT / CPR) + tid / CPR, m = m0 + half * 64 + r;
                if (m >= M || !cv) continue;
                const v4f uv = *reinterpret_cast<const v4f*>(&(it < IT / 2 ? t0 : t1)[(r & 31) * TP + ((4 * c + 32 * ((r >> 2) & 1)) & (BN - 1))]) + bv;
                float u0 = uv[0], u1 = uv[1], u2 = uv[2], u3 = uv[3];
                const int bw = m / e.ntok, n = m - bw * e.ntok;
                if (which < 2 && e.rope) {
                    const v4f cs = *reinterpret_cast<const v4f*>(&e.rope[(int64_t)n * e.hd + d]);
                    rope_pair(u0, u1, cs[0], cs[1]);
                    rope_pair(u2, u3, cs[2], cs[3]);
                }
                const uint32_t h0 = (uint32_t)f2h(u0) | ((uint32_t)f2h(u1) << 16);
                const uint32_t h1 = (uint32_t)f2h(u2) | ((uint32_t)f2h(u3) << 16);
                *reinterpret_cast<uint2*>(&dst[(((int64_t)bw * e.nh + hh) * e.ntok + n) * e.hd + d]) = make_uint2(h0, h1);
            }
        } else {
            // residual loads of four rows first, then their stores (res may be out)
#pragma unroll
            for (int i0 = 0; i0 < IT; i0 += 4) {
                int rr[4];
                v4f xs[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if (PRE) {
                        rr[k] = rr_pre[PRE ? half * 8 + i0 + k : 0];
                        xs[k] = xs_pre[PRE ? half * 8 + i0 + k : 0];
                        continue;
                    }
                    const int m = m0 + half * 64 + (i0 + k) * (NT / CPR) + tid / CPR;
                    rr[k] = m < M && cv ? map_row32(e.map, m) : -1;
                    xs[k] = rr[k] >= 0 ? *reinterpret_cast<const v4f*>(&e.res[(int64_t)rr[k] * N + nc])
                                       : v4f{0.0f, 0.0f, 0.0f, 0.0f};
                }
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int it = i0 + k, r = it * (NT / CPR) + tid / CPR;
                    const v4f v = *reinterpret_cast<const v4f*>(&(it < IT / 2 ? t0 : t1)[(r & 31) * TP + ((4 * c + 32 * ((r >> 2) & 1)) & (BN - 1))]);
                    if (rr[k] >= 0) *reinterpret_cast<v4f*>(&e.out[(int64_t)rr[k] * N + nc]) = xs[k] + (v + bv);
                }
            }
        }
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

// mmq_reduce_kernel's rn4
static double reduce_rcp(int64_t M, int64_t N) {
    const int64_t n4 = N / 4;
    return n4 > 0 && M * n4 + n4 < ((int64_t)1 << 31) && M < ((int64_t)1 << 30) ? 1.0 / (double)n4 : 0.0;
}

// Split-K: dst rows (or the fused epilogue) from the ksplit partial sums,
// added in split order; one thread per 4 columns (N % 4 == 0).  rn4 = 4 / N when
// M * N / 4 + N / 4 < 2^31 and M < 2^30: row, column and the epilogue's row splits then come
// from div_rcp instead of 64- and 32-bit integer divisions; else rn4 = 0.
template <int EPI>
__global__ __launch_bounds__(256) void mmq_reduce_kernel(const float* __restrict__ part, int ksplit, int M, int N,
                                                         char* __restrict__ D, int64_t d_nb1, const MmqEpi e,
                                                         double rn4) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int n4 = N / 4;
    if (t >= (int64_t)M * n4) return;
    const bool fast = rn4 != 0.0;
    int m, nc;
    if (fast) {
        m = div_rcp((int)t, n4, rn4, nc);
        nc *= 4;
    } else {
        m = (int)(t / n4);
        nc = (int)(t - (int64_t)m * n4) * 4;
    }
    const int64_t mn = (int64_t)M * N;
    v4f f = *reinterpret_cast<const v4f*>(&part[(int64_t)m * N + nc]);
    for (int s = 1; s < ksplit; ++s) f = f + *reinterpret_cast<const v4f*>(&part[s * mn + (int64_t)m * N + nc]);
    if (EPI == MMQ_EPI_STORE) {
        *reinterpret_cast<v4f*>(D + (int64_t)m * d_nb1 + (int64_t)nc * 4) = f;
        return;
    }
    const v4f u = f + *reinterpret_cast<const v4f*>(&e.bias[nc]);
    if (EPI == MMQ_EPI_RESIDUAL) {
        const int rr = fast ? map_row32(e.map, rowmap_rcp(e.map), m) : map_row32(e.map, m);
        if (rr >= 0) {
            const v4f x = *reinterpret_cast<const v4f*>(&e.res[(int64_t)rr * N + nc]);
            *reinterpret_cast<v4f*>(&e.out[(int64_t)rr * N + nc]) = x + u;
        }
    } else {
        const int E = e.nh * e.hd, which = nc / E, col = nc - which * E, hh = col / e.hd, d = col - hh * e.hd;
        _Float16* dst = which == 0 ? e.q : which == 1 ? e.k : e.v;
        float u0 = u[0], u1 = u[1], u2 = u[2], u3 = u[3];
        int n;
        const int bw = fast ? div_rcp(m, e.ntok, 1.0 / (double)e.ntok, n) : m / e.ntok;
        if (!fast) n = m - bw * e.ntok;
        if (which < 2 && e.rope) {
            const v4f cs = *reinterpret_cast<const v4f*>(&e.rope[(int64_t)n * e.hd + d]);
            rope_pair(u0, u1, cs[0], cs[1]);
            rope_pair(u2, u3, cs[2], cs[3]);
        }
        const uint32_t h0 = (uint32_t)f2h(u0) | ((uint32_t)f2h(u1) << 16);
        const uint32_t h1 = (uint32_t)f2h(u2) | ((uint32_t)f2h(u3) << 16);
        *reinterpret_cast<uint2*>(&dst[(((int64_t)bw * e.nh + hh) * e.ntok + n) * e.hd + d]) = make_uint2(h0, h1);
    }
}

template <int WT>
static void launch_t(const MmqArgs& a, int Z, bool dots, const MmqEpi* e, hipStream_t st) {
    if (a.ksplit > 1) {  // partial sums (STORE into the split buffer), then the reduction with the epilogue
        const int TT = a.tiles_m * a.tiles_n * a.ksplit;
        MmqEpi none{};
        mmq_kernel<WT, false, MMQ_EPI_STORE><<<dim3((unsigned)(((TT + 7) / 8) * 8)), NT, 0, st>>>(a, none);
        return;
    }
    const int T = a.tiles_m * a.tiles_n;
    const dim3 grid((unsigned)(((T + 7) / 8) * 8), (unsigned)Z);
    MmqEpi none{};
    if (dots) mmq_kernel<WT, true, MMQ_EPI_STORE><<<grid, NT, 0, st>>>(a, none);
    else if (!e || e->kind == MMQ_EPI_STORE) mmq_kernel<WT, false, MMQ_EPI_STORE><<<grid, NT, 0, st>>>(a, none);
    else if (e->kind == MMQ_EPI_RESIDUAL) mmq_kernel<WT, false, MMQ_EPI_RESIDUAL><<<grid, NT, 0, st>>>(a, *e);
    else mmq_kernel<WT, false, MMQ_EPI_QKV><<<grid, NT, 0, st>>>(a, *e);
}


// The weight DMA reads whole dwords and the buffer range check zeroes a dword
// that straddles the end, so rows must start 4-byte aligned and span a whole
// number of dwords; other weights are first copied to a zero-padded 4-byte
// pitch. F16 rows are read in 16-byte chunks: rows that are not 16-byte
// aligned or whose K is not a multiple of 8 are copied to a pitch of K
// rounded up to 8 halves, zero-filled.
size_t mmq_align_bytes(const MatW& w, int64_t N, int64_t K) {
    if (w.type == T_F16) {
        const bool a16 = K % 8 == 0 && ((reinterpret_cast<uintptr_t>(w.data) | (uintptr_t)w.nb1 | (uintptr_t)w.nb2 |
                                         (uintptr_t)w.nb3) & 15) == 0;
        return a16 ? 0 : (size_t)(N * w.ne2 * w.ne3) * (size_t)(((K + 7) & ~7) * 2);
    }
    const int64_t rowb = (K / QK) * (w.type == T_Q8_0 ? 34 : w.type == T_Q4_0 ? 18 : 20);
    const bool a4 = ((reinterpret_cast<uintptr_t>(w.data) | (uintptr_t)w.nb1 | (uintptr_t)w.nb2 | (uintptr_t)w.nb3 |
                      (uintptr_t)rowb) & 3) == 0;
    return a4 ? 0 : (size_t)(N * w.ne2 * w.ne3) * (size_t)((rowb + 3) & ~3);
}

// K split for GEMMs with too few output tiles to fill the GPU: the fewest
// (rounds of workgroups x stages per split) plus the partial-sum traffic
// (written by the GEMM, read by the reduction at ~4 TB/s) and a launch.
int mmq_ksplit(int type, int64_t M, int64_t N, int64_t K, int64_t Z, int cus) {
    if (Z != 1 || N % 4 != 0 || cus <= 0) return 1;
    // block-quantized weights split as the int8 kernel splits them: both routes then add the
    // same K ranges in the same order and stay bit-identical
    if (type != T_F16 && K % QK == 0) return mmq8_ksplit(M, N, K, cus);
    const bool quant = type != T_F16;
    const int64_t T = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    const int64_t nstage = quant ? ((K / QK) + BKB - 1) / BKB : (K + 31) / 32;
    const int64_t slots = (int64_t)cus * (quant ? 2 : 3);
    const double t_stage = quant ? 2.0 : 0.85;           // us per stage of one round of workgroups
    const double unit = (double)M * N * 4 / 4.0e6;       // us to move one M x N f32 array
    int best = 1;
    double best_cost = (double)((T + slots - 1) / slots) * nstage * t_stage;
    for (int ks = 2; ks <= 16; ++ks) {
        const int64_t sps = (nstage + ks - 1) / ks;
        if (sps < 2 || (ks - 1) * sps >= nstage) break;
        const double cost = (double)((T * ks + slots - 1) / slots) * sps * t_stage + 2.0 * ks * unit + 3.0;
        if (cost < best_cost) {
            best_cost = cost;
            best = ks;
        }
    }
    return best;
}

// ---- Skinny GEMMs: K <= 128 at large M (the Hiera stage-1 projections, K = 96)
//
// Output writes dominate these (M x N f32 against an M x K fp16 operand),
// while a 128x128 tile of mmq_kernel runs only two K stages, re-reads the
// activations for every n-tile and spends most of its time in prologue and
// epilogue.  Here one workgroup computes all N columns of 64 or 128
// activation rows: it copies the whole quantized weight matrix into LDS
// (raw rows, 16-byte loads, eight in flight per thread) while its activation
// rows are in flight, then each wavefront walks n-tiles and writes each
// 32x32 output tile through LDS as float4 row segments.  A workgroup holds
// one row block and ends after its stores are issued, so the stores of one
// overlap the loads of the next (on gfx9 a wait for loads also waits for
// every earlier store).  A 32x32 tile is computed with mmq_kernel's
// instructions on the same operands (integer block sums by two MFMAs, the
// d_a (x) d_w outer product by one, acc = fma(isum, S, acc) in block order,
// the Q4_1 offset term by MFMA per pair of blocks), so the results are
// bit-identical to mmq_kernel's.  F16 weights stay on mmq_kernel: at 2 bytes
// per element their LDS copy leaves one workgroup per CU, and the tiled
// kernel is faster there.
namespace {
constexpr int SKMAX = 128;  // largest K
}  // namespace

struct SkinnyArgs {
    const uint8_t* W;
    int64_t w_nb1;             // weight row stride (bytes, even)
    const _Float16* A;         // activation operand rows, stride a_s1 halves (16-byte aligned)
    int64_t a_s1;
    const _Float16* Ad;        // [M][dp] scales (quantized path)
    const _Float16* As;        // [M][dp] Q8_1 sums (Q4_1)
    float* D;
    int64_t d_nb1;
    int M, N, K, dp, npad;     // npad: N rounded up to 32
    int wpitch;                // LDS bytes per weight row (the raw row size)
};

template <int WT, int SMT>  // SMT: 32-row MFMA tiles per workgroup (2 or 4)
__global__ __launch_bounds__(256, 2) void mmq_skinny_kernel(const SkinnyArgs p) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr int SBM = 32 * SMT;  // activation rows of this workgroup
    constexpr int WB = WInfo<WT>::bytes, HDR = WInfo<WT>::hdr;
    constexpr int NA = SKMAX / 8 * SBM / 256;  // activation chunks per thread (at most)
    const int K = p.K, PA = K + 8, nb = K / QK, dp = p.dp, M = p.M, N = p.N;
    const int CPR = K / 8;          // 16-byte chunks per activation row
    const int ACH = SBM * CPR;      // chunks of the activation block
    const int SCH = SBM * dp / 8;   // 16-byte chunks of its scales
    // LDS: weights | activations [SBM][PA] | scales [SBM][dp] | sums [SBM][dp] | output staging [4][32][32]
    uint8_t* Wl = smem;
    _Float16* Al = reinterpret_cast<_Float16*>(smem + ((p.npad * p.wpitch + 16 + 15) & ~15));
    uint16_t* Adl = reinterpret_cast<uint16_t*>(Al + SBM * PA);
    uint16_t* Asl = Adl + SBM * dp;
    float* Ol = reinterpret_cast<float*>(Asl + SBM * dp);
    const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, g = lane >> 5;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool lo = lane < 32;
    const int m0 = blockIdx.x * SBM;

    // this block's activation rows and scales into registers (in flight during the weight copy)
    uint4 ra[NA], rd = {0, 0, 0, 0}, rs = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < NA; ++i) {
        const int c = tid + 256 * i;
        const int r = c / CPR, c8 = c - r * CPR;
        ra[i] = c < ACH && m0 + r < M ? *reinterpret_cast<const uint4*>(p.A + (int64_t)(m0 + r) * p.a_s1 + 8 * c8)
                                      : uint4{0, 0, 0, 0};
    }
    if (tid < SCH) {
        const int64_t o = (int64_t)m0 * dp + 8 * tid, end = (int64_t)M * dp;
        if (o + 8 <= end) {
            rd = *reinterpret_cast<const uint4*>(p.Ad + o);
            if (WT == T_Q4_1) rs = *reinterpret_cast<const uint4*>(p.As + o);
        } else {  // the block's last rows run past M: element loads up to the end
            uint16_t hd[8], hs[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                hd[e] = o + e < end ? reinterpret_cast<const uint16_t*>(p.Ad)[o + e] : (uint16_t)0;
                hs[e] = WT == T_Q4_1 && o + e < end ? reinterpret_cast<const uint16_t*>(p.As)[o + e] : (uint16_t)0;
            }
            rd = __builtin_bit_cast(uint4, hd);
            rs = __builtin_bit_cast(uint4, hs);
        }
    }

    // weights from contiguous rows (16-byte aligned base), 16-byte chunks with eight
    // loads in flight per thread (indices clamped, stores guarded), unpadded: row n
    // at byte n * wpitch
    {
        const int rowb = nb * WB;
        const int nch = (N * rowb) / 16;
        const uint4* src = reinterpret_cast<const uint4*>(p.W);
        for (int c0 = 0; c0 < nch; c0 += 8 * 256) {
            uint4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = src[min(c0 + u * 256 + tid, nch - 1)];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int c = c0 + u * 256 + tid;
                if (c < nch) *reinterpret_cast<uint4*>(Wl + 16 * c) = v[u];
            }
        }
        uint16_t* L16 = reinterpret_cast<uint16_t*>(Wl);
        const uint16_t* W16 = reinterpret_cast<const uint16_t*>(p.W);
        // the tail by halves, then zero rows up to npad
        for (int h = 8 * nch + tid; h < N * rowb / 2; h += 256) L16[h] = W16[h];
        for (int h = N * rowb / 2 + tid; h < p.npad * p.wpitch / 2; h += 256) L16[h] = 0;
    }
#pragma unroll
    for (int i = 0; i < NA; ++i) {
        const int c = tid + 256 * i;
        if (c < ACH) {
            const int r = c / CPR, c8 = c - r * CPR;
            *reinterpret_cast<uint4*>(&Al[r * PA + 8 * c8]) = ra[i];
        }
    }
    if (tid < SCH) {
        *reinterpret_cast<uint4*>(&Adl[8 * tid]) = rd;
        if (WT == T_Q4_1) *reinterpret_cast<uint4*>(&Asl[8 * tid]) = rs;
    }
    __syncthreads();

    const v16f zf = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    const uint32_t* As32 = reinterpret_cast<const uint32_t*>(Asl);
    auto fa = [&](int r, int c) { return *reinterpret_cast<const v8h*>(&Al[r * PA + 8 * c]); };
    float* stg = Ol + wv * 32 * 32;  // this wavefront's 32x32 staging tile
    const bool v4 = (p.d_nb1 & 15) == 0 && (reinterpret_cast<uintptr_t>(p.D) & 15) == 0;
    for (int j = wv; j < p.npad / 32; j += 4) {
        const int n = 32 * j + lr;  // this lane's weight row
        v16f acc[SMT];
#pragma unroll
        for (int mt = 0; mt < SMT; ++mt) acc[mt] = zf;
        {
            // row n starts at byte n * wpitch (even): dwords are read from the LDS base, with
            // lds_dw2 aligning a half-dword offset
            const uint32_t* rowp = reinterpret_cast<const uint32_t*>(Wl);
            const int rb0 = n * p.wpitch;
            const uint16_t* hrow = reinterpret_cast<const uint16_t*>(Wl + rb0);
            for (int s = 0; s < (nb + 1) / 2; ++s) {
                if (WT == T_Q4_1) {
                    const uint32_t m1 = 2 * s + 1 < nb ? (uint32_t)hrow[(2 * s + 1) * WB / 2 + 1] << 16 : 0u;
                    const v4i mwf = {lo ? (int)((uint32_t)hrow[s * WB + 1] | m1) : 0, 0, 0, 0};
#pragma unroll
                    for (int mt = 0; mt < SMT; ++mt) {
                        const int ar = mt * 32 + lr;
                        v4i saf = __builtin_bit_cast(v4i, fa(ar, 8 * s + g));  // finite filler
                        saf[0] = (int)As32[ar * dp / 2 + s];
                        acc[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, saf),
                                                                         __builtin_bit_cast(v8h, mwf), acc[mt], 0, 0, 0);
                    }
                }
                for (int bk = 2 * s; bk < 2 * s + 2 && bk < nb; ++bk) {
                    v8h bf[2];
                    const int o = rb0 + bk * WB + HDR;
                    if (WT == T_Q8_0) {
#pragma unroll
                        for (int h = 0; h < 2; ++h) {
                            uint32_t w0, w1;
                            lds_dw2(rowp, o + 16 * h + 8 * g, o & 3, w0, w1);
                            bf[h] = i8x8_to_h8(w0, w1);
                        }
                    } else {
                        uint32_t w0, w1;
                        lds_dw2(rowp, o + 8 * g, o & 3, w0, w1);
                        const _Float16 bias = WT == T_Q4_0 ? (_Float16)1032.0f : (_Float16)1024.0f;
                        bf[0] = n8_to_h8(w0 & 0x0f0f0f0fu, w1 & 0x0f0f0f0fu, bias);
                        bf[1] = n8_to_h8((w0 >> 4) & 0x0f0f0f0fu, (w1 >> 4) & 0x0f0f0f0fu, bias);
                    }
                    const v4i dwf = {lo ? (int)(uint32_t)hrow[bk * WB / 2] : 0, 0, 0, 0};
#pragma unroll
                    for (int mt = 0; mt < SMT; ++mt) {
                        const int ar = mt * 32 + lr;
                        const v8h a0 = fa(ar, 4 * bk + g), a1 = fa(ar, 4 * bk + 2 + g);
                        v16f I = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, bf[0], zf, 0, 0, 0);
                        I = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, bf[1], I, 0, 0, 0);
                        v4i daf = __builtin_bit_cast(v4i, a1);
                        daf[0] = (int)(uint32_t)Adl[ar * dp + bk];
                        const v16f S = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, daf),
                                                                              __builtin_bit_cast(v8h, dwf), zf, 0, 0, 0);
#pragma unroll
                        for (int i = 0; i < 16; ++i) acc[mt][i] = __builtin_fmaf(I[i], S[i], acc[mt][i]);
                    }
                }
            }
        }
        // 32x32 tiles through this wavefront's staging area (tile32_row): rows of 32 floats go
        // out as eight float4 (one 128-byte line per row)
        const int rr = lane >> 3, cc = 4 * (lane & 7), nc = 32 * j + cc;
#pragma unroll
        for (int mt = 0; mt < SMT; ++mt) {
#pragma unroll
            for (int i = 0; i < 16; ++i) stg[tile32_row(8 * (i >> 2) + 4 * g + (i & 3)) + lr] = acc[mt][i];
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int m = m0 + mt * 32 + 8 * q + rr;
                const v4f val = *reinterpret_cast<const v4f*>(&stg[tile32_row(8 * q + rr) + cc]);
                if (m < M) {
                    float* dst = reinterpret_cast<float*>(reinterpret_cast<char*>(p.D) + (int64_t)m * p.d_nb1) + nc;
                    if (v4 && nc + 4 <= N) {
                        *reinterpret_cast<v4f*>(dst) = val;
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (nc + e < N) dst[e] = val[e];
                    }
                }
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads done before the next tile overwrites
        }
    }
}

// LDS bytes of the skinny kernel with SMT row tiles, or 0 when the GEMM does not fit it.
static size_t skinny_lds(int type, int64_t N, int64_t K, int dp, int smt, int* wpitch) {
    if (K <= 0 || K > SKMAX || K % QK != 0 || N <= 0 || N > 1024) return 0;
    const int64_t wp = (K / QK) * (type == T_Q8_0 ? 34 : type == T_Q4_0 ? 18 : 20);
    const int64_t npad = (N + 31) / 32 * 32, sbm = 32 * smt;
    // weights (+16 bytes: the last row's fragment reads run up to 12 bytes past it), rounded to 16;
    // activations, scales and sums; four 32x32 f32 output staging tiles
    const size_t wbytes = ((size_t)(npad * wp) + 16 + 15) & ~(size_t)15;
    const size_t bytes = wbytes + sbm * (K + 8) * 2 + 2 * sbm * dp * 2 + 4 * 32 * 32 * 4;
    *wpitch = (int)wp;
    return bytes <= 150 * 1024 ? bytes : 0;
}

// Runs the GEMM on the skinny kernel when its shape fits; *done reports it.
static hipError_t try_skinny(const MatW& w, const ActF16& a, const MatD& d, int64_t N, int64_t ne12, int64_t ne13,
                             int32_t* dots, const MmqEpi* epi, const MmqSplit& sp, hipStream_t st, bool* done) {
    *done = false;
    if (!sp.skinny || dots || (epi && epi->kind != MMQ_EPI_STORE) || ne12 * ne13 != 1 || a.M < 4096) return hipSuccess;
    // F16 weights stay on the tiled kernel: their LDS rows (2 bytes per element) leave
    // one workgroup per CU, and the tiled kernel is faster there
    if (w.type == T_F16 || a.dp > 4 || a.dp % 2 != 0) return hipSuccess;
    const int dp = (int)a.dp;
    int wpitch = 0;
    // 128-row workgroups at large M while two fit per CU (a quarter of the weight
    // copies per output row), 64 rows otherwise
    int smt = 4;
    size_t lds = skinny_lds(w.type, N, a.K, dp, smt, &wpitch);
    if (a.M < 32768 || !lds || lds > 75 * 1024) {
        smt = 2;
        lds = skinny_lds(w.type, N, a.K, dp, smt, &wpitch);
    }
    const int64_t rowb = (a.K / QK) * (w.type == T_Q8_0 ? 34 : w.type == T_Q4_0 ? 18 : 20);
    if (!lds || a.s1 % 8 != 0 || w.nb1 != rowb || (reinterpret_cast<uintptr_t>(w.data) & 15) ||
        (reinterpret_cast<uintptr_t>(a.q) & 15) || (d.nb1 & 3) || (reinterpret_cast<uintptr_t>(d.data) & 3) ||
        (reinterpret_cast<uintptr_t>(a.d) & 15) || (w.type == T_Q4_1 && (reinterpret_cast<uintptr_t>(a.s) & 15)))
        return hipSuccess;
    SkinnyArgs p;
    p.W = w.data;
    p.w_nb1 = w.nb1;
    p.A = static_cast<const _Float16*>(a.q);
    p.a_s1 = a.s1;
    p.Ad = static_cast<const _Float16*>(a.d);
    p.As = static_cast<const _Float16*>(a.s);
    p.D = d.data;
    p.d_nb1 = d.nb1;
    p.M = (int)a.M;
    p.N = (int)N;
    p.K = (int)a.K;
    p.dp = dp;
    p.npad = (int)((N + 31) / 32 * 32);
    p.wpitch = wpitch;
    const unsigned grid = (unsigned)((a.M + 32 * smt - 1) / (32 * smt));
    // dynamic LDS beyond 64 KB, allowed once per kernel and device (the attribute is
    // per device); host threads making their first calls together may each set it,
    // which repeats the same setting, and the flags are atomics so that is no data race
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return hipSuccess;
    static std::atomic<bool> attr[64][6] = {};
    const int ti = (w.type == T_Q8_0 ? 0 : w.type == T_Q4_0 ? 1 : 2) * 2 + (smt == 4 ? 1 : 0);
    const void* fns[6] = {(const void*)mmq_skinny_kernel<T_Q8_0, 2>, (const void*)mmq_skinny_kernel<T_Q8_0, 4>,
                          (const void*)mmq_skinny_kernel<T_Q4_0, 2>, (const void*)mmq_skinny_kernel<T_Q4_0, 4>,
                          (const void*)mmq_skinny_kernel<T_Q4_1, 2>, (const void*)mmq_skinny_kernel<T_Q4_1, 4>};
    if (!attr[dev][ti].load(std::memory_order_acquire)) {
        if (hipFuncSetAttribute(fns[ti], hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024) != hipSuccess) {
            (void)hipGetLastError();  // not done: the tiled kernel takes it
            return hipSuccess;
        }
        attr[dev][ti].store(true, std::memory_order_release);
    }
    switch (ti) {
        case 0: mmq_skinny_kernel<T_Q8_0, 2><<<grid, 256, lds, st>>>(p); break;
        case 1: mmq_skinny_kernel<T_Q8_0, 4><<<grid, 256, lds, st>>>(p); break;
        case 2: mmq_skinny_kernel<T_Q4_0, 2><<<grid, 256, lds, st>>>(p); break;
        case 3: mmq_skinny_kernel<T_Q4_0, 4><<<grid, 256, lds, st>>>(p); break;
        case 4: mmq_skinny_kernel<T_Q4_1, 2><<<grid, 256, lds, st>>>(p); break;
        default: mmq_skinny_kernel<T_Q4_1, 4><<<grid, 256, lds, st>>>(p); break;
    }
    *done = true;
    return hipGetLastError();
}

static hipError_t run_mmq(const MatW& w_in, const ActF16& a, const MatD& d, int64_t N, int64_t ne12, int64_t ne13,
                          int32_t* dots, const MmqEpi* epi, void* align_buf, const MmqSplit& sp, hipStream_t st) {
    {
        bool done = false;
        const hipError_t e = try_skinny(w_in, a, d, N, ne12, ne13, dots, epi, sp, st, &done);
        if (done || e != hipSuccess) return e;
    }
    MatW w = w_in;
    // F16 runs K to a whole 16-byte chunk: the weight copy below and the
    // activation operand (a.s1 >= kk, zero from K to kk) carry zeros there
    const int64_t kk = w.type == T_F16 ? (a.K + 7) & ~7 : a.K;
    if (kk != a.K && a.s1 < kk) return hipErrorInvalidValue;
    int64_t rowb = w.type == T_F16 ? a.K * 2 : (a.K / QK) * (w.type == T_Q8_0 ? 34 : w.type == T_Q4_0 ? 18 : 20);
    if (mmq_align_bytes(w_in, N, a.K) != 0) {
        // weight rows are not aligned for the DMA: copy them to a zero-padded pitch first
        const int64_t pitch = w.type == T_F16 ? kk * 2 : (rowb + 3) & ~3, rows = N * w.ne2 * w.ne3;
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
    p.a_extent = ((a.M - 1) * a.s1 + kk) * 2;
    p.Ad = static_cast<const _Float16*>(a.d);
    p.As = static_cast<const _Float16*>(a.s);
    p.D = d.data;
    p.d_nb1 = d.nb1;
    p.d_nb2 = d.nb2;
    p.d_nb3 = d.nb3;
    p.dots = dots;
    p.M = (int)a.M;
    p.dp = (int)a.dp;
    p.N = (int)N;
    p.K = (int)kk;
    p.ne12 = (int)ne12;
    p.r2 = (int)(ne12 / w.ne2);
    p.r3 = (int)(ne13 / w.ne3);
    p.tiles_m = (int)((a.M + BM - 1) / BM);
    p.tiles_n = (int)((N + BN - 1) / BN);
    {
        // group height: the fewest L2 bytes for the ~64 workgroups an XCD runs at once
        // (32 CUs x 2): gm activation row tiles plus 64 / gm weight column tiles
        const double at = (double)BM * kk * 2, wt = (double)BN * rowb;
        double best = 0;
        p.gm = 1;
        for (int gm = 1; gm <= 16 && gm <= p.tiles_m; gm *= 2) {
            const double c = gm * at + ((64 + gm - 1) / gm) * wt;
            if (gm == 1 || c < best) {
                best = c;
                p.gm = gm;
            }
        }
    }
    const int nstage = w.type != T_F16 ? (int)(((a.K / QK) + BKB - 1) / BKB) : (int)((kk + 31) / 32);
    const bool split = sp.ks > 1 && !dots && ne12 * ne13 == 1;
    p.ksplit = split ? sp.ks : 1;
    p.sps = split ? (nstage + sp.ks - 1) / sp.ks : nstage;
    p.d_split = 0;
    if (split) {
        if (!sp.part || N % 4 != 0 || (int64_t)(sp.ks - 1) * p.sps >= nstage) return hipErrorInvalidValue;
        p.D = sp.part;
        p.d_nb1 = N * 4;
        p.d_nb2 = p.d_nb3 = 0;
        p.d_split = a.M * N * 4;
    }
    // buffer offsets are 32-bit
    if (p.w_extent >= OOB || p.a_extent >= OOB || 2 * a.M * a.dp >= OOB) return hipErrorInvalidValue;
    const int Z = (int)(ne12 * ne13);
    p.d_v4 = !dots && N % 4 == 0 && p.d_nb1 % 16 == 0 && (reinterpret_cast<uintptr_t>(p.D) & 15) == 0 &&
             (Z == 1 || (p.d_nb2 % 16 == 0 && p.d_nb3 % 16 == 0));
    switch (w.type) {
        case T_Q8_0: launch_t<T_Q8_0>(p, Z, dots, epi, st); break;
        case T_Q4_0: launch_t<T_Q4_0>(p, Z, dots, epi, st); break;
        case T_Q4_1: launch_t<T_Q4_1>(p, Z, dots, epi, st); break;
        case T_F16: launch_t<T_F16>(p, Z, false, epi, st); break;
        default: return hipErrorInvalidValue;
    }
    if (split) {
        const int64_t n = a.M * (N / 4);
        const unsigned g = (unsigned)((n + 255) / 256);
        char* D = reinterpret_cast<char*>(d.data);
        if (!epi || epi->kind == MMQ_EPI_STORE)
            mmq_reduce_kernel<MMQ_EPI_STORE><<<g, 256, 0, st>>>(sp.part, sp.ks, (int)a.M, (int)N, D, d.nb1, MmqEpi{},
                                                                reduce_rcp(a.M, N));
        else if (epi->kind == MMQ_EPI_RESIDUAL)
            mmq_reduce_kernel<MMQ_EPI_RESIDUAL><<<g, 256, 0, st>>>(sp.part, sp.ks, (int)a.M, (int)N, D, 0, *epi,
                                                                   reduce_rcp(a.M, N));
        else
            mmq_reduce_kernel<MMQ_EPI_QKV><<<g, 256, 0, st>>>(sp.part, sp.ks, (int)a.M, (int)N, D, 0, *epi,
                                                              reduce_rcp(a.M, N));
    }
    return hipGetLastError();
}

hipError_t launch_mmq_reduce(const float* part, int ks, int M, int N, char* D, int64_t d_nb1, const MmqEpi* epi,
                             hipStream_t st) {
    const int64_t n = (int64_t)M * (N / 4);
    const unsigned g = (unsigned)((n + 255) / 256);
    if (!epi || epi->kind == MMQ_EPI_STORE)
        mmq_reduce_kernel<MMQ_EPI_STORE><<<g, 256, 0, st>>>(part, ks, M, N, D, d_nb1, MmqEpi{}, reduce_rcp(M, N));
    else if (epi->kind == MMQ_EPI_RESIDUAL)
        mmq_reduce_kernel<MMQ_EPI_RESIDUAL><<<g, 256, 0, st>>>(part, ks, M, N, D, 0, *epi, reduce_rcp(M, N));
    else
        mmq_reduce_kernel<MMQ_EPI_QKV><<<g, 256, 0, st>>>(part, ks, M, N, D, 0, *epi, reduce_rcp(M, N));
    return hipGetLastError();
}

hipError_t launch_mmq(const MatW& w, const ActF16& a, const MatD& d, int64_t N, int64_t ne12, int64_t ne13,
                      int32_t* dots, void* align_buf, const MmqSplit& sp, hipStream_t st) {
    if (sp.ks > 1 && (d.nb1 % 16 != 0 || (reinterpret_cast<uintptr_t>(d.data) & 15) != 0)) return hipErrorInvalidValue;
    return run_mmq(w, a, d, N, ne12, ne13, dots, nullptr, align_buf, sp, st);
}

hipError_t launch_mmq_epi(const MatW& w, const ActF16& a, int64_t N, const MmqEpi& e, void* align_buf,
                          const MmqSplit& sp, hipStream_t st) {
    if (!e.bias || N % 4 != 0) return hipErrorInvalidValue;
    if (e.kind == MMQ_EPI_RESIDUAL) {
        if (!e.res || !e.out) return hipErrorInvalidValue;
    } else if (e.kind == MMQ_EPI_QKV) {
        if (!e.q || !e.k || !e.v || e.ntok <= 0 || e.nh <= 0 || e.hd <= 0 || e.hd % 4 != 0 || N != 3LL * e.nh * e.hd ||
            a.M % e.ntok != 0)
            return hipErrorInvalidValue;
    } else {
        return hipErrorInvalidValue;
    }
    const MatD none{nullptr, 0, 0, 0};
    return run_mmq(w, a, none, N, 1, 1, nullptr, &e, align_buf, sp, st);
}

}  // namespace mi355
