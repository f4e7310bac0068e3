// ggml MUL_MAT on gfx950 with int8 MFMA: Q8_0 / Q4_0 / Q4_1 weights against
// Q8_0 / Q8_1-quantized activations, both operands one byte per element.
//
//   dst[m][n] = sum_b fp32(d_w[n][b]) * fp32(d_a[m][b]) * isum[m][n][b]
//               (+ sum_b fp32(m_w[n][b]) * fp32(s_a[m][b]) for Q4_1)
//   isum[m][n][b] = sum_{j<32} q_w[n][32b+j] * q_a[m][32b+j]     (exact int32)
//
// One v_mfma_i32_32x32x32_i8 gives a 32x32 tile's isum of one block with
// int32 accumulation onto the bias 0x4B400000: its result is the bit pattern
// of the fp32 1.5 * 2^23 + isum (|isum| <= 32 * 128 * 128 < 2^22), so one
// full-rate subtraction recovers float(isum) exactly where v_cvt_f32_i32
// would issue at half rate.  The scale product d_a (x) d_w of the tile is one
// v_mfma_f32_32x32x8f16 (an outer product in k-slot 0 or 1; fp16 x fp16 is
// exact in fp32; 2-register operands), and the combine is
// acc = fma(float(isum), S, acc) in block order: the same
// fp32 operations in the same order as mmq_kernel, whose fp16 MFMAs over
// integer-valued halves give the same exact isum, so the two kernels' outputs
// are bit-identical.  Q4_1's offset term is accumulated into acc by one
// MFMA per stage before the stage's blocks, as mmq_kernel does.
//
// Operands (the int8 layouts, kernels.h ActI8 / WRep): activation quants
// int8 [M][K] with fp16 scales (and Q8_1 sums) [M][dp]; weights repacked
// once into int8 quants [N][K] (Q8_0 as stored, Q4_0 as nibble - 8, Q4_1 as
// the nibble) with fp16 d (and m) [N][dpw].  Rows are 16-byte aligned, so
// every stage moves by buffer_load_dwordx4 ... lds (LDS DMA): 1 KB per
// wavefront instruction, no staging registers, no decode in the K loop.
//
// Tiling: workgroup 128(m) x 128(n), four wavefronts in 2 x 2, each 64 x 64
// (2 x 2 MFMA tiles).  K advances 64 bytes (two blocks) per stage through
// three LDS stages filled two stages ahead.  A tile row is 64 bytes = four
// 16-byte chunks; chunk c of row r sits in slot c ^ ((r >> 2) & 3), so the 16
// consecutive rows one ds_read_b128 pass serves cover all 64 banks.
#include <atomic>
#include <type_traits>

#include "common.cuh"
#include "kernels.h"

namespace mi355 {

namespace {
constexpr int B8M = 128, B8N = 128, SKB = 64;  // tile rows, tile columns, K bytes per stage
constexpr int NT8 = 256;
constexpr int OOB8 = 0x40000000;
constexpr int kBias = 0x4B400000;      // fp32 1.5 * 2^23 as bits
constexpr float kBiasF = 12582912.0f;  // 1.5 * 2^23
}  // namespace

struct Mmq8Args {
    const int8_t* A;       // [M][K] activation quants, row stride a_s1 bytes (multiple of 16)
    int64_t a_s1;
    const uint32_t* Adl;   // [M][nst] d_a of block 2s in the low half of dword s
    const uint32_t* Adh;   // [M][nst] d_a of block 2s + 1 in the high half
    const _Float16* As;    // [M][2 nst] Q8_1 sums (Q4_1)
    const int8_t* W;       // [N][K] repacked weight quants, row stride w_s1 bytes (multiple of 16)
    int64_t w_s1;
    const _Float16* Wd;    // [N][2 nst] weight scales (dword s = blocks 2s, 2s+1)
    const _Float16* Wm;    // [N][2 nst] Q4_1 minima
    float* D;
    int64_t d_nb1;         // bytes
    int M, N, K, nst, tiles_m, tiles_n, gm;
    int ksplit, sps;       // K split into ksplit ranges of sps stages (partial sums at D + split * d_split)
    int64_t d_split;
    int d_v4;              // float4 row stores through LDS
    int32_t* dots;         // block-dot inspection output [M][N][nbt] (or null)
    int nbt;               // blocks per row of the whole K
};

template <int WT, int TM>
struct St8 {
    static constexpr bool Q41 = WT == T_Q4_1;
    int8_t A[TM * SKB];
    int8_t W[B8N * SKB];
    uint32_t adl[TM];          // d_a of the stage's block 0 per row (low half)
    uint32_t adh[TM];          // d_a of block 1 per row (high half)
    uint32_t wd[B8N];          // d_w of blocks 0, 1 per row
    uint32_t as[Q41 ? TM : 1];
    uint32_t wm[Q41 ? B8N : 1];
    uint32_t zero[4];          // read by lanes 32..63 for the scale MFMA's B operand
};

__device__ __forceinline__ int slot8(int r, int c) { return c ^ ((r >> 2) & 3); }

// The epilogue of one float4 of results: row m, columns nc .. nc + 3 (nc < N, N % 4 == 0):
// stored to Dz (row pitch d_nb1 bytes), or + bias and added to the residual row rr = map(m)
// (pv: that row's four values, loaded by the caller), or + bias, split into q / k / v as
// fp16 (RoPE on q and k by the factors pv, loaded by the caller from e.rope row tn, column
// d).  The qkv columns (destination, head, first dimension) are the lane's, fixed for the
// whole epilogue, and the row's window bw and token tn come from the caller.
struct QkvLane {
    _Float16* dst;
    int hh, d;
    bool rope;
};
template <int EPI>
__device__ __forceinline__ void epi4(char* Dz, int64_t d_nb1, const MmqEpi& e, int N, int m, int nc, v4f v, v4f bv,
                                     int rr, const QkvLane& ql, int bw, int tn, v4f pv) {
    if (EPI == MMQ_EPI_STORE) {
        *reinterpret_cast<v4f*>(Dz + (int64_t)m * d_nb1 + (int64_t)nc * 4) = v;
    } else if (EPI == MMQ_EPI_RESIDUAL) {
        if (rr >= 0) *reinterpret_cast<v4f*>(&e.out[(int64_t)rr * N + nc]) = pv + (v + bv);
    } else {
        const v4f uv = v + bv;
        float u0 = uv[0], u1 = uv[1], u2 = uv[2], u3 = uv[3];
        if (ql.rope) {
            rope_pair(u0, u1, pv[0], pv[1]);
            rope_pair(u2, u3, pv[2], pv[3]);
        }
        const uint32_t h0 = (uint32_t)f2h(u0) | ((uint32_t)f2h(u1) << 16);
        const uint32_t h1 = (uint32_t)f2h(u2) | ((uint32_t)f2h(u3) << 16);
        *reinterpret_cast<uint2*>(&ql.dst[((int64_t)bw * e.nh + ql.hh) * ((int64_t)e.ntok * e.hd) + tn * e.hd + ql.d]) =
            make_uint2(h0, h1);
    }
}

// Per-stage pipeline (three LDS buffers, DMA three stages ahead):
//   units of block 0 (fragments prefetched in registers)
//   wait for stage s+1's DMA, barrier: every wavefront has also finished
//     reading stage s's buffer, which is refilled with stage s+3
//   prefetch stage s+1's block-0 fragments; units of block 1;
//   prefetch stage s+1's block-1 fragments.
// A unit (block, m-tile, n-tile) issues its scale MFMA and isum MFMA into
// buffer u % 2 and combines the previous unit (across stage boundaries).
// TM = 128: each wavefront computes 64 x 64 (2 x 2 MFMA tiles), two workgroups per CU.
// TM = 64 (GEMMs whose 128-row grid leaves CUs idle): 32 x 64 per wavefront (1 x 2 tiles),
// also two workgroups per CU (three would cap the registers at 168 and spill in the K loop).
template <int WT, int EPI, bool DOTS = false, int TM = 128>
__global__ __launch_bounds__(NT8, 2) void mmq8_kernel(const Mmq8Args p, const MmqEpi e) {
    using St = St8<WT, TM>;
    constexpr bool Q41 = WT == T_Q4_1;
    constexpr int MT = TM / 64;   // 32-row MFMA tiles per wavefront
    constexpr int WMR = 32 * MT;  // rows per wavefront (wavefronts 2 (m) x 2 (n))
    constexpr int NU = 2 * MT;    // units (MFMA tile pairs) per block
    __shared__ __attribute__((aligned(16))) St st0;
    __shared__ __attribute__((aligned(16))) St st1;
    __shared__ __attribute__((aligned(16))) St st2;

    // XCD-aware, grouped tile order (as mmq_kernel): each XCD walks a contiguous band. The K
    // split is the slowest index, so the workgroups an XCD runs at once share one K range
    const int tiles = p.tiles_m * p.tiles_n, TT = tiles * p.ksplit;
    const int per_xcd = (TT + 7) / 8;
    const int tl = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (tl >= TT) return;
    const int split = tl / tiles, t = tl - split * tiles;
    const int gsz = p.gm * p.tiles_n, grp = t / gsz, gr = t - grp * gsz;
    const int gmr = min(p.gm, p.tiles_m - grp * p.gm);
    const int m0 = (grp * p.gm + gr % gmr) * TM, n0 = (gr / gmr) * B8N;

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int M = p.M, N = p.N;
    const int kb0 = split * p.sps * SKB;        // first K byte of this split
    const int K = min(p.K - kb0, p.sps * SKB);  // K bytes (elements) of this split
    const int nstage = (K / QK + 1) / 2;
    const int so0 = kb0 / SKB;                  // first stage (scale dword) of this split
    const int8_t* Az = p.A + kb0;
    const int8_t* Wz = p.W + kb0;
    const int64_t a_ext = (int64_t)(M - 1) * p.a_s1 + p.K - kb0;
    const int64_t w_ext = (int64_t)(N - 1) * p.w_s1 + p.K - kb0;
    const int64_t sa_ext = 4LL * M * p.nst - 4LL * so0, sw_ext = 4LL * N * p.nst - 4LL * so0;

    if (tid < 4) st0.zero[tid] = st1.zero[tid] = st2.zero[tid] = 0u;
    // fused epilogues: where each of the tile's rows goes, worked out once per workgroup (one
    // row per thread; published by the barrier before the K loop): residual -> the mapped row,
    // or -1 (padding or past M); qkv -> window and token
    __shared__ int rtab[EPI == MMQ_EPI_STORE ? 1 : 2 * TM];
    if (EPI != MMQ_EPI_STORE && tid < TM) {
        const int m = m0 + tid;
        if (EPI == MMQ_EPI_RESIDUAL) {
            rtab[tid] = m < M ? map_row32(e.map, rowmap_rcp(e.map), m) : -1;
        } else {
            int tn;
            rtab[tid] = div_rcp(m, e.ntok, 1.0 / (double)e.ntok, tn);
            rtab[TM + tid] = tn;
        }
    }

    // ---- DMA offsets (fixed for the whole K loop)
    // A-tile instruction i of wavefront w: rows (MT w + i) * 16 + lane / 4; W-tile instruction i:
    // rows (2w + i) * 16 + lane / 4; LDS slot lane % 4.  The global chunk a lane loads,
    // slot8(row, lane % 4), depends on the row only through (row >> 2) & 3 = (lane >> 4) & 3.
    const int tch = slot8(lane >> 2, lane & 3);
    int aoff[MT], woff[2];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const int row = (MT * w + i) * 16 + (lane >> 2);
        aoff[i] = m0 + row < M ? (int)((int64_t)(m0 + row) * p.a_s1) + tch * 16 : OOB8;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int row = (2 * w + i) * 16 + (lane >> 2);
        woff[i] = n0 + row < N ? (int)((int64_t)(n0 + row) * p.w_s1) + tch * 16 : OOB8;
    }
    // scale dwords: wavefronts 0, 1 load d_a (both halves, and for Q4_1 the Q8_1 sums) of rows
    // 64 (w & 1) + lane, 2 and 3 d_w (and for Q4_1 the minima); at 128 rows the d_w side issues
    // one scale DMA fewer than the d_a side (NL - 1 per stage), and each side waits on its own count
    // (TM = 64: d_a has one wavefront's worth of rows; wavefront 0 loads its low halves and
    // wavefront 1 its high halves, Q4_1's sums loaded by both)
    const bool a_side = w < 2;
    const int srow = (a_side && TM == 64 ? 0 : 64 * (w & 1)) + lane;
    const int soff = a_side ? (m0 + srow < M ? (int)((int64_t)(m0 + srow) * p.nst * 4) : OOB8)
                            : (n0 + srow < N ? (int)((int64_t)(n0 + srow) * p.nst * 4) : OOB8);
    constexpr int NS = (TM == 128 ? 2 : 1) + (Q41 ? 1 : 0);  // scale DMA instructions per stage and wavefront
    constexpr int NL = MT + 2 + NS;                          // all DMA instructions per stage, d_a side
    // the d_w side at 128 rows: rs[0] and rs[1] would both be d_w; it loads it once (NL - 1 instructions)
    const bool wdup = TM == 128 && !a_side;
    // descriptors and LDS destinations, fixed for the whole K loop: stage s adds s * SKB (tiles)
    // or 4 s (scale dwords) in the instructions' SGPR offset
    const v4i ar = make_rsrc(Az, a_ext), wr = make_rsrc(Wz, w_ext);
    v4i rs[NS];
    uint32_t ls[NS];
    {
        const uint32_t half = 256u * (uint32_t)(w & 1);
        if (TM == 64 && a_side) {
            const bool hi = w & 1;
            rs[0] = make_rsrc(hi ? p.Adh + so0 : p.Adl + so0, sa_ext);
            ls[0] = (uint32_t)(hi ? offsetof(St, adh) : offsetof(St, adl));
            if (Q41) {
                rs[NS - 1] = make_rsrc(p.As + 2 * so0, sa_ext);
                ls[NS - 1] = (uint32_t)offsetof(St, as);
            }
        } else if (a_side) {
            rs[0] = make_rsrc(p.Adl + so0, sa_ext);
            ls[0] = (uint32_t)offsetof(St, adl) + half;
            rs[NS > 1 ? 1 : 0] = make_rsrc(p.Adh + so0, sa_ext);
            ls[NS > 1 ? 1 : 0] = (uint32_t)offsetof(St, adh) + half;
            if (Q41) {
                rs[NS - 1] = make_rsrc(p.As + 2 * so0, sa_ext);
                ls[NS - 1] = (uint32_t)offsetof(St, as) + half;
            }
        } else {
            for (int j = 0; j < NS; ++j) {  // d_w (twice at 128 rows, the first skipped; then Q4_1's minima)
                rs[j] = make_rsrc(p.Wd + 2 * so0, sw_ext);
                ls[j] = (uint32_t)offsetof(St, wd) + half;
            }
            if (Q41) {
                rs[NS - 1] = make_rsrc(p.Wm + 2 * so0, sw_ext);
                ls[NS - 1] = (uint32_t)offsetof(St, wm) + half;
            }
        }
    }
    uint32_t lta[MT], ltw[2];  // this wavefront's tile rows inside a stage buffer
#pragma unroll
    for (int i = 0; i < MT; ++i) lta[i] = (uint32_t)offsetof(St, A) + (uint32_t)((MT * w + i) * 16 * SKB);
#pragma unroll
    for (int i = 0; i < 2; ++i) ltw[i] = (uint32_t)offsetof(St, W) + (uint32_t)((2 * w + i) * 16 * SKB);
    const uint32_t lbuf[3] = {(uint32_t)__builtin_amdgcn_readfirstlane(lds_addr(&st0)),
                              (uint32_t)__builtin_amdgcn_readfirstlane(lds_addr(&st1)),
                              (uint32_t)__builtin_amdgcn_readfirstlane(lds_addr(&st2))};

    // stage s into the buffer at LDS address lb; chunks past the split's K read zero
    auto dma_stage = [&](int s, uint32_t lb) __attribute__((always_inline)) {
        const int k0 = s * SKB;
        const bool past = k0 + SKB > K && k0 + tch * 16 >= K;
#pragma unroll
        for (int i = 0; i < MT; ++i) dma_b128_so(ar, lb + lta[i], past ? OOB8 : aoff[i], k0);
#pragma unroll
        for (int i = 0; i < 2; ++i) dma_b128_so(wr, lb + ltw[i], past ? OOB8 : woff[i], k0);
#pragma unroll
        for (int j = 0; j < NS; ++j)
            if (j > 0 || !wdup) dma_b32_so(rs[j], lb + ls[j], soff, 4 * s);
    };
    // DMA instruction i (< NL) of stage s into the buffer at lb: the A-tile rows, the W-tile rows,
    // then the scale dwords (the d_w side's duplicate skipped)
    auto dma_one = [&](int i, int s, uint32_t lb) __attribute__((always_inline)) {
        const int k0 = s * SKB;
        if (i < MT) {
            dma_b128_so(ar, lb + lta[i < MT ? i : 0], aoff[i < MT ? i : 0], k0);
        } else if (i < MT + 2) {
            dma_b128_so(wr, lb + ltw[i - MT < 2 ? i - MT : 0], woff[i - MT < 2 ? i - MT : 0], k0);
        } else {
            const int j = i - MT - 2 < NS ? i - MT - 2 : 0;
            if (j > 0 || !wdup) dma_b32_so(rs[j], lb + ls[j], soff, 4 * s);
        }
    };
    // wait until this wavefront's DMA of all but the last `later` stages issued has landed
    auto wait_dma = [&](int later) __attribute__((always_inline)) {
        if (wdup) {
            if (later >= 2) wait_vmcnt<2 * (NL - 1)>();
            else if (later == 1) wait_vmcnt<NL - 1>();
            else wait_vmcnt<0>();
        } else {
            if (later >= 2) wait_vmcnt<2 * NL>();
            else if (later == 1) wait_vmcnt<NL>();
            else wait_vmcnt<0>();
        }
    };

    const int wm = w & 1, wn = w >> 1;
    const int lr = lane & 31, g = lane >> 5;
    const bool lo = lane < 32;
    // per-lane LDS offsets inside a stage buffer (the same for all three)
    int ra_off[MT], rw_off[2], sda[MT], sdw[2];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const int r = WMR * wm + 32 * i + lr;
        ra_off[i] = r * SKB;
        sda[i] = r * 4;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int n = 64 * wn + 32 * i + lr;
        rw_off[i] = n * SKB;
        // lanes 32..63 carry k-slots 8..15 of the scale MFMA: a zero B operand there
        sdw[i] = lo ? (int)offsetof(St, wd) + n * 4 : (int)offsetof(St, zero);
    }
    v16f acc[MT][2];
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[a][c][i] = 0.0f;
    const v16i zi = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    const v16f zf = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

    // fragments of one block: the lane's 16 K bytes (chunk 2 bk + g) of its A and W rows, and
    // the scale MFMA's A operand (d_a of the block in k-slot 0 or 1 of dword 0, dword 1 zero)
    struct FragB {
        v4i a[MT], b[2];
        v2i da[MT];
    };
    auto load_blk = [&](const St& b, int bk, FragB& f) __attribute__((always_inline)) {
        const char* base = reinterpret_cast<const char*>(&b);
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            f.a[i] = *reinterpret_cast<const v4i*>(&b.A[ra_off[i] + slot8(ra_off[i] / SKB, 2 * bk + g) * 16]);
            f.da[i][0] = *reinterpret_cast<const int*>(base + (bk ? offsetof(St, adh) : offsetof(St, adl)) + sda[i]);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
            f.b[i] = *reinterpret_cast<const v4i*>(&b.W[rw_off[i] + slot8(rw_off[i] / SKB, 2 * bk + g) * 16]);
    };
    // scale MFMA B operands of a stage: d_w of both blocks in k-slots 0, 1 (lanes 0..31)
    auto load_dw = [&](const St& b, v2i (&dw)[2]) __attribute__((always_inline)) {
        const char* base = reinterpret_cast<const char*>(&b);
#pragma unroll
        for (int i = 0; i < 2; ++i) dw[i][0] = *reinterpret_cast<const int*>(base + sdw[i]);
    };
    // the isum MFMA's accumulator input, held in one register block for the whole loop
    v16i kbias = {kBias, kBias, kBias, kBias, kBias, kBias, kBias, kBias,
                  kBias, kBias, kBias, kBias, kBias, kBias, kBias, kBias};
    asm volatile("" : "+v"(kbias));
    // combine of elements i0 .. i0 + 7: acc += float(isum) * S
    auto apply_half = [&](v16f& a, const v16i& I, const v16f& S, int i0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = i0; i < i0 + 8; ++i) {
            // through a scalar: this clang's __builtin_bit_cast of an ext_vector element
            // expression reads element 0 whatever the index
            const int bits = I[i];
            a[i] = __builtin_fmaf(__builtin_bit_cast(float, bits) - kBiasF, S[i], a[i]);
        }
    };
    auto apply = [&](v16f& a, const v16i& I, const v16f& S) __attribute__((always_inline)) {
        apply_half(a, I, S, 0);
        apply_half(a, I, S, 8);
    };

    FragB f0, f1;
    v2i dw[2], dwn[2];
#pragma unroll
    for (int i = 0; i < MT; ++i) f0.da[i] = f1.da[i] = v2i{0, 0};
#pragma unroll
    for (int i = 0; i < 2; ++i) dw[i] = dwn[i] = v2i{0, 0};
    v16i PI[2];
    v16f PS[2];
    for (int i = 0; i < 2; ++i) {
        PI[i] = kbias;
        PS[i] = zf;
    }

    // prologue: stages 0..2 in flight, stage 0 published, its fragments in registers
    dma_stage(0, lbuf[0]);
    if (nstage > 1) dma_stage(1, lbuf[1]);
    if (nstage > 2) dma_stage(2, lbuf[2]);
    wait_dma(min(nstage - 1, 2));
    __syncthreads();  // also publishes the zero words
    // 64-row residual epilogue: the lane's eight residual float4 (two staging passes of four
    // rows, as the epilogue reads them) are loaded here, so their latency passes under the K
    // loop instead of being paid once per staging pass after it (32 VGPRs; the tile's rows
    // are in rtab since the barrier above; each element is read and later written by this
    // lane only, so an in-place residual is safe)
    constexpr bool PRE = EPI == MMQ_EPI_RESIDUAL && TM == 64;
    int rr_pre[PRE ? 8 : 1];
    v4f pv_pre[PRE ? 8 : 1];
    if (PRE) {
        const int nc = n0 + 64 * wn + 4 * (lane & 15);
#pragma unroll
        for (int q = 0; q < (PRE ? 8 : 1); ++q) {
            const int tr = WMR * wm + 16 * (q >> 2) + 4 * (q & 3) + (lane >> 4);  // pass q / 4, row group q % 4
            rr_pre[q] = nc < N ? rtab[tr] : -1;
            pv_pre[q] = rr_pre[q] >= 0 ? *reinterpret_cast<const v4f*>(&e.res[(int64_t)rr_pre[q] * N + nc])
                                       : v4f{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    load_blk(st0, 0, f0);
    load_blk(st0, 1, f1);
    load_dw(st0, dw);

    // units of one block of stage s: (mt, nt) = (0,0), (0,1), (1,0), (1,1); the previous unit's
    // combine (buffer p2) runs behind this unit's MFMAs (buffer u2)
    // s3 >= 0: unit q also issues DMA instructions [q NL / NU, (q + 1) NL / NU) of stage s3 into the
    // buffer at lb3, right after its isum MFMA, so the refill is spread over the block's units
    auto units = [&](int s, int bk, const FragB& f, const St& b, bool first, int s3 = -1, uint32_t lb3 = 0)
                     __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < NU; ++q) {
            const int mt = q >> 1, nt = q & 1;
            const int u2 = (bk * NU + q) & 1, p2 = u2 ^ 1;
            if (DOTS) {
                const v16i I = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[mt], f.b[nt], zi, 0, 0, 0);
                const int n = n0 + 64 * wn + 32 * nt + lr, blk = 2 * (so0 + s) + bk;
                if (blk < p.nbt) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int m = m0 + WMR * wm + 32 * mt + 8 * (i >> 2) + 4 * g + (i & 3);
                        if (m < M && n < N) p.dots[((int64_t)m * N + n) * p.nbt + blk] = I[i];
                    }
                }
                if (s3 >= 0) {  // this unit's share of the refill, as below
#pragma unroll
                    for (int i = q * NL / NU; i < (q + 1) * NL / NU; ++i) dma_one(i, s3, lb3);
                }
                continue;
            }
            if (Q41 && bk == 0) {
                // acc += s_a (x) m_w over the stage's two blocks, before the stage's block terms
                const int r = WMR * wm + 32 * mt + lr, n = 64 * wn + 32 * nt + lr;
                const v4i saf = {(int)b.as[Q41 ? r : 0], 0, 0, 0};
                const v4i mwf = {lo ? (int)b.wm[Q41 ? n : 0] : 0, 0, 0, 0};
                acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, saf),
                                                                     __builtin_bit_cast(v8h, mwf), acc[mt][nt], 0, 0, 0);
            }
            // the previous unit: (bk, q - 1), or block 0's last unit, or the previous stage's last;
            // its combine is split around this unit's second MFMA so neither MFMA issue waits
            const bool has_prev = !first || bk > 0 || q > 0;
            const int pq = (q + NU - 1) % NU;
            PI[u2] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[mt], f.b[nt], kbias, 0, 0, 0);
            if (s3 >= 0) {
#pragma unroll
                for (int i = q * NL / NU; i < (q + 1) * NL / NU; ++i) dma_one(i, s3, lb3);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (has_prev) apply_half(acc[pq >> 1][pq & 1], PI[p2], PS[p2], 0);
            __builtin_amdgcn_sched_barrier(0);
            PS[u2] = __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(v4h, f.da[mt]),
                                                         __builtin_bit_cast(v4h, dw[nt]), zf, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (has_prev) {
                apply_half(acc[pq >> 1][pq & 1], PI[p2], PS[p2], 8);
                asm volatile("" : "+v"(acc[pq >> 1][pq & 1]));
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // one stage: cur (at LDS address lcur) holds stage s, whose block-0 fragments are in
    // registers; nxt holds stage s + 1
    auto stage = [&](int s, St& cur, St& nxt, uint32_t lcur) __attribute__((always_inline)) {
        units(s, 0, f0, cur, s == 0);
        if (s + 1 < nstage) {
            wait_dma(min(nstage - 2 - s, 1));
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (s + 3 < nstage) dma_stage(s + 3, lcur);
            load_blk(nxt, 0, f0);
            load_dw(nxt, dwn);
        }
        units(s, 1, f1, cur, false);
        if (s + 1 < nstage) {
            load_blk(nxt, 1, f1);
#pragma unroll
            for (int i = 0; i < 2; ++i) dw[i] = dwn[i];
        }
    };
    // the steady state: 0 < s, stage s + 3 exists and has no chunk past K; its refill is spread
    // over block 1's units (the fragments of block 1 are already in registers)
    auto stage_full = [&](int s, St& cur, St& nxt, uint32_t lcur) __attribute__((always_inline)) {
        units(s, 0, f0, cur, false);
        wait_dma(1);  // stage s + 1 has landed (s + 2 may be in flight)
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        load_blk(nxt, 0, f0);
        load_dw(nxt, dwn);
        units(s, 1, f1, cur, false, s + 3, lcur);
        load_blk(nxt, 1, f1);
#pragma unroll
        for (int i = 0; i < 2; ++i) dw[i] = dwn[i];
    };
    // stages whose DMA reads no chunk past K: all, or all but a last half-filled stage
    const int nfull = K % SKB ? nstage - 1 : nstage;
    int s = 0;
    // the steady state from the second group of three stages: their refills s + 3 .. s + 5 are
    // full stages; the first group and the last (at most three) groups take the general form
    if (5 < nfull) {
        stage(0, st0, st1, lbuf[0]);
        stage(1, st1, st2, lbuf[1]);
        stage(2, st2, st0, lbuf[2]);
        for (s = 3; s + 5 < nfull; s += 3) {
            stage_full(s, st0, st1, lbuf[0]);
            stage_full(s + 1, st1, st2, lbuf[1]);
            stage_full(s + 2, st2, st0, lbuf[2]);
        }
    }
    for (; s < nstage; s += 3) {
        stage(s, st0, st1, lbuf[0]);
        if (s + 1 < nstage) stage(s + 1, st1, st2, lbuf[1]);
        if (s + 2 < nstage) stage(s + 2, st2, st0, lbuf[2]);
    }
    if (!DOTS) apply(acc[MT - 1][1], PI[1], PS[1]);  // the last unit (block 1, tile (MT - 1, 1))
    if (DOTS) return;
    // ---- epilogue: the wavefront's WMR x 64 region, RP rows at a time through LDS
    char* Dz = reinterpret_cast<char*>(p.D) + split * p.d_split;
    if (EPI == MMQ_EPI_STORE && !p.d_v4) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int m = m0 + WMR * wm + 32 * mt + 8 * (i >> 2) + 4 * g + (i & 3);
                    const int n = n0 + 64 * wn + 32 * nt + lr;
                    if (m < M && n < N) *reinterpret_cast<float*>(Dz + (int64_t)m * p.d_nb1 + (int64_t)n * 4) = acc[mt][nt][i];
                }
        return;
    }
    // staging rows of 64 floats (256 bytes, one line of the 64 4-byte LDS banks); rows with bit 2
    // set hold their columns rotated by 32, so a write pass (lanes 0..31 row R, lanes 32..63 row
    // R + 4) covers all 64 banks, and a read (16 lanes per row) sweeps one row
    constexpr int TP = 64;
    constexpr int RP = TM == 128 ? 32 : 16;  // rows per staging pass: two wavefronts per stage buffer
    constexpr int NP = 32 / RP;              // passes per 32-row m-tile
    static_assert(2 * RP * TP * 4 <= (int)sizeof(St), "epilogue staging exceeds a stage buffer");
    __syncthreads();  // every wavefront is done with the stage buffers
    float* stg = reinterpret_cast<float*>(w < 2 ? &st0 : &st1) + (w & 1) * RP * TP;
    const int c4 = lane & 15;                 // this lane's float4 column chunk
    const int nc = n0 + 64 * wn + 4 * c4;     // its first output column
    const bool cv = nc < N;                   // N % 4 == 0 on the float4 paths
    v4f bv = {0.0f, 0.0f, 0.0f, 0.0f};
    if (EPI != MMQ_EPI_STORE && cv) bv = *reinterpret_cast<const v4f*>(&e.bias[nc]);
    // the lane's qkv columns
    QkvLane ql{nullptr, 0, 0, false};
    if (EPI == MMQ_EPI_QKV) {
        const int E = e.nh * e.hd, which = nc / E, col = nc - which * E;
        ql.hh = col / e.hd;
        ql.d = col - ql.hh * e.hd;
        ql.dst = which == 0 ? e.q : which == 1 ? e.k : e.v;
        ql.rope = e.rope && which < 2;
    }
#pragma unroll
    for (int mp = 0; mp < MT * NP; ++mp) {
        const int mt = mp / NP, h = mp % NP;  // m-tile, and the RP-row pass inside it
        // element i of an m-tile is row 8 (i >> 2) + 4 g + (i & 3): pass h holds i in [16 h / NP, +16 / NP)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int i = 16 * h / NP; i < 16 * (h + 1) / NP; ++i)
                stg[(8 * (i >> 2) + 4 * g + (i & 3) - RP * h) * TP + ((32 * nt + lr + 32 * g) & 63)] = acc[mt][nt][i];
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wavefront's LDS writes are done
        __builtin_amdgcn_wave_barrier();
        // the pass's rows from the row table, and what their stores add, loaded before the stores
        // so the latency is paid once per group of rows instead of once per row: qkv RoPE factors
        // (the whole pass), residual rows (four at a time, which keeps 128-row tiles from
        // spilling; each element is read and written by this lane only, so in place is fine)
        constexpr int CH = EPI == MMQ_EPI_RESIDUAL ? 4 : RP / 4;
#pragma unroll
        for (int c0 = 0; c0 < RP / 4; c0 += CH) {
            int bwv[CH], tnv[CH], rrv[CH];
            v4f pvv[CH];
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const int tr = WMR * wm + 32 * mt + RP * h + (c0 + j) * 4 + (lane >> 4);  // row in the tile
                bwv[j] = tnv[j] = rrv[j] = 0;
                pvv[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
                if (EPI == MMQ_EPI_QKV) {
                    bwv[j] = rtab[tr];
                    tnv[j] = rtab[TM + tr];
                    if (ql.rope && cv && m0 + tr < M) pvv[j] = *reinterpret_cast<const v4f*>(&e.rope[(int64_t)tnv[j] * e.hd + ql.d]);
                }
                if (EPI == MMQ_EPI_RESIDUAL && PRE) {
                    rrv[j] = rr_pre[PRE ? (mp * 4 + c0 + j) & 7 : 0];
                    pvv[j] = pv_pre[PRE ? (mp * 4 + c0 + j) & 7 : 0];
                } else if (EPI == MMQ_EPI_RESIDUAL) {
                    rrv[j] = cv ? rtab[tr] : -1;
                    if (rrv[j] >= 0) pvv[j] = *reinterpret_cast<const v4f*>(&e.res[(int64_t)rrv[j] * N + nc]);
                }
            }
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const int r = (c0 + j) * 4 + (lane >> 4);
                const int m = m0 + WMR * wm + 32 * mt + RP * h + r;
                const v4f v = *reinterpret_cast<const v4f*>(&stg[r * TP + ((4 * c4 + 32 * ((r >> 2) & 1)) & 63)]);
                if (m >= M || !cv) continue;
                epi4<EPI>(Dz, p.d_nb1, e, N, m, nc, v, bv, rrv[j], ql, bwv[j], tnv[j], pvv[j]);
            }
        }
        __builtin_amdgcn_wave_barrier();  // the reads are done before the next pass overwrites
        __builtin_amdgcn_s_waitcnt(0xc07f);
    }
}

// ---- weight repack: ggml rows -> int8 quants [N][K] + fp16 d (and m) [N][dpw]
// One thread per 32-element block.  Q8_0 quants are copied, Q4_0 nibbles
// become q - 8, Q4_1 nibbles stay 0..15; the padding scale slot (dpw > nb) is
// zero.  src rows at src + r * nb1 for r < rows (2-D weights; batched
// weights arrive as consecutive row ranges).
template <int WT>
__global__ __launch_bounds__(256) void repack_weights_kernel(const uint8_t* __restrict__ src, int64_t nb1, int64_t rows,
                                                             int64_t nbr, int dpw, int8_t* __restrict__ q,
                                                             int64_t q_s1, _Float16* __restrict__ d,
                                                             _Float16* __restrict__ mm) {
    const int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gi >= rows * nbr) return;
    const int64_t r = gi / nbr, b = gi - r * nbr;
    constexpr int BS = WT == T_Q8_0 ? 34 : WT == T_Q4_0 ? 18 : 20;
    const uint8_t* blk = src + r * nb1 + b * BS;
    uint32_t out[8];
    if (WT == T_Q8_0) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
            out[j] = (uint32_t)blk[2 + 4 * j] | ((uint32_t)blk[3 + 4 * j] << 8) | ((uint32_t)blk[4 + 4 * j] << 16) |
                     ((uint32_t)blk[5 + 4 * j] << 24);
    } else {
        constexpr int HDR = WT == T_Q4_0 ? 2 : 4;
        uint32_t raw[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            raw[j] = (uint32_t)blk[HDR + 4 * j] | ((uint32_t)blk[HDR + 1 + 4 * j] << 8) |
                     ((uint32_t)blk[HDR + 2 + 4 * j] << 16) | ((uint32_t)blk[HDR + 3 + 4 * j] << 24);
        // element j < 16 is the low nibble of byte j, element j + 16 its high nibble
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t lo4 = raw[j] & 0x0f0f0f0fu, hi4 = (raw[j] >> 4) & 0x0f0f0f0fu;
            if (WT == T_Q4_0) {  // per byte (n | 0x80) - 8, then ^ 0x80: n - 8 without borrows
                lo4 = ((lo4 | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
                hi4 = ((hi4 | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
            }
            out[j] = lo4;
            out[4 + j] = hi4;
        }
    }
    uint4* qd = reinterpret_cast<uint4*>(q + r * q_s1 + b * QK);
    qd[0] = make_uint4(out[0], out[1], out[2], out[3]);
    qd[1] = make_uint4(out[4], out[5], out[6], out[7]);
    uint16_t dh, mh = 0;
    __builtin_memcpy(&dh, blk, 2);
    if (WT == T_Q4_1) __builtin_memcpy(&mh, blk + 2, 2);
    reinterpret_cast<uint16_t*>(d)[r * dpw + b] = dh;
    if (WT == T_Q4_1) reinterpret_cast<uint16_t*>(mm)[r * dpw + b] = mh;
    if (b == nbr - 1 && dpw > nbr) {
        reinterpret_cast<uint16_t*>(d)[r * dpw + nbr] = 0;
        if (WT == T_Q4_1) reinterpret_cast<uint16_t*>(mm)[r * dpw + nbr] = 0;
    }
}

size_t wrep_bytes(int type, int64_t N, int64_t K) {
    if (!(type == T_Q8_0 || type == T_Q4_0 || type == T_Q4_1) || K % QK != 0 || N < 0 || K < 0) return 0;
    const size_t dpw = (size_t)mmq_scale_pitch(K);
    const size_t q = ((size_t)N * (size_t)K + 255) & ~(size_t)255;
    const size_t d = ((size_t)N * dpw * 2 + 255) & ~(size_t)255;
    return q + d * (type == T_Q4_1 ? 2 : 1);
}

WRep wrep_view(int type, int64_t N, int64_t K, void* base) {
    const int dpw = (int)mmq_scale_pitch(K);
    const size_t q = ((size_t)N * (size_t)K + 255) & ~(size_t)255;
    const size_t db = ((size_t)N * dpw * 2 + 255) & ~(size_t)255;
    WRep r;
    r.type = type;
    r.q = static_cast<int8_t*>(base);
    r.q_s1 = K;
    r.d = reinterpret_cast<_Float16*>(static_cast<char*>(base) + q);
    r.m = type == T_Q4_1 ? reinterpret_cast<_Float16*>(static_cast<char*>(base) + q + db) : nullptr;
    r.dpw = dpw;
    r.N = N;
    r.K = K;
    return r;
}

hipError_t launch_repack_weights(const MatW& w, int64_t N, int64_t K, void* dst, WRep* out, hipStream_t st) {
    if (!(w.type == T_Q8_0 || w.type == T_Q4_0 || w.type == T_Q4_1) || K % QK != 0 || !dst)
        return hipErrorInvalidValue;
    const int64_t nbr = K / QK;
    const int dpw = (int)mmq_scale_pitch(K);
    const WRep r = wrep_view(w.type, N, K, dst);
    const int64_t n = N * nbr;
    if (n > 0) {
        const dim3 grid((unsigned)((n + 255) / 256));
        switch (w.type) {
            case T_Q8_0:
                repack_weights_kernel<T_Q8_0><<<grid, 256, 0, st>>>(w.data, w.nb1, N, nbr, dpw, r.q, r.q_s1, r.d, r.m);
                break;
            case T_Q4_0:
                repack_weights_kernel<T_Q4_0><<<grid, 256, 0, st>>>(w.data, w.nb1, N, nbr, dpw, r.q, r.q_s1, r.d, r.m);
                break;
            default:
                repack_weights_kernel<T_Q4_1><<<grid, 256, 0, st>>>(w.data, w.nb1, N, nbr, dpw, r.q, r.q_s1, r.d, r.m);
                break;
        }
    }
    *out = r;
    return hipGetLastError();
}

// Modelled time (us) of the int8 kernel, plus the split reduction, at tile height tm and K split
// ks. Two workgroups fit a CU. A grid of at most one workgroup per CU runs at the one-workgroup
// rate; beyond that the first round spreads over the CUs and later workgroups fill freed slots
// in pairs, the last round faster the emptier it is. The rates are fitted to the kernel times
// of 19 GEMM shapes of the ViT and Hiera encoders at every valid tile height and split (M 1024
// to 16384, N 192 to 4736, K 192 to 4736; 164 points, 7.7% rms error) on a 256-CU MI355X.
static double mmq8_cost(int64_t M, int64_t N, int64_t K, int tm, int ks, int cus) {
    const int64_t nst = (K / QK + 1) / 2, sps = (nst + ks - 1) / ks;
    const int64_t n = ((M + tm - 1) / tm) * ((N + B8N - 1) / B8N) * ks;
    const double pair = tm == B8M ? 1.472 : 0.734;  // us per stage, two workgroups per CU
    const double one = tm == B8M ? 0.719 : 0.363;   // us per stage, one workgroup per CU
    const double wg = 1.9;                          // prologue and epilogue of one workgroup
    double t;
    if (n <= cus) {
        t = sps * one + wg;
    } else {
        const int64_t slots = 2LL * cus, rounds = (n + slots - 1) / slots;
        const double fill = (double)(n - (rounds - 1) * slots) / slots;
        t = (rounds - 1) * (sps * pair + wg) + sps * pair * (0.622 + 0.378 * fill) + wg;
    }
    if (ks > 1) t += 3.3 + (double)(ks + 1) * M * N * 4 / 6.07e6;  // reduction: ks reads and one write of M x N f32
    return t;
}

// A split is valid when each of its ks K ranges holds at least two stages and none is empty.
static bool mmq8_split_valid(int64_t K, int ks) {
    const int64_t nst = (K / QK + 1) / 2, sps = (nst + ks - 1) / ks;
    return ks == 1 || (sps >= 2 && (ks - 1) * sps < nst);
}

int mmq8_tile_rows(int64_t M, int64_t N, int64_t K, int ks, int cus) {
    if (cus <= 0 || M <= 64) return B8M;
    // unsplit grids of at most 1.4 128-row tiles per CU take 64-row tiles, where the model
    // undervalues them (5184 x 1024 x 1024: 28.4 -> 27.3 us; 16384 x 192 x 768: 18.3 -> 17.2 us);
    // at 1.5 tiles per CU the 64-row grid's second round costs more (4096 x 1536 x 384: 16.6 -> 17.2 us)
    const int64_t t128 = ((M + B8M - 1) / B8M) * ((N + B8N - 1) / B8N);
    if (ks == 1 && 5 * t128 <= 7LL * cus) return 64;
    return mmq8_cost(M, N, K, 64, ks, cus) < mmq8_cost(M, N, K, B8M, ks, cus) ? 64 : B8M;
}

int mmq8_ksplit(int64_t M, int64_t N, int64_t K, int cus) {
    if (cus <= 0 || N % 4 != 0 || M <= 0 || K < QK) return 1;
    int best = 1;
    double best_cost = mmq8_cost(M, N, K, mmq8_tile_rows(M, N, K, 1, cus), 1, cus);
    for (int ks = 2; ks <= 16; ++ks) {
        if (!mmq8_split_valid(K, ks)) continue;
        const double c = mmq8_cost(M, N, K, mmq8_tile_rows(M, N, K, ks, cus), ks, cus);
        if (c < best_cost) {
            best_cost = c;
            best = ks;
        }
    }
    return best;
}

// ---- skinny K (K <= 128, large M: Hiera's stage-1 projections at 65536 tokens)
// The tiled kernel spends such a GEMM in prologue and epilogue: a 128-row tile has at most
// two K stages.  Here a wavefront owns 32 activation rows and NPW consecutive 32-column
// n-tiles: its A fragments (at most four blocks) and d_a stay in registers, the weight
// fragments and d_w of each n-tile come straight from global memory (the weights are a few
// KB and L2-resident), and each 32 x 32 tile leaves through the wavefront's own LDS staging
// as float4 row segments into the same epilogue as the tiled kernel (epi4).  No barriers and
// no LDS sharing between wavefronts, so small workgroups fill the CUs.  The arithmetic is
// the tiled kernel's, in its order: per stage (two blocks, the second a zero block past K
// for odd block counts) Q4_1's offset MFMA, then per block the isum MFMA, the d_a (x) d_w
// MFMA and acc = fma(float(isum), S, acc), so the results are bit-identical (float(isum)
// by conversion here, which frees the tiled kernel's bias registers; both are exact).
// npw n-tiles per wavefront, sized by the host for about four wavefronts per SIMD.
namespace {
constexpr int SK8_WPS = 4;   // wavefronts per SIMD the registers allow
}  // namespace

template <int WT, int EPI>
__global__ __launch_bounds__(256, SK8_WPS) void mmq8_skinny_kernel(const Mmq8Args p, const MmqEpi e, int npw) {
    constexpr bool Q41 = WT == T_Q4_1;
    __shared__ __attribute__((aligned(16))) float stg_all[4][32 * 32];
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lr = lane & 31, g = lane >> 5;
    const int M = p.M, N = p.N, ntn = (N + 31) / 32, ngr = (ntn + npw - 1) / npw;
    const int gw = blockIdx.x * 4 + w;  // this wavefront's task: (m-tile, group of n-tiles)
    if (gw >= ((M + 31) / 32) * ngr) return;
    const int mt = gw / ngr, j0 = (gw - mt * ngr) * npw, j1 = min(j0 + npw, ntn);
    const int m0 = 32 * mt, nstg = (p.K / QK + 1) / 2;  // stages of two blocks (at most 2)
    float* stg = stg_all[w];

    // A fragments (bytes 32 b + 16 g of row m0 + lr), d_a in k-slot b % 2 of the scale MFMA's
    // A operand, Q4_1's Q8_1 sums (dword s = blocks 2s, 2s + 1); blocks past K are zero
    const int ma = m0 + lr;
    const bool mv = ma < M;
    v4i af[4];
    v2i da[4];
    int sa[2] = {0, 0};
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const bool in = mv && b < 2 * nstg && 32 * b < p.K;
        af[b] = in ? *reinterpret_cast<const v4i*>(p.A + (int64_t)ma * p.a_s1 + 32 * b + 16 * g) : v4i{0, 0, 0, 0};
        const uint32_t dd = mv && b < 2 * nstg ? ((b & 1) ? p.Adh : p.Adl)[(int64_t)ma * p.nst + (b >> 1)] : 0u;
        da[b] = v2i{(int)dd, 0};
    }
    if (Q41) {
#pragma unroll
        for (int st = 0; st < 2; ++st)
            if (mv && st < nstg) sa[st] = (int)reinterpret_cast<const uint32_t*>(p.As)[(int64_t)ma * p.nst + st];
    }
    // the epilogue rows of this lane: 8 q + lane / 8 of the m-tile, q < 4; their residual
    // destinations or (qkv) windows and tokens, fixed for all n-tiles
    const int rl = lane >> 3, c4 = lane & 7;
    int rrv[4] = {-1, -1, -1, -1}, bwv[4] = {0, 0, 0, 0}, tnv[4] = {0, 0, 0, 0};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int m = m0 + 8 * q + rl;
        if (EPI == MMQ_EPI_RESIDUAL && m < M) rrv[q] = map_row32(e.map, rowmap_rcp(e.map), m);
        if (EPI == MMQ_EPI_QKV && m < M) bwv[q] = div_rcp(m, e.ntok, 1.0 / (double)e.ntok, tnv[q]);
    }
    const v16i zi = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    const v16f zf = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

    for (int j = j0; j < j1; ++j) {
        const int n = 32 * j + lr;
        const bool nv = n < N;
        // weight fragments, d_w (k-slot 0 or 1; lanes 32..63 carry k-slots 4..7 of the scale
        // MFMA and 8..15 of Q4_1's: zero) and Q4_1's minima of this n-tile
        v4i wf[4];
        v2i dw[2];
        int mw[2] = {0, 0};
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const bool in = nv && b < 2 * nstg && 32 * b < p.K;
            wf[b] = in ? *reinterpret_cast<const v4i*>(p.W + (int64_t)n * p.w_s1 + 32 * b + 16 * g) : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            const bool in = nv && g == 0 && st < nstg;
            dw[st] = v2i{in ? (int)reinterpret_cast<const uint32_t*>(p.Wd)[(int64_t)n * p.nst + st] : 0, 0};
            if (Q41) mw[st] = in ? (int)reinterpret_cast<const uint32_t*>(p.Wm)[(int64_t)n * p.nst + st] : 0;
        }
        v16f acc = zf;
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            if (st >= nstg) break;
            if (Q41) {
                const v4i saf = {sa[st], 0, 0, 0}, mwf = {mw[st], 0, 0, 0};
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, saf), __builtin_bit_cast(v8h, mwf),
                                                             acc, 0, 0, 0);
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int b = 2 * st + h;
                const v16i I = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[b], wf[b], zi, 0, 0, 0);
                const v16f S = __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(v4h, da[b]),
                                                                    __builtin_bit_cast(v4h, dw[st]), zf, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[i] = __builtin_fmaf((float)I[i], S[i], acc[i]);
                __builtin_amdgcn_sched_barrier(0);  // one block's MFMA results live at a time
            }
        }
        // the tile through this wavefront's staging: element i is row 8 (i >> 2) + 4 g + (i & 3)
#pragma unroll
        for (int i = 0; i < 16; ++i) stg[tile32_row(8 * (i >> 2) + 4 * g + (i & 3)) + lr] = acc[i];
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wavefront's LDS writes are done
        __builtin_amdgcn_wave_barrier();
        const int nc = 32 * j + 4 * c4;
        const bool cv = nc < N;  // N % 4 == 0
        v4f bv = {0.0f, 0.0f, 0.0f, 0.0f};
        if (EPI != MMQ_EPI_STORE && cv) bv = *reinterpret_cast<const v4f*>(&e.bias[nc]);
        QkvLane ql{nullptr, 0, 0, false};
        if (EPI == MMQ_EPI_QKV && cv) {
            const int E = e.nh * e.hd, which = nc / E, col = nc - which * E;
            ql.hh = col / e.hd;
            ql.d = col - ql.hh * e.hd;
            ql.dst = which == 0 ? e.q : which == 1 ? e.k : e.v;
            ql.rope = e.rope && which < 2;
        }
        // what the stores add (residual rows, RoPE factors), loaded before the stores
        v4f pvv[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            pvv[q] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            const int m = m0 + 8 * q + rl;
            if (EPI == MMQ_EPI_RESIDUAL && cv && rrv[q] >= 0)
                pvv[q] = *reinterpret_cast<const v4f*>(&e.res[(int64_t)rrv[q] * N + nc]);
            if (EPI == MMQ_EPI_QKV && ql.rope && cv && m < M)
                pvv[q] = *reinterpret_cast<const v4f*>(&e.rope[(int64_t)tnv[q] * e.hd + ql.d]);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int r = 8 * q + rl, m = m0 + r;
            const v4f v = *reinterpret_cast<const v4f*>(&stg[tile32_row(r) + 4 * c4]);
            if (m >= M || !cv) continue;
            epi4<EPI>(reinterpret_cast<char*>(p.D), p.d_nb1, e, N, m, nc, v, bv, rrv[q], ql, bwv[q], tnv[q], pvv[q]);
        }
        __builtin_amdgcn_wave_barrier();  // the reads are done before the next tile overwrites
        __builtin_amdgcn_s_waitcnt(0xc07f);
    }
}

// K <= 128 at M >= 4096, no split or inspection, float4 rows: the skinny kernel (true)
static bool launch8_skinny(const Mmq8Args& a, int wtype, const MmqEpi* e, int cus, hipStream_t st) {
    const int kind = e ? e->kind : MMQ_EPI_STORE;
    // as many wavefronts as the CUs hold at once
    const int64_t mtiles = (a.M + 31) / 32, ntn = (a.N + 31) / 32;
    const int64_t target = 4LL * SK8_WPS * (cus > 0 ? cus : 256);
    const int npw = (int)std::max<int64_t>(1, (mtiles * ntn + target - 1) / target);
    const int64_t waves = mtiles * ((ntn + npw - 1) / npw);
    const dim3 grid((unsigned)((waves + 3) / 4));
    MmqEpi none{};
    const MmqEpi& ee = e ? *e : none;
#define SK8(WT)                                                                                           \
    do {                                                                                                  \
        if (kind == MMQ_EPI_STORE) mmq8_skinny_kernel<WT, MMQ_EPI_STORE><<<grid, 256, 0, st>>>(a, none, npw);  \
        else if (kind == MMQ_EPI_RESIDUAL) mmq8_skinny_kernel<WT, MMQ_EPI_RESIDUAL><<<grid, 256, 0, st>>>(a, ee, npw); \
        else mmq8_skinny_kernel<WT, MMQ_EPI_QKV><<<grid, 256, 0, st>>>(a, ee, npw);                            \
    } while (0)
    switch (wtype) {
        case T_Q8_0: SK8(T_Q8_0); break;
        case T_Q4_0: SK8(T_Q4_0); break;
        default: SK8(T_Q4_1); break;
    }
#undef SK8
    return true;
}

template <int WT, int TM>
static void launch8_t(const Mmq8Args& a, const MmqEpi* e, hipStream_t st) {
    const int TT = a.tiles_m * a.tiles_n * a.ksplit;
    const dim3 grid((unsigned)(((TT + 7) / 8) * 8));
    MmqEpi none{};
    if (a.dots) mmq8_kernel<WT, MMQ_EPI_STORE, true, TM><<<grid, NT8, 0, st>>>(a, none);
    else if (a.ksplit > 1 || !e || e->kind == MMQ_EPI_STORE) mmq8_kernel<WT, MMQ_EPI_STORE, false, TM><<<grid, NT8, 0, st>>>(a, none);
    else if (e->kind == MMQ_EPI_RESIDUAL) mmq8_kernel<WT, MMQ_EPI_RESIDUAL, false, TM><<<grid, NT8, 0, st>>>(a, *e);
    else mmq8_kernel<WT, MMQ_EPI_QKV, false, TM><<<grid, NT8, 0, st>>>(a, *e);
}

bool mmq8_supported(const WRep& w, const ActI8& a) {
    return (w.type == T_Q8_0 || w.type == T_Q4_0 || w.type == T_Q4_1) && a.K == w.K && a.K % QK == 0 && a.K > 0 &&
           w.q_s1 % 16 == 0 && a.s1 % 16 == 0 && 2 * a.nst == mmq_scale_pitch(a.K) && w.dpw == 2 * a.nst &&
           (reinterpret_cast<uintptr_t>(w.q) & 15) == 0 && (reinterpret_cast<uintptr_t>(a.q) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(w.d) & 3) == 0 && (reinterpret_cast<uintptr_t>(a.dl) & 3) == 0 &&
           (reinterpret_cast<uintptr_t>(a.dh) & 3) == 0 &&
           (w.type != T_Q4_1 || (((reinterpret_cast<uintptr_t>(w.m) | reinterpret_cast<uintptr_t>(a.s)) & 3) == 0 &&
                                 w.m && a.s)) &&
           (int64_t)(a.M - 1) * a.s1 + a.K < OOB8 && (int64_t)(w.N - 1) * w.q_s1 + w.K < OOB8 &&
           4LL * a.M * a.nst < OOB8 && 4LL * w.N * a.nst < OOB8;
}

hipError_t launch_mmq8(const WRep& w, const ActI8& a, const MatD& d, const MmqEpi* epi, const MmqSplit& sp,
                       hipStream_t st, int32_t* dots) {
    if (!mmq8_supported(w, a)) return hipErrorInvalidValue;
    const int64_t N = w.N;
    Mmq8Args p;
    p.dots = dots;
    p.nbt = (int)(a.K / QK);
    p.A = static_cast<const int8_t*>(a.q);
    p.a_s1 = a.s1;
    p.Adl = a.dl;
    p.Adh = a.dh;
    p.As = static_cast<const _Float16*>(a.s);
    p.W = w.q;
    p.w_s1 = w.q_s1;
    p.Wd = w.d;
    p.Wm = w.m;
    p.D = d.data;
    p.d_nb1 = d.nb1;
    p.M = (int)a.M;
    p.N = (int)N;
    p.K = (int)a.K;
    p.nst = (int)a.nst;
    const bool split = sp.ks > 1 && !dots;
    const int TMv = dots ? B8M : mmq8_tile_rows(a.M, N, a.K, split ? sp.ks : 1, sp.cus);
    p.tiles_m = (int)((a.M + TMv - 1) / TMv);
    p.tiles_n = (int)((N + B8N - 1) / B8N);
    const int nstage = (int)((a.K / QK + 1) / 2);
    p.ksplit = split ? sp.ks : 1;
    p.sps = split ? (nstage + sp.ks - 1) / sp.ks : nstage;
    {
        // group height: the fewest L2 bytes for the workgroups an XCD runs at once (32 CUs x 2),
        // each reading one K range
        const double kr = (double)std::min<int64_t>(a.K, (int64_t)p.sps * SKB);
        const double at = TMv * kr, wt = B8N * kr;
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
    p.d_split = 0;
    if (split) {
        if (!sp.part || N % 4 != 0 || (int64_t)(sp.ks - 1) * p.sps >= nstage) return hipErrorInvalidValue;
        p.D = sp.part;
        p.d_nb1 = N * 4;
        p.d_split = a.M * N * 4;
    } else if (epi && epi->kind != MMQ_EPI_STORE) {
        // the fused epilogues split rows with div_rcp (rows below 2^30)
        if (N % 4 != 0 || !epi->bias || a.M >= ((int64_t)1 << 30)) return hipErrorInvalidValue;
    }
    p.d_v4 = N % 4 == 0 && p.d_nb1 % 16 == 0 && (reinterpret_cast<uintptr_t>(p.D) & 15) == 0;
    if (epi && epi->kind != MMQ_EPI_STORE && !split) p.d_v4 = 1;
    if (!split && !dots && (!epi || epi->kind == MMQ_EPI_STORE) && !d.data) return hipErrorInvalidValue;
    const LnArgs* ln = epi && epi->kind == MMQ_EPI_RESIDUAL ? epi->ln_next : nullptr;
    if (!split && !dots && sp.skinny && a.K <= 128 && a.M >= 4096 && N % 4 == 0 &&
        ((epi && epi->kind != MMQ_EPI_STORE) || p.d_v4)) {
        launch8_skinny(p, w.type, epi, sp.cus, st);
        const hipError_t e1 = hipGetLastError();
        if (e1 != hipSuccess) return e1;
        return ln ? launch_layer_norm(*ln, st) : hipSuccess;
    }
    switch (w.type * 2 + (TMv == 64 ? 1 : 0)) {
        case T_Q8_0 * 2: launch8_t<T_Q8_0, 128>(p, epi, st); break;
        case T_Q8_0 * 2 + 1: launch8_t<T_Q8_0, 64>(p, epi, st); break;
        case T_Q4_0 * 2: launch8_t<T_Q4_0, 128>(p, epi, st); break;
        case T_Q4_0 * 2 + 1: launch8_t<T_Q4_0, 64>(p, epi, st); break;
        case T_Q4_1 * 2: launch8_t<T_Q4_1, 128>(p, epi, st); break;
        default: launch8_t<T_Q4_1, 64>(p, epi, st); break;
    }
    hipError_t e0 = hipGetLastError();
    if (e0 != hipSuccess) return e0;
    if (split) {
        // a 1024-wide residual into its own rows: the reduction and the next LayerNorm in one pass
        if (ln && N == 1024 && sp.ks <= 4 && epi->map.kind == ROWMAP_IDENTITY && epi->res == epi->out &&
            ln->x == epi->out && ln->rows == a.M && !ln->add)
            return launch_reduce_residual_ln1024(sp.part, sp.ks, epi->bias, epi->out, *ln, st);
        e0 = launch_mmq_reduce(sp.part, sp.ks, (int)a.M, (int)N, reinterpret_cast<char*>(d.data), d.nb1, epi, st);
        if (e0 != hipSuccess) return e0;
    }
    return ln ? launch_layer_norm(*ln, st) : hipSuccess;
}

}  // namespace mi355
