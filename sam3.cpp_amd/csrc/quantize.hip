// Activation from_float kernels: F32 -> Q8_0 / Q8_1 / F16, bit-exact with
// ggml-cpu's quantize_row_q8_0 / q8_1 (x86 SIMD and scalar _ref variants)
// and ggml_cpu_fp32_to_fp16.
//
// Work split: 8 lanes per 32-element block, 4 elements per lane, so one
// wavefront quantizes 8 blocks.  The block's |x| max is reduced across its 8
// lanes with a butterfly, every lane derives d and id itself (IEEE-correct
// fp32 division), rounds its 4 values and writes 4 packed int8.
#include <cfloat>

#include "common.cuh"
#include "kernels.h"

namespace mi355 {

struct RowAddr {
    int64_t ne1, ne2;
    int64_t nb0, nb1, nb2, nb3;
    __device__ __forceinline__ const char* row(const char* base, int64_t r) const {
        const int64_t i1 = r % ne1;
        const int64_t i2 = (r / ne1) % ne2;
        const int64_t i3 = r / (ne1 * ne2);
        return base + i1 * nb1 + i2 * nb2 + i3 * nb3;
    }
};

__device__ __forceinline__ float ld_elem(const char* p, int type) {
    return type == T_F32 ? *reinterpret_cast<const float*>(p) : h2f(*reinterpret_cast<const uint16_t*>(p));
}

// Quantize one 32-block spread over 8 lanes.  Returns the 4 packed int8 of
// this lane, the fp16 d and (when wanted) the fp16 s; all lanes of the group
// get d and s.
template <bool REF>
__device__ __forceinline__ uint32_t q8_lanes(const float x[4], uint16_t& dh, float& d32, int& isum) {
    float amax = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
    amax = group_max<8>(amax);
    const float d = amax / 127.0f;
    float id;
    if (REF) id = d != 0.0f ? 1.0f / d : 0.0f;
    else id = amax != 0.0f ? 127.0f / amax : 0.0f;
    uint32_t packed = 0;
    int s = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float v = x[j] * id;
        const int q = (int)(REF ? roundf(v) : rintf(v));
        s += q;
        packed |= ((uint32_t)q & 0xffu) << (8 * j);
    }
    isum = group_sum_i<8>(s);
    dh = f2h(d);
    d32 = d;
    return packed;
}

template <int OUT, bool REF>  // OUT: T_Q8_0 or T_Q8_1 (ggml layout)
__global__ __launch_bounds__(256) void quantize_ggml_kernel(const char* __restrict__ src, int stype, RowAddr ra,
                                                            int64_t ne0, int64_t nblocks, uint8_t* __restrict__ dst) {
    const int64_t gt = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t g = gt >> 3;
    const int t = threadIdx.x & 7;
    const bool valid = g < nblocks;
    const int64_t nbpr = ne0 / QK;
    const int64_t r = valid ? g / nbpr : 0;
    const int64_t b = valid ? g % nbpr : 0;
    float x[4] = {0.f, 0.f, 0.f, 0.f};
    if (valid) {
        const char* rp = ra.row(src, r);
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = ld_elem(rp + (b * QK + 4 * t + j) * ra.nb0, stype);
    }
    uint16_t dh;
    float d32;
    int isum;
    const uint32_t packed = q8_lanes<REF>(x, dh, d32, isum);
    if (!valid) return;
    if (OUT == T_Q8_0) {
        uint8_t* blk = dst + (r * nbpr + b) * (int64_t)sizeof(blk_q8_0);
        uint16_t* q16 = reinterpret_cast<uint16_t*>(blk + 2 + 4 * t);  // 2-byte aligned
        q16[0] = (uint16_t)(packed & 0xffffu);
        q16[1] = (uint16_t)(packed >> 16);
        if (t == 0) *reinterpret_cast<uint16_t*>(blk) = dh;
    } else {
        uint8_t* blk = dst + (r * nbpr + b) * (int64_t)sizeof(blk_q8_1);
        *reinterpret_cast<uint32_t*>(blk + 4 + 4 * t) = packed;  // 36-byte blocks: 4-byte aligned
        if (t == 0) {
            reinterpret_cast<uint16_t*>(blk)[0] = dh;
            reinterpret_cast<uint16_t*>(blk)[1] = f2h(d32 * (float)isum);
        }
    }
}

// Weight quantizers quantize_row_q4_0_ref / quantize_row_q4_1_ref (what
// ggml_quantize_chunk runs when no importance matrix is given), 8 lanes per
// block as above, lane t holding elements 4t..4t+3.  The serial loops keep
// the FIRST element on equal comparisons (strict < / >), which decides the
// sign of Q4_0's d when +a and -a are both extreme and the sign of a zero
// Q4_1 min; the cross-lane reduction therefore breaks ties by element index.
// No multiply-add contraction: x*id + 8.5 and (x-min)*id + 0.5 round twice,
// as the unfused C expressions do.
template <int OUT>  // T_Q4_0 or T_Q4_1 (ggml layout)
__global__ __launch_bounds__(256) void quantize_q4_kernel(const char* __restrict__ src, int stype, RowAddr ra,
                                                          int64_t ne0, int64_t nblocks, uint8_t* __restrict__ dst) {
#pragma clang fp contract(off)
    const int64_t gt = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t g = gt >> 3;
    const int t = threadIdx.x & 7;
    const bool valid = g < nblocks;
    const int64_t nbpr = ne0 / QK;
    const int64_t r = valid ? g / nbpr : 0;
    const int64_t b = valid ? g % nbpr : 0;
    float x[4] = {0.f, 0.f, 0.f, 0.f};
    if (valid) {
        const char* rp = ra.row(src, r);
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = ld_elem(rp + (b * QK + 4 * t + j) * ra.nb0, stype);
    }
    float d, id, base, add;
    uint16_t dh, mh = 0;
    if (OUT == T_Q4_0) {
        // max = the x of largest |x|
        float amax = 0.0f, mx = 0.0f;
        int ix = QK;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (amax < fabsf(x[j])) {
                amax = fabsf(x[j]);
                mx = x[j];
                ix = 4 * t + j;
            }
#pragma unroll
        for (int o = 4; o > 0; o >>= 1) {
            const float oa = __shfl_xor(amax, o, 8), om = __shfl_xor(mx, o, 8);
            const int oi = __shfl_xor(ix, o, 8);
            if (oa > amax || (oa == amax && oi < ix)) {
                amax = oa;
                mx = om;
                ix = oi;
            }
        }
        d = mx / -8.0f;
        base = 0.0f;
        add = 8.5f;
    } else {
        float mn = FLT_MAX, mx = -FLT_MAX;
        int imn = QK, imx = QK;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (x[j] < mn) {
                mn = x[j];
                imn = 4 * t + j;
            }
            if (x[j] > mx) {
                mx = x[j];
                imx = 4 * t + j;
            }
        }
#pragma unroll
        for (int o = 4; o > 0; o >>= 1) {
            const float omn = __shfl_xor(mn, o, 8), omx = __shfl_xor(mx, o, 8);
            const int oin = __shfl_xor(imn, o, 8), oix = __shfl_xor(imx, o, 8);
            if (omn < mn || (omn == mn && oin < imn)) {
                mn = omn;
                imn = oin;
            }
            if (omx > mx || (omx == mx && oix < imx)) {
                mx = omx;
                imx = oix;
            }
        }
        d = (mx - mn) / 15.0f;
        base = mn;
        add = 0.5f;
        mh = f2h(mn);
    }
    id = d != 0.0f ? 1.0f / d : 0.0f;
    dh = f2h(d);
    uint32_t nib = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float v = (OUT == T_Q4_0 ? x[j] : x[j] - base) * id;
        const int q = min((int)(v + add), 15);
        nib |= (uint32_t)q << (8 * j);
    }
    // element j's nibble is low, element j+16's high: lanes 0..3 take lanes 4..7's values
    const uint32_t hi = __shfl_xor(nib, 4, 8);
    if (!valid || t >= 4) return;
    const uint32_t bytes = nib | (hi << 4);
    constexpr int BB = OUT == T_Q4_0 ? (int)sizeof(blk_q4_0) : (int)sizeof(blk_q4_1);
    constexpr int QS = OUT == T_Q4_0 ? 2 : 4;
    uint8_t* blk = dst + (r * nbpr + b) * (int64_t)BB;
    uint16_t* q16 = reinterpret_cast<uint16_t*>(blk + QS + 4 * t);  // 2-byte aligned
    q16[0] = (uint16_t)(bytes & 0xffffu);
    q16[1] = (uint16_t)(bytes >> 16);
    if (t == 0) {
        reinterpret_cast<uint16_t*>(blk)[0] = dh;
        if (OUT == T_Q4_1) reinterpret_cast<uint16_t*>(blk)[1] = mh;
    }
}

// Same arithmetic (x86 variant) into the MFMA operand layout, one thread per
// 32-element block: quants as fp16 integers (exact) [rows][K], scale and Q8_1
// sum as the fp16 values ggml stores, [rows][dp] (dp = block count rounded up
// to even; the padding slot is written as zero).  A wavefront covers 64
// consecutive blocks of the flattened [rows][nb] grid.  Flat 16-byte aligned F32
// rows take quantize_chunks_kernel (below) instead; this kernel serves strided,
// unaligned and F16 sources and quant row pitches wider than K.
// I8: quants as int8 [rows][q_s1 bytes] (the int8-MFMA operand) instead of fp16 [rows][ne0].
// rnb = 1 / (blocks per row) when the rows lie at a fixed pitch nb1 and nblocks plus a row's
// blocks stay below 2^31: row and block then come from div_rcp, not from 64-bit divisions
// (whose dependent chain delayed every thread's first load); else rnb = 0.
template <bool WITH_SUM, bool I8 = false>
__global__ __launch_bounds__(256) void quantize_mmq_kernel(const char* __restrict__ src, int stype, RowAddr ra,
                                                           int64_t ne0, int64_t nblocks, int64_t dp,
                                                           uint16_t* __restrict__ qout, uint16_t* __restrict__ dout,
                                                           uint16_t* __restrict__ sout, double rnb, int64_t q_s1 = 0) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= nblocks) return;
    const int64_t nbpr = ne0 / QK;
    int64_t r, b;
    const char* rp;
    if (rnb != 0.0) {
        int bi;
        const int ri = div_rcp((int)g, (int)nbpr, rnb, bi);
        r = ri;
        b = bi;
        rp = src + (int64_t)ri * ra.nb1;
    } else {
        r = g / nbpr;
        b = g - r * nbpr;
        rp = ra.row(src, r);
    }
    float x[QK];
    if (stype == T_F32 && ra.nb0 == 4 && ((reinterpret_cast<uintptr_t>(rp) & 15) == 0)) {
        const v4f* p4 = reinterpret_cast<const v4f*>(rp + b * QK * 4);
#pragma unroll
        for (int j = 0; j < QK / 4; ++j) {
            const v4f v = p4[j];
            x[4 * j] = v[0];
            x[4 * j + 1] = v[1];
            x[4 * j + 2] = v[2];
            x[4 * j + 3] = v[3];
        }
    } else {
#pragma unroll
        for (int j = 0; j < QK; ++j) x[j] = ld_elem(rp + (b * QK + j) * ra.nb0, stype);
    }
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < QK; ++j) amax = fmaxf(amax, fabsf(x[j]));
    const float d = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    int isum = 0;
    if (I8) {
        uint32_t bq[QK / 4];
#pragma unroll
        for (int j = 0; j < QK / 4; ++j) {
            const int q0 = (int)rintf(x[4 * j] * id), q1 = (int)rintf(x[4 * j + 1] * id);
            const int q2 = (int)rintf(x[4 * j + 2] * id), q3 = (int)rintf(x[4 * j + 3] * id);
            isum += q0 + q1 + q2 + q3;
            bq[j] = (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) | ((uint32_t)(q2 & 0xff) << 16) |
                    ((uint32_t)(q3 & 0xff) << 24);
        }
        uint4* qd = reinterpret_cast<uint4*>(reinterpret_cast<int8_t*>(qout) + r * q_s1 + b * QK);
        qd[0] = make_uint4(bq[0], bq[1], bq[2], bq[3]);
        qd[1] = make_uint4(bq[4], bq[5], bq[6], bq[7]);
    } else {
        uint32_t hq[QK / 2];
#pragma unroll
        for (int j = 0; j < QK / 2; ++j) {
            const int q0 = (int)rintf(x[2 * j] * id), q1 = (int)rintf(x[2 * j + 1] * id);
            isum += q0 + q1;
            hq[j] = (uint32_t)f2h((float)q0) | ((uint32_t)f2h((float)q1) << 16);
        }
        uint4* qd = reinterpret_cast<uint4*>(qout + r * ne0 + b * QK);
#pragma unroll
        for (int j = 0; j < QK / 8; ++j) qd[j] = make_uint4(hq[4 * j], hq[4 * j + 1], hq[4 * j + 2], hq[4 * j + 3]);
    }
    if (I8) {
        // scales as the int8 kernel's scale-MFMA operands: dword [r][b / 2] of dl holds d of an
        // even block in its low half, of dh d of an odd block in its high half (dout = dl,
        // dh = dl + rows * nst); a missing odd block (odd count) leaves a zero dword in dh
        const int64_t nst = dp / 2, rows = nblocks / nbpr;
        uint32_t* dl = reinterpret_cast<uint32_t*>(dout);
        uint32_t* dh = dl + rows * nst;
        if ((b & 1) == 0) dl[r * nst + b / 2] = (uint32_t)f2h(d);
        else dh[r * nst + b / 2] = (uint32_t)f2h(d) << 16;
        if (b == nbpr - 1 && (nbpr & 1)) dh[r * nst + b / 2] = 0;
    } else {
        dout[r * dp + b] = f2h(d);
    }
    if (WITH_SUM) sout[r * dp + b] = f2h(d * (float)isum);
    if (b == nbpr - 1 && dp > nbpr) {
        if (!I8) dout[r * dp + nbpr] = 0;
        if (WITH_SUM) sout[r * dp + nbpr] = 0;
    }
}

// Flat F32 rows (row r at src + r * nb1, elements contiguous, base and nb1 16-byte aligned) ->
// the MUL_MAT operand (o: the int8 or fp16-quant layout, quant rows of K = ne0), the same
// from_float as quantize_mmq_kernel.  The grid walks 4-value chunks of the flattened
// [rows][K / 4] grid: a workgroup owns CH_U * 256 consecutive chunks, thread t chunks
// base + 256 u + t, so every load and store instruction of a wavefront covers 1 KB (loads) or
// 256 / 512 bytes (quants) of consecutive addresses, and all CH_U 16-byte loads are issued
// before the first block is reduced.  The 8 lanes of a 32-value block (consecutive chunks,
// consecutive lanes) reduce it by DPP (act_store_chunk); K % 32 == 0 makes the bounds test
// uniform over each such group.
// MODE (ACT_Q8, ACT_Q8S, ACT_I8 or ACT_I8S) replaces o.mode, so the operand layout is fixed
// at compile time.  DENSE: rows back to back (nb1 = 4 K) and an even block count per row
// (dp = K / 32, no padding slot), so chunk i's values, quants and block i / 8's scale slots
// all follow from i without a division.
constexpr int CH_U = 4;
template <int MODE>
__device__ __forceinline__ void dense_chunk(const ActOut& o, int i, v4f x) {
    float amax = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
    amax = group_max<8>(amax);
    const float d = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    const int q0 = (int)rintf(x[0] * id), q1 = (int)rintf(x[1] * id);
    const int q2 = (int)rintf(x[2] * id), q3 = (int)rintf(x[3] * id);
    int isum = 0;
    if (act_has_sums(MODE)) isum = group_sum_i<8>(q0 + q1 + q2 + q3);
    const int g = i >> 3;  // the block: row * (K / 32) + block in the row
    if ((i & 7) == 0) {
        if (MODE >= ACT_I8) {  // dword g / 2 of dl (even g: low half) or dh (odd g: high half)
            if ((g & 1) == 0) reinterpret_cast<uint32_t*>(o.d)[g >> 1] = (uint32_t)f2h(d);
            else o.dh[g >> 1] = (uint32_t)f2h(d) << 16;
        } else {
            o.d[g] = f2h(d);
        }
        if (act_has_sums(MODE)) o.s[g] = f2h(d * (float)isum);
    }
    if (MODE >= ACT_I8) {
        reinterpret_cast<uint32_t*>(o.q)[i] = (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) |
                                              ((uint32_t)(q2 & 0xff) << 16) | ((uint32_t)(q3 & 0xff) << 24);
    } else {
        const uint32_t h0 = (uint32_t)f2h((float)q0) | ((uint32_t)f2h((float)q1) << 16);
        const uint32_t h1 = (uint32_t)f2h((float)q2) | ((uint32_t)f2h((float)q3) << 16);
        reinterpret_cast<uint2*>(o.q)[i] = make_uint2(h0, h1);
    }
}
// Rows back to back, two lanes per 32-value block: lane 2j + e holds values 16 e .. 16 e + 15
// of its block (half i of the flattened grid, 64 bytes: four 16-byte loads), the pair's max by
// one DPP swap (act_store_half16's arithmetic), 16 quant bytes (or 16 halves) per lane.  A
// block's division pair is done by two lanes instead of eight, a quarter of the VALU work of
// the chunk form per byte.  DENSE (an even block count per row, no padding slot): the scale
// slots follow from the flat block index; otherwise the row and block come from div_rcp
// (rnb = 1 / blocks per row) and act_store_scale writes the slots and the padding.
constexpr int HF_U = 2;
template <int MODE, bool DENSE>
__device__ __forceinline__ void dense_half(const ActOut& o, int i, const v4f (&xv)[4], int nbpr, double rnb, int64_t K) {
    float x[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) x[j] = xv[j >> 2][j & 3];
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) amax = fmaxf(amax, fabsf(x[j]));
    amax = fmaxf(amax, lane_swap_f<1>(amax));  // quad_perm [1, 0, 3, 2]: the block's other half
    const float d = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    int q[16], isum = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        q[j] = (int)rintf(x[j] * id);
        isum += q[j];
    }
    if (act_has_sums(MODE)) isum += lane_swap<1>(isum);
    const int g = i >> 1;  // the block: row * (K / 32) + block in the row
    if (!DENSE && (i & 1) == 0) {
        int b;
        const int r = div_rcp(g, nbpr, rnb, b);
        act_store_scale(o, r, K, b, d, isum);
    } else if ((i & 1) == 0) {
        if (MODE >= ACT_I8) {  // dword g / 2 of dl (even g: low half) or dh (odd g: high half)
            if ((g & 1) == 0) reinterpret_cast<uint32_t*>(o.d)[g >> 1] = (uint32_t)f2h(d);
            else o.dh[g >> 1] = (uint32_t)f2h(d) << 16;
        } else {
            o.d[g] = f2h(d);
        }
        if (act_has_sums(MODE)) o.s[g] = f2h(d * (float)isum);
    }
    if (MODE >= ACT_I8) {
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            w[j] = (uint32_t)(q[4 * j] & 0xff) | ((uint32_t)(q[4 * j + 1] & 0xff) << 8) |
                   ((uint32_t)(q[4 * j + 2] & 0xff) << 16) | ((uint32_t)(q[4 * j + 3] & 0xff) << 24);
        reinterpret_cast<uint4*>(o.q)[i] = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
        uint32_t hw[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) hw[j] = (uint32_t)f2h((float)q[2 * j]) | ((uint32_t)f2h((float)q[2 * j + 1]) << 16);
        uint4* dst = reinterpret_cast<uint4*>(o.q) + 2 * (int64_t)i;
        dst[0] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        dst[1] = make_uint4(hw[4], hw[5], hw[6], hw[7]);
    }
}
// thread t of workgroup b: halves (b HF_U + u) 256 + t, u < HF_U (nh halves, nh even)
template <int MODE, bool DENSE>
__global__ __launch_bounds__(256) void quantize_halves_kernel(const char* __restrict__ src, int nh, ActOut o, int nbpr,
                                                              double rnb, int64_t K) {
    o.mode = MODE;
    const int i0 = blockIdx.x * (256 * HF_U) + threadIdx.x;
    v4f x[HF_U][4];
#pragma unroll
    for (int u = 0; u < HF_U; ++u) {
        const v4f* p = reinterpret_cast<const v4f*>(src + (int64_t)min(i0 + 256 * u, nh - 1) * 64);
#pragma unroll
        for (int j = 0; j < 4; ++j) x[u][j] = p[j];
    }
#pragma unroll
    for (int u = 0; u < HF_U; ++u) {
        if (i0 + 256 * u >= nh) break;
        dense_half<MODE, DENSE>(o, i0 + 256 * u, x[u], nbpr, rnb, K);
    }
}
template <int MODE, bool DENSE>
__global__ __launch_bounds__(256) void quantize_chunks_kernel(const char* __restrict__ src, int64_t nb1, int cpr,
                                                              int nch, double rcpr, ActOut o, int64_t K) {
    o.mode = MODE;
    const int i0 = blockIdx.x * (256 * CH_U) + threadIdx.x;
    v4f x[CH_U];
    int row[CH_U], c[CH_U];
#pragma unroll
    for (int u = 0; u < CH_U; ++u) {
        const int i = min(i0 + 256 * u, nch - 1);  // past the end: a valid chunk, loaded and dropped
        if (DENSE) {
            x[u] = *reinterpret_cast<const v4f*>(src + (int64_t)i * 16);
        } else {
            row[u] = div_rcp(i, cpr, rcpr, c[u]);
            x[u] = *reinterpret_cast<const v4f*>(src + (int64_t)row[u] * nb1 + (int64_t)c[u] * 16);
        }
    }
#pragma unroll
    for (int u = 0; u < CH_U; ++u) {
        const int i = i0 + 256 * u;
        if (i >= nch) break;
        if (DENSE) dense_chunk<MODE>(o, i, x[u]);
        else act_store_chunk(o, row[u], K, c[u], x[u]);
    }
}
// Flat F32 rows (as above) -> contiguous F16 rows of ne0 halves (pitch == ne0, ne0 % 4 == 0):
// chunk i (4 values) of the flattened grid to halves 4i .. 4i + 3, CH_U chunks per thread
// at a stride of 256 chunks, so a wavefront's loads cover 1 KB and its stores 512 bytes of
// consecutive addresses, all loads issued before the first conversion.
__global__ __launch_bounds__(256) void convert_f16_flat_kernel(const char* __restrict__ src, int64_t nb1, int cpr,
                                                               int nch, double rcpr, uint16_t* __restrict__ dst) {
    const int i0 = blockIdx.x * (256 * CH_U) + threadIdx.x;
    v4f x[CH_U];
#pragma unroll
    for (int u = 0; u < CH_U; ++u) {
        int k;
        const int r = div_rcp(min(i0 + 256 * u, nch - 1), cpr, rcpr, k);
        x[u] = *reinterpret_cast<const v4f*>(src + (int64_t)r * nb1 + (int64_t)k * 16);
    }
#pragma unroll
    for (int u = 0; u < CH_U; ++u) {
        const int i = i0 + 256 * u;
        if (i >= nch) break;
        const uint32_t h0 = (uint32_t)f2h(x[u][0]) | ((uint32_t)f2h(x[u][1]) << 16);
        const uint32_t h1 = (uint32_t)f2h(x[u][2]) | ((uint32_t)f2h(x[u][3]) << 16);
        *reinterpret_cast<uint2*>(dst + (int64_t)i * 4) = make_uint2(h0, h1);
    }
}

// dst rows of `pitch` halves; columns ne0..pitch are zero
__global__ __launch_bounds__(256) void convert_f16_kernel(const char* __restrict__ src, int stype, RowAddr ra,
                                                          int64_t ne0, int64_t pitch, int64_t n,
                                                          uint16_t* __restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int64_t r = i / pitch, k = i % pitch;
    if (k >= ne0) {
        dst[i] = 0;
        return;
    }
    const char* p = ra.row(src, r) + k * ra.nb0;
    dst[i] = stype == T_F32 ? f2h(*reinterpret_cast<const float*>(p)) : *reinterpret_cast<const uint16_t*>(p);
}

// 1 / (blocks per row) for quantize_mmq_kernel's fast indexing, or 0 where it does not apply
static double blocks_rcp(const SrcView& s, int64_t nblocks) {
    const int64_t nbpr = s.ne[0] / QK;
    const bool flat = s.ne[2] * s.ne[3] == 1 || (s.nb[2] == s.ne[1] * s.nb[1] && (s.ne[3] == 1 || s.nb[3] == s.ne[2] * s.nb[2]));
    return flat && nbpr > 0 && nblocks + nbpr < ((int64_t)1 << 31) ? 1.0 / (double)nbpr : 0.0;
}

// F32 rows at one pitch nb[1] (the batch dims folded in), elements contiguous, base and pitch
// 16-byte aligned, and n units (blocks or chunks) plus a row's units below 2^31: the layout
// convert_f16_flat_kernel takes
static bool flat_f32(const SrcView& s, int64_t n) {
    const bool flat = s.ne[2] * s.ne[3] == 1 || (s.nb[2] == s.ne[1] * s.nb[1] && (s.ne[3] == 1 || s.nb[3] == s.ne[2] * s.nb[2]));
    return s.type == T_F32 && s.nb[0] == 4 && flat && s.ne[0] >= QK && ((reinterpret_cast<uintptr_t>(s.data) | (uintptr_t)s.nb[1]) & 15) == 0 &&
           n + s.ne[0] < ((int64_t)1 << 31) && s.ne[1] * s.ne[2] * s.ne[3] * s.nb[1] < ((int64_t)1 << 40);
}

// the chunk kernels' layout: flat_f32 rows, n chunks of 4 values, and the last workgroup's
// chunk indices below 2^31
static bool chunk_path(const SrcView& s, int64_t n) {
    return flat_f32(s, n) && n + 256 * CH_U < ((int64_t)1 << 31);
}
static dim3 chunk_grid(int64_t n) { return dim3((unsigned)((n + 256 * CH_U - 1) / (256 * CH_U))); }
// the chunk kernel for the operand mode and layout
template <int MODE>
static void launch_chunks(const SrcView& src, const ActOut& o, int64_t nch, hipStream_t st) {
    const int64_t K = src.ne[0], cpr = K / 4;
    if (src.nb[1] == 4 * K) {  // rows back to back: the two-lane form
        const int64_t nh = nch / 4, nbpr = K / 32;
        const dim3 grid((unsigned)((nh + 256 * HF_U - 1) / (256 * HF_U)));
        if (K % 64 == 0 && o.dp == K / 32)
            quantize_halves_kernel<MODE, true><<<grid, 256, 0, st>>>(src.data, (int)nh, o, (int)nbpr, 0.0, K);
        else
            quantize_halves_kernel<MODE, false><<<grid, 256, 0, st>>>(src.data, (int)nh, o, (int)nbpr,
                                                                      1.0 / (double)nbpr, K);
        return;
    }
    quantize_chunks_kernel<MODE, false><<<chunk_grid(nch), 256, 0, st>>>(src.data, src.nb[1], (int)cpr, (int)nch,
                                                                         1.0 / (double)cpr, o, K);
}


static RowAddr row_addr(const SrcView& s) {
    RowAddr ra;
    ra.ne1 = s.ne[1];
    ra.ne2 = s.ne[2];
    ra.nb0 = s.nb[0];
    ra.nb1 = s.nb[1];
    ra.nb2 = s.nb[2];
    ra.nb3 = s.nb[3];
    return ra;
}

hipError_t launch_quantize_ggml(const SrcView& src, int type, bool ref_variant, void* dst, hipStream_t st) {
    const int64_t rows = src.ne[1] * src.ne[2] * src.ne[3];
    if (type == T_F16) return launch_convert_f16(src, static_cast<uint16_t*>(dst), src.ne[0], st);
    const int64_t nblocks = rows * (src.ne[0] / QK);
    if (nblocks == 0) return hipSuccess;
    const dim3 grid((unsigned)((nblocks * 8 + 255) / 256));
    const RowAddr ra = row_addr(src);
    uint8_t* out = static_cast<uint8_t*>(dst);
    if (type == T_Q4_0 || type == T_Q4_1) {  // one (_ref) quantizer each
        if (type == T_Q4_0)
            quantize_q4_kernel<T_Q4_0><<<grid, 256, 0, st>>>(src.data, src.type, ra, src.ne[0], nblocks, out);
        else
            quantize_q4_kernel<T_Q4_1><<<grid, 256, 0, st>>>(src.data, src.type, ra, src.ne[0], nblocks, out);
        return hipGetLastError();
    }
    if (type == T_Q8_0 && !ref_variant)
        quantize_ggml_kernel<T_Q8_0, false><<<grid, 256, 0, st>>>(src.data, src.type, ra, src.ne[0], nblocks, out);
    else if (type == T_Q8_0)
        quantize_ggml_kernel<T_Q8_0, true><<<grid, 256, 0, st>>>(src.data, src.type, ra, src.ne[0], nblocks, out);
    else if (!ref_variant)
        quantize_ggml_kernel<T_Q8_1, false><<<grid, 256, 0, st>>>(src.data, src.type, ra, src.ne[0], nblocks, out);
    else
        quantize_ggml_kernel<T_Q8_1, true><<<grid, 256, 0, st>>>(src.data, src.type, ra, src.ne[0], nblocks, out);
    return hipGetLastError();
}

hipError_t launch_quantize_mmq(const SrcView& src, bool with_sum, int64_t dp, uint16_t* q, uint16_t* d, uint16_t* s,
                               hipStream_t st) {
    const int64_t rows = src.ne[1] * src.ne[2] * src.ne[3];
    const int64_t nblocks = rows * (src.ne[0] / QK);
    if (nblocks == 0) return hipSuccess;
    if (chunk_path(src, nblocks * 8)) {
        const ActOut o{with_sum ? ACT_Q8S : ACT_Q8, nullptr, q, d, s, dp};
        if (with_sum) launch_chunks<ACT_Q8S>(src, o, nblocks * 8, st);
        else launch_chunks<ACT_Q8>(src, o, nblocks * 8, st);
        return hipGetLastError();
    }
    const dim3 grid((unsigned)((nblocks + 255) / 256));
    const RowAddr ra = row_addr(src);
    if (with_sum)
        quantize_mmq_kernel<true><<<grid, 256, 0, st>>>(src.data, src.type, ra, src.ne[0], nblocks, dp, q, d, s,
                                                        blocks_rcp(src, nblocks));
    else
        quantize_mmq_kernel<false><<<grid, 256, 0, st>>>(src.data, src.type, ra, src.ne[0], nblocks, dp, q, d, s,
                                                         blocks_rcp(src, nblocks));
    return hipGetLastError();
}

hipError_t launch_quantize_mmq_i8(const SrcView& src, bool with_sum, int64_t s1, int64_t dp, int8_t* q, uint16_t* d,
                                  uint16_t* s, hipStream_t st) {
    const int64_t rows = src.ne[1] * src.ne[2] * src.ne[3];
    const int64_t nblocks = rows * (src.ne[0] / QK);
    if (nblocks == 0) return hipSuccess;
    if (s1 < src.ne[0] || s1 % 16 != 0) return hipErrorInvalidValue;
    uint16_t* qq = reinterpret_cast<uint16_t*>(q);
    if (s1 == src.ne[0] && chunk_path(src, nblocks * 8)) {
        uint32_t* dl = reinterpret_cast<uint32_t*>(d);
        const ActOut o{with_sum ? ACT_I8S : ACT_I8, nullptr, qq, d, s, dp, dl + rows * (dp / 2)};
        if (with_sum) launch_chunks<ACT_I8S>(src, o, nblocks * 8, st);
        else launch_chunks<ACT_I8>(src, o, nblocks * 8, st);
        return hipGetLastError();
    }
    const dim3 grid((unsigned)((nblocks + 255) / 256));
    const RowAddr ra = row_addr(src);
    if (with_sum)
        quantize_mmq_kernel<true, true><<<grid, 256, 0, st>>>(src.data, src.type, ra, src.ne[0], nblocks, dp, qq, d, s,
                                                              blocks_rcp(src, nblocks), s1);
    else
        quantize_mmq_kernel<false, true><<<grid, 256, 0, st>>>(src.data, src.type, ra, src.ne[0], nblocks, dp, qq, d, s,
                                                               blocks_rcp(src, nblocks), s1);
    return hipGetLastError();
}

hipError_t launch_convert_f16(const SrcView& src, uint16_t* dst, int64_t pitch, hipStream_t st) {
    if (pitch < src.ne[0]) return hipErrorInvalidValue;
    const int64_t n = pitch * src.ne[1] * src.ne[2] * src.ne[3];
    if (n == 0) return hipSuccess;
    if (pitch == src.ne[0] && src.ne[0] % 4 == 0 && chunk_path(src, n / 4) && (reinterpret_cast<uintptr_t>(dst) & 7) == 0) {
        const int64_t cpr = src.ne[0] / 4, nch = n / 4;
        convert_f16_flat_kernel<<<chunk_grid(nch), 256, 0, st>>>(src.data, src.nb[1], (int)cpr, (int)nch,
                                                                 1.0 / (double)cpr, dst);
        return hipGetLastError();
    }
    const dim3 grid((unsigned)((n + 255) / 256));
    convert_f16_kernel<<<grid, 256, 0, st>>>(src.data, src.type, row_addr(src), src.ne[0], pitch, n, dst);
    return hipGetLastError();
}

// weight conversions for the model-file loader: one thread per 32 elements
__global__ __launch_bounds__(256) void convert_weights_kernel(const uint8_t* __restrict__ src, int src_type,
                                                              void* __restrict__ dst, int dst_type, int64_t n) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b * QK >= n) return;
    const int64_t e0 = b * QK;
    const int cnt = (int)min((int64_t)QK, n - e0);
    float x[QK];
    if (src_type == T_F32) {
        const float* s = reinterpret_cast<const float*>(src) + e0;
        for (int j = 0; j < cnt; ++j) x[j] = s[j];
    } else if (src_type == T_F16) {
        const uint16_t* s = reinterpret_cast<const uint16_t*>(src) + e0;
        for (int j = 0; j < cnt; ++j) x[j] = h2f(s[j]);
    } else if (src_type == T_Q8_0) {
        const blk_q8_0* blk = reinterpret_cast<const blk_q8_0*>(src) + b;
        const float d = h2f(blk->d);
#pragma unroll
        for (int j = 0; j < QK; ++j) x[j] = (float)blk->qs[j] * d;
    } else if (src_type == T_Q4_0) {
        const blk_q4_0* blk = reinterpret_cast<const blk_q4_0*>(src) + b;
        const float d = h2f(blk->d);
#pragma unroll
        for (int j = 0; j < QK / 2; ++j) {
            x[j] = (float)((blk->qs[j] & 0x0f) - 8) * d;
            x[j + QK / 2] = (float)((blk->qs[j] >> 4) - 8) * d;
        }
    } else {  // Q4_1: q*d + m, each rounded (no contraction)
        const blk_q4_1* blk = reinterpret_cast<const blk_q4_1*>(src) + b;
        const float d = h2f(blk->d), m = h2f(blk->m);
#pragma unroll
        for (int j = 0; j < QK / 2; ++j) {
            x[j] = __fadd_rn(__fmul_rn((float)(blk->qs[j] & 0x0f), d), m);
            x[j + QK / 2] = __fadd_rn(__fmul_rn((float)(blk->qs[j] >> 4), d), m);
        }
    }
    if (dst_type == T_F32) {
        float* o = reinterpret_cast<float*>(dst) + e0;
        for (int j = 0; j < cnt; ++j) o[j] = x[j];
    } else {
        uint16_t* o = reinterpret_cast<uint16_t*>(dst) + e0;
        for (int j = 0; j < cnt; ++j) o[j] = f2h(x[j]);
    }
}

hipError_t launch_convert_weights(const void* src, int src_type, void* dst, int dst_type, int64_t n, hipStream_t st) {
    const bool ok = (src_type == T_F16 && dst_type == T_F32) || (src_type == T_F32 && dst_type == T_F16) ||
                    ((src_type == T_Q8_0 || src_type == T_Q4_0 || src_type == T_Q4_1) && dst_type == T_F32 && n % QK == 0);
    if (!ok) return hipErrorInvalidValue;
    const int64_t nb = (n + QK - 1) / QK;
    if (nb > 0)
        convert_weights_kernel<<<(unsigned)((nb + 255) / 256), 256, 0, st>>>(static_cast<const uint8_t*>(src), src_type,
                                                                             dst, dst_type, n);
    return hipGetLastError();
}

}  // namespace mi355
