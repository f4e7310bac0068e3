// ggml FLASH_ATTN_EXT (mask = NULL, max_bias = 0, logit_softcap = 0) on
// gfx950 fp16 MFMA with fp32 online softmax.
//
//   dst[b][iq][h][:] = sum_j softmax_j(scale * q.k_j) v_j
//   q [D, n_q, n_head, B], k [D, n_kv, n_head_k, B], v [D, n_kv, n_head_v, B]
//   (F32 or F16, any row strides), dst [D, n_head, n_q, B] F32 contiguous.
//
// Q, K and V enter the MFMAs as fp16 (round to nearest even, as ggml-cpu
// converts Q for an F16 K); scores, the softmax statistics and the output
// accumulate in fp32.
//
// Workgroup: 128 queries of one (head, batch), four wavefronts of 32
// queries; the key/value sequence streams through LDS in tiles of 64 keys.
//   scores:  S^T[key][q] = K Q^T (v_mfma_f32_32x32x16_f16, A = K rows from
//            LDS, B = the wavefront's Q fragment held in registers), so each
//            lane owns one query column and 16 keys of every 32-key block:
//            row max / row sum are in-lane plus one exchange with lane l ^ 32.
//   softmax: exp2 domain, c = |scale| * log2(e) folded into one FMA per score;
//            the running max is raised lazily (only by more than 8), so most
//            tiles skip rescaling O; P is packed to fp16 pairs by one convert
//            and the row sum takes the same fp16 values through dot2.
//   output:  O^T[d][q] += V^T P^T.  The P registers are used directly as the
//            B operand: MFMA k-slot j of lane group g carries key
//            16h + 8(j/4) + 4g + j%4 of the 32-key block, and the V^T rows
//            are read from LDS with the same key order.
// K is staged row-major with rows padded by 16 bytes and V transposed with
// rows padded by 8 bytes, so the 32-row fragment reads spread over all LDS
// banks (no bank conflicts in rocprofv3's counters).  Two K / V^T buffers:
// after tile t's MFMAs tile t + 1 goes from registers into the free buffer
// and tile t + 2's global loads are issued, with one LDS-only barrier per
// tile.  An fp16 K with D = 64, 96 or 128 (16-byte aligned rows) skips the
// registers: right after the barrier that frees its buffer, tile t + 1's K
// is copied by LDS DMA (buffer_load ... lds) into unpadded rows whose 16-byte
// chunks are XOR-swizzled by row, and the next barrier waits for it with an
// explicit vmcnt that leaves the V loads issued after it in flight.
#include <algorithm>

#include "common.cuh"
#include "kernels.h"

namespace mi355 {

namespace {
constexpr int FA_BQ = 128, FA_BKV = 64, FA_NT = 256;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef u32x4 u32x4_a4 __attribute__((aligned(4)));
typedef v4f v4f_a4 __attribute__((aligned(4)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
}  // namespace

// 8 consecutive elements of a row as fp16 (RNE), packed in 4 dwords
template <bool F32>
__device__ __forceinline__ u32x4 load8_h(const char* p) {
    if (F32) {
        const v4f a = *reinterpret_cast<const v4f_a4*>(p);
        const v4f b = *reinterpret_cast<const v4f_a4*>(p + 16);
        u32x4 r;
        r[0] = (uint32_t)f2h(a[0]) | ((uint32_t)f2h(a[1]) << 16);
        r[1] = (uint32_t)f2h(a[2]) | ((uint32_t)f2h(a[3]) << 16);
        r[2] = (uint32_t)f2h(b[0]) | ((uint32_t)f2h(b[1]) << 16);
        r[3] = (uint32_t)f2h(b[2]) | ((uint32_t)f2h(b[3]) << 16);
        return r;
    } else {
        return *reinterpret_cast<const u32x4_a4*>(p);
    }
}

// max / sum over lanes l and l ^ 32 (the two halves of the wavefront hold the same
// queries): v_permlane32_swap of x with itself leaves x_l and x_(l^32) in its two
// results, in an order that depends on the half, and both operations are commutative
__device__ __forceinline__ float xmax32(float x) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
    return fmaxf(__int_as_float((int)p[0]), __int_as_float((int)p[1]));
}
// Workgroup barrier for LDS hazards only: waits for this wavefront's LDS accesses,
// not for its global loads still in flight (__syncthreads() also waits for those).
// The "memory" clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ float xsum32(float x) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
    return __int_as_float((int)p[0]) + __int_as_float((int)p[1]);
}

// K row slot of 16-byte chunk c in row r of an unpadded fp16 K tile (DMA staging):
// the 32-row fragment reads of one chunk then fall in distinct bank quads
// (D = 96: 192-byte rows, four to three bank lines; (r >> 2) & 3 keeps a chunk inside its
// aligned group of four, so the twelve slots stay twelve)
template <int D>
__device__ __forceinline__ int kswz(int r) { return D == 64 ? ((r & 7) ^ ((r >> 3) & 1)) : D == 96 ? ((r >> 2) & 3) : (r & 15); }
// V row slot of 16-byte chunk c in row r of an unpadded fp16 V tile (DMA staging): slot
// c ^ vswz(r).  A transposing read of the PV operand takes 64 bytes (4 chunks 4 db .. +3)
// from each of 4 consecutive rows per half-wavefront; the 64 banks of 4 bytes then hold each
// byte once when the 4 rows' chunks land in distinct 64-byte quarters of a 256-byte bank
// line: D = 64 (128-byte rows: odd rows are the upper bank half) moves rows 2, 3 (mod 4) to
// the other half of their row's slots and rows 4..7 (mod 8) by one chunk; D = 128 (256-byte
// rows) moves row r by 4 (r % 4) chunks; D = 96 (192-byte rows) needs none: the 4 rows start
// at 0, 192, 384 and 576 bytes, so their 64-byte pieces fall in distinct quarters already.
// (The transposing reads add whole 8-row blocks to a swizzled row offset, so vswz may
// depend on r % 8 only.)
template <int D>
__device__ __forceinline__ int vswz(int r) { return D == 64 ? (((r & 2) << 1) | ((r >> 2) & 1)) : D == 96 ? 0 : ((r & 3) << 2); }

// 4 fp16 of LDS by the transposing read of gfx950 (ds_read_b64_tr_b16): within each group
// of 16 lanes, lane i receives element i % 4 of the 8 bytes addressed by lanes i / 4,
// 4 + i / 4, 8 + i / 4 and 12 + i / 4 of its group, in that order
__device__ __forceinline__ uint2 lds_read_tr16(const void* a) {
    typedef short v4s __attribute__((ext_vector_type(4)));
    const v4s r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(a));
    return __builtin_bit_cast(uint2, r);
}

// NW wavefronts of 32 queries per workgroup (4; 1 or 2 for small windows) and NBUF K/V tile
// buffers (2; 1 when the launcher guarantees a single key tile): a window of at most 64
// keys and 32 or 64 queries then runs in a workgroup of its own size with half the LDS, so
// several times more windows are in flight; the arithmetic per query is the same.
// KDMA: fp16 K and V with 16-byte rows reach LDS by DMA (buffer_load ... lds) and the loop
// is software-pipelined; otherwise they pass through registers.
template <int D, bool QF32, bool KVF32, bool KDMA, int NW = 4, int NBUF = 2>
__global__ __launch_bounds__(64 * NW, NW == 4 ? 2 : 1) void fattn_kernel(const FaArgs p) {
    static_assert(!KDMA || (!KVF32 && (D == 64 || D == 96 || D == 128)), "K/V DMA staging: fp16 K and V, D = 64, 96 or 128");
    static_assert((NW == 4 && NBUF == 2) || (!KDMA && NBUF == 1 && (NW == 1 || NW == 2)), "workgroup shape");
    constexpr int NT = 64 * NW, BQ = 32 * NW;  // threads and queries per workgroup
    constexpr int KS = KDMA ? D : D + 8;  // K tile row stride (halves)
    constexpr int VS = FA_BKV + 4;  // V^T tile row stride (halves): 34 dwords, so the 8-byte reads of 32 rows hit distinct bank pairs
    constexpr int VTILE = KDMA ? FA_BKV * D : D * VS;  // V tile (halves): rows of keys (DMA) or of V^T
    constexpr int NC = D / 16;      // MFMA k-chunks of a score
    constexpr int NDB = D / 32;     // 32-row blocks of O^T
    constexpr int C8 = D / 8;       // 8-element chunks per key row
    constexpr int LPT = FA_BKV * C8 / NT;  // chunks per thread per tile (K and V each)
    static_assert(FA_BKV * C8 % NT == 0, "tile split");
    // two K / V buffers: tile t + 1 is stored while tile t is computed
    __shared__ __attribute__((aligned(16))) _Float16 sK[NBUF][FA_BKV * KS];
    __shared__ __attribute__((aligned(16))) _Float16 sV[NBUF][VTILE];
    // the pipelined loop (K DMA) needs two tiles of scores in registers and keeps each
    // lane's Q fragment in LDS instead: slot (w, c, lane), written and read by that lane only
    constexpr bool QLDS = KDMA;
    __shared__ __attribute__((aligned(16))) u32x4 sQ[QLDS ? NW * NC * 64 : 1];

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 31, g = lane >> 5;
    // XCD-aware order: workgroups go round-robin to the 8 XCDs, so workgroup g takes item
    // (g % 8) * per_xcd + g / 8 of the (batch x key range, head, query tile) list and each
    // XCD walks a contiguous band: the query tiles of a few heads at a time, whose K and V
    // then stay in that XCD's L2 instead of every head's K and V passing through every L2
    const int qtiles = (p.nq + BQ - 1) / BQ, items = qtiles * p.nh * p.B * p.kv_split;
    const int per_xcd = (items + 7) / 8;
    const int item = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (item >= items) return;
    const int qt = item % qtiles, hz = item / qtiles, h = hz % p.nh, z = hz / p.nh;
    const int b = z / p.kv_split, ks = z - b * p.kv_split;
    const int qi = qt * BQ + w * 32 + lr;  // this lane's query
    // a key split attends to keys kbeg .. kbeg + nkv: shifted K/V bases, the same code
    const int kbeg = ks * p.kv_chunk, nkv = min(p.nkv - kbeg, p.kv_chunk);
    const char* kb = p.k + (int64_t)(h / p.rk2) * p.k_nb2 + (int64_t)b * p.k_nb3 + (int64_t)kbeg * p.k_nb1;
    const char* vb = p.v + (int64_t)(h / p.rv2) * p.v_nb2 + (int64_t)b * p.v_nb3 + (int64_t)kbeg * p.v_nb1;
    constexpr int KES = KVF32 ? 4 : 2;

    // Q fragment (B operand of S^T): query qi, elements 16c + 8g .. +7
    v8h qf[NC];
    {
        const char* qrow = p.q + (int64_t)qi * p.q_nb1 + (int64_t)h * p.q_nb2 + (int64_t)b * p.q_nb3;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            u32x4 r = {0, 0, 0, 0};
            if (qi < p.nq) r = load8_h<QF32>(qrow + (16 * c + 8 * g) * (QF32 ? 4 : 2));
            if (p.negq) r ^= 0x80008000u;
            if (QLDS) sQ[(w * NC + c) * 64 + lane] = r;
            else qf[c] = __builtin_bit_cast(v8h, r);
        }
    }

    // global -> register staging of one K/V tile (the non-DMA path).  K chunk j of thread t:
    // key (t + 256j) / C8, column (t + 256j) % C8 (a key row's chunks on consecutive lanes).
    // V, when C8 % 8 == 0: thread t takes keys 2q, 2q + 1 (q = (t + 256i) % 32) of column
    // chunk (t + 256i) / 32, so each V^T row gets the pair as one 32-bit write; otherwise V
    // chunk j is key (t + 256j) % 64, column (t + 256j) / 64, written as 16-bit halves.
    constexpr bool VPAIR = C8 % 8 == 0;
    u32x4 kreg[KDMA ? 1 : LPT], vreg[KDMA ? 1 : LPT];
    auto load_tile = [&](int kv0) {
#pragma unroll
        for (int j = 0; j < (KDMA ? 0 : LPT); ++j) {
            const int id = tid + NT * j;
            const int kk = id / C8, kc = id % C8;
            kreg[j] = u32x4{0, 0, 0, 0};
            if (kv0 + kk < nkv) kreg[j] = load8_h<KVF32>(kb + (int64_t)(kv0 + kk) * p.k_nb1 + kc * 8 * KES);
            int vk, vc;
            if (VPAIR) {
                const int pid = tid + NT * (j >> 1);
                vk = 2 * (pid % 32) + (j & 1);
                vc = pid / 32;
            } else {
                vk = id % FA_BKV;
                vc = id / FA_BKV;
            }
            vreg[j] = u32x4{0, 0, 0, 0};
            if (kv0 + vk < nkv) vreg[j] = load8_h<KVF32>(vb + (int64_t)(kv0 + vk) * p.v_nb1 + vc * 8 * KES);
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int j = 0; j < (KDMA ? 0 : LPT); ++j) {
            const int id = tid + NT * j;
            const int kk = id / C8, kc = id % C8;
            *reinterpret_cast<u32x4*>(&sK[buf][kk * KS + kc * 8]) = kreg[j];
        }
        if (KDMA) {
        } else if (VPAIR) {
#pragma unroll
            for (int j = 0; j < LPT; j += 2) {
                const int pid = tid + NT * (j >> 1);
                const int vk = 2 * (pid % 32), vc = pid / 32;
                uint32_t* col = reinterpret_cast<uint32_t*>(&sV[buf][(vc * 8) * VS + vk]);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    col[(2 * e) * (VS / 2)] = (vreg[j][e] & 0xffffu) | (vreg[j + 1][e] << 16);
                    col[(2 * e + 1) * (VS / 2)] = (vreg[j][e] >> 16) | (vreg[j + 1][e] & 0xffff0000u);
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < LPT; ++j) {
                const int id = tid + NT * j;
                const int vk = id % FA_BKV, vc = id / FA_BKV;
                uint16_t* col = reinterpret_cast<uint16_t*>(&sV[buf][(vc * 8) * VS + vk]);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    col[(2 * e) * VS] = (uint16_t)(vreg[j][e] & 0xffffu);
                    col[(2 * e + 1) * VS] = (uint16_t)(vreg[j][e] >> 16);
                }
            }
        }
    };
    // K and V tiles by LDS DMA (buffer_load ... lds): wavefront w fills bytes
    // [1024 (w KDI + j), +1024) of a tile with instruction j, lane i writing 16 bytes at
    // + 16 i, i.e. slot s of row r; it loads chunk s ^ kswz(r) (K) or s ^ vswz(r) (V) of key
    // kv0 + r.  Keys past nkv lie past the end of the buffer resource and read as zero.
    constexpr int KDI = KDMA ? FA_BKV * D * 2 / 1024 / (NT / 64) : 1;
    const v4i krsrc = make_rsrc(kb, (int64_t)nkv * p.k_nb1);
    const v4i vrsrc = make_rsrc(vb, (int64_t)nkv * p.v_nb1);
    auto dma_k = [&](int kv0, int buf) {
#pragma unroll
        for (int j = 0; j < KDI; ++j) {
            const int base = (w * KDI + j) << 10, byte = base + 16 * lane;
            const int r = byte / (2 * D), s = (byte % (2 * D)) / 16;
            dma_b128(krsrc, reinterpret_cast<const char*>(sK[buf]) + base,
                     (kv0 + r) * (int)p.k_nb1 + 16 * (s ^ kswz<D>(r)));
        }
    };
    auto dma_v = [&](int kv0, int buf) {
#pragma unroll
        for (int j = 0; j < KDI; ++j) {
            const int base = (w * KDI + j) << 10, byte = base + 16 * lane;
            const int r = byte / (2 * D), s = (byte % (2 * D)) / 16;
            dma_b128(vrsrc, reinterpret_cast<const char*>(sV[buf]) + base,
                     (kv0 + r) * (int)p.v_nb1 + 16 * (s ^ vswz<D>(r)));
        }
    };

    v16f O[NDB];
#pragma unroll
    for (int i = 0; i < NDB; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) O[i][e] = 0.0f;
    const v16f zf = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    float m_run = -__builtin_inff(), l_run = 0.0f;
    const float c = p.c;

    // S^T of one key tile (K in buffer kbuf) for its two 32-key halves
    auto score = [&](int kbuf, v16f* S) {
        S[0] = zf;
        S[1] = zf;
#pragma unroll
        for (int cc = 0; cc < NC; ++cc) {
            const v8h bq = QLDS ? __builtin_bit_cast(v8h, sQ[(w * NC + cc) * 64 + lane]) : qf[cc];
#pragma unroll
            for (int kh = 0; kh < 2; ++kh) {
                const int r = 32 * kh + lr, slot = KDMA ? (2 * cc + g) ^ kswz<D>(r) : 2 * cc + g;
                const v8h a = *reinterpret_cast<const v8h*>(&sK[kbuf][r * KS + 8 * slot]);
                S[kh] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bq, S[kh], 0, 0, 0);
            }
        }
    };
    // keys kv0 + 64 > nkv of the tile take no weight
    auto mask = [&](v16f* S, int kv0) {
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int key = kv0 + 32 * kh + 8 * (i >> 2) + 4 * g + (i & 3);
                if (key >= nkv) S[kh][i] = -__builtin_inff();
            }
    };
    // Online softmax of one tile's scores into the fp16 probability pairs P, with the
    // running max, the row sum and (when the max moved) O updated.
    // Online softmax of one tile's scores into the fp16 probability pairs P, with the
    // running max, the lane's part of the row sum and (when the max moved) O updated.
    // The probabilities are first taken against the running max as it stands; only when
    // some lane's sum of them exceeds 2^12 (or is not finite: the first tile, whose
    // running max is -inf) does the wavefront find the tile's max and take them again
    // against the raised max, rescaling O and the sum.  Every probability is at most its
    // lane's sum, so P stays below 2^12 (fp16), and most tiles skip the max altogether.
    // The two lanes of a query pair compute the same max, so they agree on the reference.
    auto softmax = [&](const v16f* S, uint32_t (*P)[8]) {
        const h2v ones = {(_Float16)1.0f, (_Float16)1.0f};
        // probabilities rounded to fp16 in pairs (the PV operand); the row sum adds the same
        // rounded values (one dot2 per pair), so numerator and denominator agree
        auto probs = [&](float m) {
            float ls = 0.0f;
#pragma unroll
            for (int kh = 0; kh < 2; ++kh)
#pragma unroll
                for (int i = 0; i < 16; i += 2) {
                    const v2f pp = {__builtin_amdgcn_exp2f(__builtin_fmaf(S[kh][i], c, -m)),
                                    __builtin_amdgcn_exp2f(__builtin_fmaf(S[kh][i + 1], c, -m))};
                    const h2v ph = __builtin_convertvector(pp, h2v);
                    ls = __builtin_amdgcn_fdot2(ph, ones, ls, false);
                    P[kh][i >> 1] = __builtin_bit_cast(uint32_t, ph);
                }
            return ls;
        };
        float ls = probs(m_run);
        if (__builtin_amdgcn_ballot_w64(!(ls <= 4096.0f))) {
            // four independent max chains, then the pair of lanes holding the same query
            float m4[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const v16f& sv = S[j >> 1];
                const int o = 8 * (j & 1);
                m4[j] = fmaxf(fmaxf(fmaxf(sv[o], sv[o + 1]), fmaxf(sv[o + 2], sv[o + 3])),
                              fmaxf(fmaxf(sv[o + 4], sv[o + 5]), fmaxf(sv[o + 6], sv[o + 7])));
            }
            const float mx = xmax32(fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3])));
            const float m_new = fmaxf(m_run, mx * c);
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            m_run = m_new;
            ls = probs(m_new);
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int e = 0; e < 16; ++e) O[db][e] *= alpha;
        }
        l_run += ls;
    };
    // O^T += V^T P^T over the 64 keys of V buffer vbuf (four 16-key MFMA chunks)
    // V^T fragment rows by transposing reads of the DMA-staged V tile: lane (lr, g) of
    // 16-lane group (lane / 16) addresses key 4g + j (j = (lane % 16) / 4) of an 8-key block,
    // columns 32 db + 16 ((lane / 16) % 2) + 4q .. +3 (q = lane % 4), and receives column
    // 32 db + lr of keys 4g .. 4g + 3 of the block
    int vtoff[NDB];
    if (KDMA) {
        const int j = (lane & 15) >> 2, q = lane & 3, rw = 4 * g + j;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
            vtoff[db] = rw * 2 * D + 16 * ((4 * db + 2 * ((lane >> 4) & 1) + (q >> 1)) ^ vswz<D>(rw)) + 8 * (q & 1);
    }
    // O^T += V^T P^T over the 64 keys of V buffer vbuf (four 16-key MFMA chunks)
    auto pv = [&](int vbuf, uint32_t (*P)[8]) {
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            const _Float16* vrow = &sV[vbuf][(32 * db + lr) * VS];
#pragma unroll
            for (int kh = 0; kh < 2; ++kh)
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int k0 = 32 * kh + 16 * hh + 4 * g;
                    uint2 lo, hi;
                    if (KDMA) {
                        const char* vt = reinterpret_cast<const char*>(sV[vbuf]) + vtoff[db] + (32 * kh + 16 * hh) * 2 * D;
                        lo = lds_read_tr16(vt);
                        hi = lds_read_tr16(vt + 8 * 2 * D);
                    } else {
                        lo = *reinterpret_cast<const uint2*>(&vrow[k0]);
                        hi = *reinterpret_cast<const uint2*>(&vrow[k0 + 8]);
                    }
                    const v4i av = {(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
                    const v4i bp = {(int)P[kh][4 * hh], (int)P[kh][4 * hh + 1], (int)P[kh][4 * hh + 2],
                                    (int)P[kh][4 * hh + 3]};
                    O[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, av),
                                                                  __builtin_bit_cast(v8h, bp), O[db], 0, 0, 0);
                }
        }
    };

    const int ntile = (nkv + FA_BKV - 1) / FA_BKV;
    if (NBUF == 1 && ntile > 1) return;  // one buffer holds one tile (the launcher's condition)
    if constexpr (KDMA) {
        // Software pipeline, the K tiles one ahead of V: step t issues the score MFMAs of
        // tile t + 1 and then does the softmax of tile t (scored in step t - 1), so the
        // matrix core works on the next scores while the VALU works on these, and then the
        // PV MFMAs of tile t.  One LDS-only barrier per step, after the wait for this
        // wavefront's DMAs of step t - 1, publishes K(t + 1) and V(t) and frees K buffer
        // t % 2 (K(t), read in step t - 1) and V buffer (t + 1) % 2 (V(t - 1)), which take
        // K(t + 2) and V(t + 1) by DMA.  No DMA is left in flight past the last step.
        v16f SA[2], SB[2];
        uint32_t P[2][8];
        dma_k(0, 0);
        dma_v(0, 0);
        if (ntile > 1) dma_k(FA_BKV, 1);
        if (ntile > 1) wait_vmcnt<KDI>();
        else wait_vmcnt<0>();
        lds_barrier();
        score(0, SA);
        auto step = [&](int t, int cb, v16f* Sc, v16f* Sn) {
            const int kv0 = t * FA_BKV;
            wait_vmcnt<0>();
            lds_barrier();
            if (t + 2 < ntile) dma_k(kv0 + 2 * FA_BKV, cb);
            if (t + 1 < ntile) dma_v(kv0 + FA_BKV, cb ^ 1);
            if (kv0 + FA_BKV > nkv) mask(Sc, kv0);
            score(cb ^ 1, Sn);  // tile t + 1 (past the last tile: stale LDS, never used)
            softmax(Sc, P);
            pv(cb, P);
        };
        for (int t = 0; t < ntile; t += 2) {
            step(t, 0, SA, SB);
            if (t + 1 < ntile) step(t + 1, 1, SB, SA);
        }
    } else {
        // One LDS-only barrier per tile: it publishes tile t (stored at the end of tile
        // t - 1) and frees the other buffer (read by tile t - 1).  After tile t's compute,
        // tile t + 1 goes from the registers (loaded during tile t) into that buffer and
        // tile t + 2's loads are issued, so each load has a whole tile to land.
        load_tile(0);
        store_tile(0);
        if (ntile > 1) load_tile(FA_BKV);
        for (int t = 0; t < ntile; ++t) {
            const int kv0 = t * FA_BKV, cb = NBUF == 1 ? 0 : (t & 1);
            lds_barrier();
            v16f S[2];
            uint32_t P[2][8];
            score(cb, S);
            if (kv0 + FA_BKV > nkv) mask(S, kv0);
            softmax(S, P);
            pv(cb, P);
            if (NBUF == 2 && t + 1 < ntile) {
                store_tile(cb ^ 1);
                if (t + 2 < ntile) load_tile(kv0 + 2 * FA_BKV);
            }
        }
    }

    l_run = xsum32(l_run);  // the two lanes of a query summed over different keys
    if (qi < p.nq && p.kv_split > 1) {  // this key range's unnormalised O and (max, sum)
        const int64_t pr = ((int64_t)ks * p.B * p.nh + (int64_t)b * p.nh + h) * p.nq + qi;
        float* orow = p.part + pr * D;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                const int d = 32 * db + 8 * i4 + 4 * g;
                *reinterpret_cast<v4f*>(orow + d) = v4f{O[db][4 * i4], O[db][4 * i4 + 1], O[db][4 * i4 + 2], O[db][4 * i4 + 3]};
            }
        if (g == 0) {
            const int64_t rows = (int64_t)p.B * p.nh * p.nq;
            float* ml = p.part + (int64_t)p.kv_split * rows * D + pr * 2;
            ml[0] = m_run;
            ml[1] = l_run;
        }
    } else if (qi < p.nq) {
        const float inv = l_run == 0.0f ? 0.0f : 1.0f / l_run;
        if (p.out.mode == ACT_F32) {
            float* orow = p.dst + (((int64_t)b * p.nq + qi) * p.nh + h) * D;
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4) {
                    const int d = 32 * db + 8 * i4 + 4 * g;
                    v4f o = {O[db][4 * i4] * inv, O[db][4 * i4 + 1] * inv, O[db][4 * i4 + 2] * inv,
                             O[db][4 * i4 + 3] * inv};
                    *reinterpret_cast<v4f*>(orow + d) = o;
                }
        } else {
            // the projection's operand: row b*nq + qi, columns h*D + d.  Lanes l and
            // l ^ 32 hold the two halves of each 32-value block (ggml from_float x86:
            // d = amax/127, q = rint(x * 127/amax)).
            const ActOut& o = p.out;
            const int64_t K = (int64_t)p.nh * D, row = (int64_t)b * p.nq + qi;
            uint16_t* qrow = o.q + row * K + (int64_t)h * D;
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
                float x[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) x[i] = O[db][i] * inv;
                float sc = 1.0f;
                if (o.mode != ACT_F16) {
                    float amax = 0.0f;
#pragma unroll
                    for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(x[i]));
                    amax = xmax32(amax);
                    sc = amax != 0.0f ? 127.0f / amax : 0.0f;
                    int isum = 0;
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        x[i] = rintf(x[i] * sc);
                        isum += (int)x[i];
                    }
                    if (act_has_sums(o.mode))
                        isum += lane_swap<32>(isum);
                    if (g == 0) act_store_scale(o, row, K, ((int64_t)h * D + 32 * db) / 32, amax / 127.0f, isum);
                }
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4) {
                    const int d = 32 * db + 8 * i4 + 4 * g;
                    if (o.mode >= ACT_I8) {
                        const uint32_t b4 = (uint32_t)((int)x[4 * i4] & 0xff) | ((uint32_t)((int)x[4 * i4 + 1] & 0xff) << 8) |
                                            ((uint32_t)((int)x[4 * i4 + 2] & 0xff) << 16) |
                                            ((uint32_t)((int)x[4 * i4 + 3] & 0xff) << 24);
                        *reinterpret_cast<uint32_t*>(reinterpret_cast<int8_t*>(o.q) + row * K + (int64_t)h * D + d) = b4;
                    } else {
                        const uint32_t h0 = (uint32_t)f2h(x[4 * i4]) | ((uint32_t)f2h(x[4 * i4 + 1]) << 16);
                        const uint32_t h1 = (uint32_t)f2h(x[4 * i4 + 2]) | ((uint32_t)f2h(x[4 * i4 + 3]) << 16);
                        *reinterpret_cast<uint2*>(qrow + d) = make_uint2(h0, h1);
                    }
                }
            }
        }
    }
}

// Key-split combine: thread per (batch, head, query, 4 outputs); m* = max of the
// ranges' maxima, O = sum_s 2^(m_s - m*) O_s, l likewise, out = O / l.  The
// operand output keeps 8 consecutive threads on one 32-block.
template <int D>
__global__ __launch_bounds__(256) void fattn_combine_kernel(const FaArgs p, int B) {
    constexpr int CPR = D / 4;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t rows = (int64_t)B * p.nh * p.nq;
    if (t >= rows * CPR) return;
    const int64_t pr = t / CPR;
    const int c = (int)(t - pr * CPR);
    const int qi = (int)(pr % p.nq), h = (int)((pr / p.nq) % p.nh), b = (int)(pr / ((int64_t)p.nq * p.nh));
    const float* ml = p.part + (int64_t)p.kv_split * rows * D;
    float mx = -__builtin_inff();
    for (int s = 0; s < p.kv_split; ++s) mx = fmaxf(mx, ml[(s * rows + pr) * 2]);
    float l = 0.0f;
    v4f o = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s = 0; s < p.kv_split; ++s) {
        const float wgt = __builtin_amdgcn_exp2f(ml[(s * rows + pr) * 2] - mx);
        l = l + wgt * ml[(s * rows + pr) * 2 + 1];
        o = o + wgt * *reinterpret_cast<const v4f*>(&p.part[(s * rows + pr) * D + 4 * c]);
    }
    const float inv = l == 0.0f ? 0.0f : 1.0f / l;
    o = o * inv;
    if (p.out.mode == ACT_F32)
        *reinterpret_cast<v4f*>(p.dst + (((int64_t)b * p.nq + qi) * p.nh + h) * D + 4 * c) = o;
    else
        act_store_chunk(p.out, (int64_t)b * p.nq + qi, (int64_t)p.nh * D, ((int64_t)h * D) / 4 + c, o);
}

int fattn_kv_split(int nq, int nkv, int nh, int B, int cus) {
    const int64_t wgs = (int64_t)((nq + FA_BQ - 1) / FA_BQ) * nh * B;
    const int ntile = (nkv + FA_BKV - 1) / FA_BKV;
    // below eight key tiles the combine pass costs more than the idle CUs (Hiera-tiny's 14x14
    // windows, 4 tiles over 200 workgroups: 12.2 us split in two + 7 us combine, against one pass)
    if (cus <= 0 || wgs >= cus || ntile < 8) return 1;
    const int64_t want = (2LL * cus + wgs - 1) / wgs;
    const int ks = (int)std::min<int64_t>(want, ntile / 2);
    return ks < 2 ? 1 : std::min(ks, 16);
}

size_t fattn_part_bytes(int D, int nq, int nh, int B, int kv_split) {
    if (kv_split <= 1) return 0;
    return (size_t)kv_split * B * nh * nq * (D + 2) * 4;
}

template <int D>
static void fa_launch_d(const FaArgs& a, bool qf32, bool kvf32, int B, hipStream_t st) {
    const int64_t items = (int64_t)((a.nq + FA_BQ - 1) / FA_BQ) * a.nh * B * a.kv_split;
    const dim3 grid((unsigned)((items + 7) / 8 * 8));
    bool launched = false;
    // windows of at most one key tile and 64 queries, fp16 operands, no key split: one or two
    // wavefronts per workgroup and one K/V buffer (taken before the DMA path, which would
    // give such a window four wavefronts and two buffers)
    const int nw = a.nq <= 32 ? 1 : 2;
    const bool small = !qf32 && !kvf32 && a.kv_split == 1 && a.nkv <= FA_BKV && a.nq <= 64;
    if (small) {
        const int64_t sitems = (int64_t)((a.nq + 32 * nw - 1) / (32 * nw)) * a.nh * B;
        const dim3 sgrid((unsigned)((sitems + 7) / 8 * 8));
        if (nw == 1) fattn_kernel<D, false, false, false, 1, 1><<<sgrid, 64, 0, st>>>(a);
        else fattn_kernel<D, false, false, false, 2, 1><<<sgrid, 128, 0, st>>>(a);
        launched = true;
    }
    if constexpr (D == 64 || D == 96 || D == 128) {
        // fp16 K and V rows and bases on 16 bytes, key offsets within the 32-bit buffer offset
        const bool kdma = !kvf32 && reinterpret_cast<uintptr_t>(a.k) % 16 == 0 && a.k_nb1 % 16 == 0 &&
                          a.k_nb2 % 16 == 0 && a.k_nb3 % 16 == 0 && (int64_t)(a.nkv + FA_BKV) * a.k_nb1 < INT32_MAX &&
                          reinterpret_cast<uintptr_t>(a.v) % 16 == 0 && a.v_nb1 % 16 == 0 && a.v_nb2 % 16 == 0 &&
                          a.v_nb3 % 16 == 0 && (int64_t)(a.nkv + FA_BKV) * a.v_nb1 < INT32_MAX;
        if (!launched && kdma) {
            if (qf32) fattn_kernel<D, true, false, true><<<grid, FA_NT, 0, st>>>(a);
            else fattn_kernel<D, false, false, true><<<grid, FA_NT, 0, st>>>(a);
            launched = true;
        }
    }
    if (launched) {
    } else if (qf32 && kvf32) fattn_kernel<D, true, true, false><<<grid, FA_NT, 0, st>>>(a);
    else if (qf32) fattn_kernel<D, true, false, false><<<grid, FA_NT, 0, st>>>(a);
    else if (kvf32) fattn_kernel<D, false, true, false><<<grid, FA_NT, 0, st>>>(a);
    else fattn_kernel<D, false, false, false><<<grid, FA_NT, 0, st>>>(a);
    if (a.kv_split > 1) {
        const int64_t n = (int64_t)B * a.nh * a.nq * (D / 4);
        fattn_combine_kernel<D><<<(unsigned)((n + 255) / 256), 256, 0, st>>>(a, B);
    }
}

hipError_t launch_fattn(const FaArgs& a_in, int D, bool qf32, bool kvf32, int B, hipStream_t st) {
    if (a_in.nq <= 0 || a_in.nkv <= 0 || a_in.nh <= 0 || B <= 0) return hipSuccess;
    if ((int64_t)((a_in.nq + FA_BQ - 1) / FA_BQ) * a_in.nh * B * a_in.kv_split + 7 >= INT32_MAX)
        return hipErrorInvalidValue;
    FaArgs a = a_in;
    a.B = B;
    if (a.kv_split < 1 || (a.kv_split > 1 && (!a.part || a.kv_chunk % FA_BKV != 0 ||
                                              (int64_t)(a.kv_split - 1) * a.kv_chunk >= a.nkv)))
        return hipErrorInvalidValue;
    switch (D) {
        case 64: fa_launch_d<64>(a, qf32, kvf32, B, st); break;
        case 96: fa_launch_d<96>(a, qf32, kvf32, B, st); break;
        case 128: fa_launch_d<128>(a, qf32, kvf32, B, st); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mi355
