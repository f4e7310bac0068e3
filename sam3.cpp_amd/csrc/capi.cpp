// C-ABI of the MI355X backend (include/sam3_mi355.h): ggml-semantics checks,
// workspace management and kernel dispatch.  Every entry point validates on
// the host before touching the GPU and reports problems as mi355_status,
// never by aborting (sam3.cpp returns bool/nullptr on failure, CLAUDE.md:62).
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "context.h"

thread_local std::string g_noctx_error;

namespace mi355 {

mi355_status fail(mi355_context* ctx, mi355_status st, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    if (ctx) ctx->last_error = buf;
    else g_noctx_error = buf;
    return st;
}

mi355_status hip_check(mi355_context* ctx, hipError_t e, const char* what) {
    if (e == hipSuccess) return MI355_STATUS_SUCCESS;
    return fail(ctx, MI355_STATUS_FAILED, "%s: %s", what, hipGetErrorString(e));
}

int64_t type_size(int t) {
    switch (t) {
        case T_F32: return 4;
        case T_F16: return 2;
        case T_Q4_0: return 18;
        case T_Q4_1: return 20;
        case T_Q8_0: return 34;
        case T_Q8_1: return 36;
        default: return 0;
    }
}
int blck(int t) { return (t == T_F32 || t == T_F16) ? 1 : (type_size(t) ? 32 : 0); }
int64_t row_size(int t, int64_t ne0) { return blck(t) ? type_size(t) * (ne0 / blck(t)) : 0; }

bool dims_ok(const mi355_tensor* t) {
    if (t->layout != MI355_LAYOUT_GGML) return false;
    for (int i = 0; i < 4; ++i)
        if (t->ne[i] < 0 || t->nb[i] < 0) return false;
    return true;
}

bool prepared_ok(const mi355_tensor* t) {
    return t->layout == MI355_LAYOUT_INT8 && (t->type == T_Q8_0 || t->type == T_Q4_0 || t->type == T_Q4_1) &&
           t->ne[0] >= 0 && t->ne[1] >= 0 && t->ne[2] == 1 && t->ne[3] == 1 && t->ne[0] % 32 == 0 &&
           (reinterpret_cast<uintptr_t>(t->data) & 255) == 0;
}

SrcView view_of(const mi355_tensor* t) {
    SrcView v;
    v.data = static_cast<const char*>(t->data);
    v.type = t->type;
    for (int i = 0; i < 4; ++i) {
        v.ne[i] = t->ne[i];
        v.nb[i] = t->nb[i];
    }
    return v;
}

constexpr size_t kAlign = 256;
size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

mi355_status ensure_buffer(mi355_context* ctx, void** buf, size_t* size, size_t bytes) {
    if (bytes <= *size) return MI355_STATUS_SUCCESS;
    if (*buf) {
        hipError_t e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) return hip_check(ctx, e, "hipStreamSynchronize");
        (void)hipFree(*buf);
        *buf = nullptr;
        *size = 0;
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) return fail(ctx, MI355_STATUS_ALLOC_FAILED, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    *buf = p;
    *size = bytes;
    return MI355_STATUS_SUCCESS;
}

}  // namespace mi355

namespace {

using namespace mi355;

MatW matw_of(const mi355_tensor* s0) {
    MatW w;
    w.data = static_cast<const uint8_t*>(s0->data);
    w.type = s0->type;
    w.nb1 = s0->nb[1];
    w.nb2 = s0->nb[2];
    w.nb3 = s0->nb[3];
    w.ne2 = s0->ne[2];
    w.ne3 = s0->ne[3];
    return w;
}
MatD matd_of(const mi355_tensor* d) {
    MatD o;
    o.data = static_cast<float*>(d->data);
    o.nb1 = d->nb[1];
    o.nb2 = d->nb[2];
    o.nb3 = d->nb[3];
    return o;
}

bool f16_src1_direct(const mi355_tensor* s1) {
    return s1->type == T_F16 && s1->ne[0] % 8 == 0 && s1->nb[0] == 2 && s1->nb[1] % 16 == 0 && s1->nb[2] % 16 == 0 && s1->nb[3] % 16 == 0 &&
           (reinterpret_cast<uintptr_t>(s1->data) & 15) == 0;
}

// Workspace of one MUL_MAT: activation operand (q, d, s), the 4-byte-pitch
// weight copy, then the split-K partial sums.
struct MmPlan {
    size_t q = 0, d = 0, s = 0, align = 0, part = 0;
    int ks = 1;
    bool i8 = false;    // int8-MFMA path: q holds int8 quants, align the repacked weights
    bool prep = false;  // src0 is a prepared weight: no repack (align empty)
    size_t total() const { return q + d + s + align + part; }
};

// The int8-MFMA kernel takes plain 2-D GEMMs with block-quantized weights.
bool mm_i8_eligible(const mi355_tensor* s0, const mi355_tensor* s1) {
    return (s0->type == T_Q8_0 || s0->type == T_Q4_0 || s0->type == T_Q4_1) && s0->ne[2] == 1 && s0->ne[3] == 1 &&
           s1->ne[2] == 1 && s1->ne[3] == 1 && s0->ne[0] % 32 == 0;
}

// The MUL_MAT kernels address their operands with 32-bit buffer offsets below 2^30 bytes
// (OOB8 / OOB mark lanes past the end): the int8 route's quants and scale dwords, the fp16
// route's weight slice, fp16 activation slice and scales.
constexpr int64_t kExtent = (int64_t)1 << 30;
bool i8_extents_ok(const mi355_tensor* s0, const mi355_tensor* s1) {
    const int64_t K = s0->ne[0], N = s0->ne[1], M = s1->ne[1], nst = mmq_scale_pitch(K) / 2;
    return M * K < kExtent && N * K < kExtent && 4 * M * nst < kExtent && 4 * N * nst < kExtent;
}
bool f16_extents_ok(const mi355_tensor* s0, const mi355_tensor* s1) {
    const int64_t K = s0->ne[0], N = s0->ne[1], M = s1->ne[1];
    const int64_t s1h = f16_src1_direct(s1) ? s1->nb[1] / 2 : (s0->type == T_F16 ? (K + 7) & ~(int64_t)7 : K);
    return (N - 1) * s0->nb[1] + row_size(s0->type, K) < kExtent && ((M - 1) * s1h + K) * 2 < kExtent &&
           2 * M * mmq_scale_pitch(K) < kExtent;
}

int device_cus(int device) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return 0;
    return n;
}

// split = false: the caller's dst cannot take the float4 stores of the split reduction;
// kernel: the MI355_MMQ_* route when the operands are eligible for it
MmPlan mm_plan(const mi355_tensor* s0, const mi355_tensor* s1, int cus, bool split = true, int kernel = 0) {
    const bool prep = s0->layout == MI355_LAYOUT_INT8;
    const bool i8 = prep || kernel == MI355_MMQ_INT8 ||
                    (kernel == MI355_MMQ_AUTO && (s0->type == T_Q8_0 || s0->type == T_Q4_0));
    MmPlan pl;
    if (s0->type == T_F32) return pl;
    const int64_t K = s1->ne[0], M = s1->ne[1], Z = s1->ne[2] * s1->ne[3];
    if (split) pl.ks = mmq_ksplit(s0->type, M, s0->ne[1], K, Z, cus);
    if (pl.ks > 1) pl.part = align_up((size_t)pl.ks * (size_t)M * (size_t)s0->ne[1] * 4);
    if (i8 && mm_i8_eligible(s0, s1) && i8_extents_ok(s0, s1)) {
        pl.i8 = true;
        pl.q = align_up((size_t)(M * K));
        pl.d = align_up((size_t)(M * mmq_scale_pitch(K)) * 4);  // dl and dh dwords
        if (s0->type == T_Q4_1) pl.s = align_up((size_t)(M * mmq_scale_pitch(K)) * 2);
        pl.prep = prep;
        pl.align = prep ? 0 : align_up(wrep_bytes(s0->type, s0->ne[1], K));
        return pl;
    }
    if (s0->type == T_F16) {
        if (!f16_src1_direct(s1)) pl.q = align_up((size_t)(Z * M * ((K + 7) & ~7)) * 2);
        pl.align = align_up(mmq_align_bytes(matw_of(s0), s0->ne[1], K));
        return pl;
    }
    pl.q = align_up((size_t)(Z * M * K) * 2);
    pl.d = align_up((size_t)(Z * M * mmq_scale_pitch(K)) * 2);
    if (s0->type == T_Q4_1) pl.s = pl.d;
    pl.align = align_up(mmq_align_bytes(matw_of(s0), s0->ne[1], K));
    return pl;
}

// ggml_soft_max_ext(a, mask, scale, max_bias) shape rules plus what softmax.hip implements.
mi355_status check_soft_max(mi355_context* ctx, const mi355_tensor* src, const mi355_tensor* mask, float max_bias,
                            const mi355_tensor* dst) {
    if (!src || !dst || !src->data || !dst->data) return fail(ctx, MI355_STATUS_INVALID_ARG, "soft_max: null argument");
    if (!dims_ok(src) || !dims_ok(dst)) return fail(ctx, MI355_STATUS_INVALID_ARG, "soft_max: negative ne/nb or not the ggml layout");
    if (mask || max_bias != 0.0f) return fail(ctx, MI355_STATUS_UNSUPPORTED, "soft_max: mask/ALiBi not supported");
    if (src->type != T_F32 || dst->type != T_F32) return fail(ctx, MI355_STATUS_UNSUPPORTED, "soft_max: F32 only");
    for (int i = 0; i < 4; ++i)
        if (src->ne[i] != dst->ne[i]) return fail(ctx, MI355_STATUS_INVALID_ARG, "soft_max: shape mismatch");
    if (src->ne[0] > 8192) return fail(ctx, MI355_STATUS_UNSUPPORTED, "soft_max: rows longer than 8192");
    return MI355_STATUS_SUCCESS;
}

bool dst_split_ok(const mi355_tensor* d) {
    return d->nb[1] % 16 == 0 && (reinterpret_cast<uintptr_t>(d->data) & 15) == 0;
}
mi355_status ensure_ws(mi355_context* ctx, size_t bytes) { return ensure_buffer(ctx, &ctx->ws, &ctx->ws_size, bytes); }


// ggml_mul_mat shape rules (ggml.c ggml_can_mul_mat / ggml_compute_forward_mul_mat)
// plus what the kernels here implement.
mi355_status check_mul_mat(mi355_context* ctx, const mi355_tensor* s0, const mi355_tensor* s1,
                           const mi355_tensor* d) {
    if (!s0 || !s1 || !d) return fail(ctx, MI355_STATUS_INVALID_ARG, "mul_mat: null tensor");
    if (!s0->data || !s1->data || !d->data) return fail(ctx, MI355_STATUS_INVALID_ARG, "mul_mat: null data pointer");
    const bool prep = s0->layout == MI355_LAYOUT_INT8;
    if (!dims_ok(s1) || !dims_ok(d)) return fail(ctx, MI355_STATUS_INVALID_ARG, "mul_mat: negative ne/nb or not a ggml layout");
    if (prep ? !prepared_ok(s0) : !dims_ok(s0))
        return fail(ctx, MI355_STATUS_INVALID_ARG, "mul_mat: src0 is neither a ggml tensor nor a prepared weight");
    const int t0 = s0->type;
    if (!(t0 == T_F32 || t0 == T_F16 || t0 == T_Q8_0 || t0 == T_Q4_0 || t0 == T_Q4_1))
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "mul_mat: src0 type %d not supported", t0);
    if (!(s1->type == T_F32 || (s1->type == T_F16 && t0 == T_F16)))
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "mul_mat: src1 type %d with src0 type %d not supported", s1->type, t0);
    if (d->type != T_F32) return fail(ctx, MI355_STATUS_UNSUPPORTED, "mul_mat: dst type %d not supported", d->type);
    const int64_t K = s0->ne[0];
    if (s1->ne[0] != K) return fail(ctx, MI355_STATUS_INVALID_ARG, "mul_mat: K mismatch %lld vs %lld", (long long)K, (long long)s1->ne[0]);
    if (K % blck(t0) != 0) return fail(ctx, MI355_STATUS_INVALID_ARG, "mul_mat: ne0 %lld not a multiple of the block size", (long long)K);
    if (s0->ne[2] == 0 || s0->ne[3] == 0 || s1->ne[2] % s0->ne[2] != 0 || s1->ne[3] % s0->ne[3] != 0)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "mul_mat: src1 batch dims not a multiple of src0's");
    if (d->ne[0] != s0->ne[1] || d->ne[1] != s1->ne[1] || d->ne[2] != s1->ne[2] || d->ne[3] != s1->ne[3])
        return fail(ctx, MI355_STATUS_INVALID_ARG, "mul_mat: dst shape mismatch");
    if (!prep && (s0->nb[0] != type_size(t0) || s0->nb[1] < row_size(t0, K)))
        return fail(ctx, MI355_STATUS_INVALID_ARG, "mul_mat: src0 rows must be contiguous");
    if (prep && (s1->ne[2] != 1 || s1->ne[3] != 1))
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "mul_mat: a prepared weight takes a 2-D src1");
    if (d->nb[0] != 4) return fail(ctx, MI355_STATUS_INVALID_ARG, "mul_mat: dst nb[0] must be 4");
    if (s1->nb[0] != type_size(s1->type) && s1->type != T_F32)
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "mul_mat: strided F16 src1 elements");
    const int64_t lim = (int64_t)1 << 30;
    if (K >= lim || s0->ne[1] >= lim || s1->ne[1] >= lim || s1->ne[2] * s1->ne[3] > 65535)
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "mul_mat: dimensions beyond kernel limits");
    if (prep ? !i8_extents_ok(s0, s1)
             : t0 != T_F32 && !(mm_i8_eligible(s0, s1) && i8_extents_ok(s0, s1)) && !f16_extents_ok(s0, s1))
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "mul_mat: operands beyond the kernels' 1 GiB buffer extents");
    if (t0 == T_F32) {
        if (s1->nb[0] != 4 || ((reinterpret_cast<uintptr_t>(s0->data) | (uintptr_t)s0->nb[1] | (uintptr_t)s0->nb[2] |
                                (uintptr_t)s0->nb[3] | reinterpret_cast<uintptr_t>(s1->data) | (uintptr_t)s1->nb[1] |
                                (uintptr_t)s1->nb[2] | (uintptr_t)s1->nb[3]) & 3))
            return fail(ctx, MI355_STATUS_UNSUPPORTED, "mul_mat f32: needs contiguous, 4-byte aligned rows");
    } else if (t0 == T_F16) {
        if (((reinterpret_cast<uintptr_t>(s0->data) | (uintptr_t)s0->nb[1] | (uintptr_t)s0->nb[2] |
              (uintptr_t)s0->nb[3]) & 1))
            return fail(ctx, MI355_STATUS_INVALID_ARG, "mul_mat f16: src0 rows must be 2-byte aligned");
    } else {
        if (reinterpret_cast<uintptr_t>(s0->data) & 1)
            return fail(ctx, MI355_STATUS_INVALID_ARG, "mul_mat: src0 data must be 2-byte aligned");
    }
    return MI355_STATUS_SUCCESS;
}

// Quantize src1 for src0's vec_dot_type into the workspace (x86 from_float).
// The workspace must already hold mm_plan(s0, s1).total() bytes.
mi355_status prep_act_q8(mi355_context* ctx, const mi355_tensor* s0, const mi355_tensor* s1, const MmPlan& pl,
                         char* p, bool timed, ActF16& a) {
    const int64_t K = s1->ne[0], M = s1->ne[1];
    const bool with_sum = s0->type == T_Q4_1;
    uint16_t* q = reinterpret_cast<uint16_t*>(p);
    uint16_t* d = reinterpret_cast<uint16_t*>(p + pl.q);
    uint16_t* sm = with_sum ? reinterpret_cast<uint16_t*>(p + pl.q + pl.d) : nullptr;
    a.q = q;
    a.s1 = K;
    a.s2 = K * M;
    a.s3 = K * M * s1->ne[2];
    a.d = d;
    a.s = sm;
    a.dp = mmq_scale_pitch(K);
    a.M = M;
    a.K = K;
    Timed tm(timed ? ctx : nullptr, "quantize_mmq");
    return hip_check(ctx, tm.done(launch_quantize_mmq(view_of(s1), with_sum, a.dp, q, d, sm, ctx->stream)),
                     "quantize_mmq launch");
}

// The int8 activation operand's carve-up of a workspace planned with pl.i8:
// quants [M][K], then dl and dh [M][nst], then the Q8_1 sums [M][2 nst].
ActI8 act_i8(char* ws, const MmPlan& pl, int wtype, int64_t M, int64_t K) {
    ActI8 a;
    a.q = ws;
    a.s1 = K;
    a.nst = mmq_scale_pitch(K) / 2;
    a.dl = reinterpret_cast<const uint32_t*>(ws + pl.q);
    a.dh = a.dl + M * a.nst;
    a.s = wtype == T_Q4_1 ? ws + pl.q + pl.d : nullptr;
    a.M = M;
    a.K = K;
    return a;
}

// MUL_MAT of validated operands with the workspace ws (at least
// mm_plan(...).total() bytes): the activation conversion, then the GEMM.
// timed = false: no timing events (the no-allocation entry point).
mi355_status mul_mat_run(mi355_context* ctx, const mi355_tensor* s0, const mi355_tensor* s1, const mi355_tensor* d,
                         const MmPlan& pl, char* ws, bool timed) {
    mi355_context* tctx = timed ? ctx : nullptr;
    const int64_t K = s0->ne[0], N = s0->ne[1], M = s1->ne[1];
    mi355_status st;
    if (pl.i8) {
        // weights -> int8 rows + scale arrays, src1 -> int8 quants + scales, then the int8-MFMA GEMM
        WRep wr = wrep_view(s0->type, N, K, s0->data);
        if (!pl.prep) {
            Timed tr(tctx, "repack_weights");
            st = hip_check(ctx, tr.done(launch_repack_weights(matw_of(s0), N, K, ws + pl.q + pl.d + pl.s, &wr,
                                                              ctx->stream)),
                           "repack_weights launch");
            if (st != MI355_STATUS_SUCCESS) return st;
        }
        const ActI8 a8 = act_i8(ws, pl, s0->type, M, K);
        {
            Timed tq8(tctx, "quantize_mmq_i8");
            st = hip_check(ctx, tq8.done(launch_quantize_mmq_i8(view_of(s1), s0->type == T_Q4_1, K, 2 * a8.nst,
                                                                reinterpret_cast<int8_t*>(ws),
                                                                reinterpret_cast<uint16_t*>(ws + pl.q),
                                                                reinterpret_cast<uint16_t*>(const_cast<void*>(a8.s)),
                                                                ctx->stream)),
                           "quantize_mmq_i8 launch");
            if (st != MI355_STATUS_SUCCESS) return st;
        }
        if (!mmq8_supported(wr, a8)) return fail(ctx, MI355_STATUS_UNSUPPORTED, "mul_mat: operands beyond the int8 kernel");
        MmqSplit sp8{pl.ks, pl.ks > 1 ? reinterpret_cast<float*>(ws + pl.q + pl.d + pl.s + pl.align) : nullptr,
                     ctx->skinny};
        sp8.cus = ctx->cus;
        const char* kname = s0->type == T_Q8_0 ? "mmq8_q8_0" : s0->type == T_Q4_0 ? "mmq8_q4_0" : "mmq8_q4_1";
        Timed tk(tctx, kname);
        return hip_check(ctx, tk.done(launch_mmq8(wr, a8, matd_of(d), nullptr, sp8, ctx->stream)), "mmq8 launch");
    }
    ActF16 a;
    if (s0->type == T_F16) {
        a.M = M;
        a.K = K;
        a.d = a.s = nullptr;
        a.dp = 0;
        if (f16_src1_direct(s1)) {
            a.q = s1->data;
            a.s1 = s1->nb[1] / 2;
            a.s2 = s1->nb[2] / 2;
            a.s3 = s1->nb[3] / 2;
        } else {
            // rows padded with zeros to a whole 16-byte chunk
            const int64_t K8 = (K + 7) & ~7;
            uint16_t* buf = reinterpret_cast<uint16_t*>(ws);
            Timed tc(tctx, "convert_f16");
            st = hip_check(ctx, tc.done(launch_convert_f16(view_of(s1), buf, K8, ctx->stream)), "convert_f16 launch");
            if (st != MI355_STATUS_SUCCESS) return st;
            a.q = buf;
            a.s1 = K8;
            a.s2 = K8 * M;
            a.s3 = K8 * M * s1->ne[2];
        }
    } else {
        st = prep_act_q8(ctx, s0, s1, pl, ws, timed, a);
        if (st != MI355_STATUS_SUCCESS) return st;
    }
    void* align_buf = pl.align ? ws + pl.q + pl.d + pl.s : nullptr;
    const MmqSplit sp{pl.ks, pl.ks > 1 ? reinterpret_cast<float*>(ws + pl.q + pl.d + pl.s + pl.align) : nullptr,
                      ctx->skinny};
    const char* kname = s0->type == T_F16 ? "mmq_f16" : s0->type == T_Q8_0 ? "mmq_q8_0" : s0->type == T_Q4_0 ? "mmq_q4_0" : "mmq_q4_1";
    Timed tq(tctx, kname);
    return hip_check(ctx, tq.done(launch_mmq(matw_of(s0), a, matd_of(d), N, s1->ne[2], s1->ne[3], nullptr, align_buf,
                                             sp, ctx->stream)),
                     "mmq launch");
}

// MUL_MAT with F32 weights: the fp32 MFMA GEMM, no workspace.
mi355_status mul_mat_f32(mi355_context* ctx, const mi355_tensor* s0, const mi355_tensor* s1, const mi355_tensor* d,
                         bool timed) {
    GemmF32Args g;
    g.W = static_cast<const float*>(s0->data);
    g.w_nb1 = s0->nb[1]; g.w_nb2 = s0->nb[2]; g.w_nb3 = s0->nb[3];
    g.X = static_cast<const float*>(s1->data);
    g.x_nb1 = s1->nb[1]; g.x_nb2 = s1->nb[2]; g.x_nb3 = s1->nb[3];
    g.D = static_cast<float*>(d->data);
    g.d_nb1 = d->nb[1]; g.d_nb2 = d->nb[2]; g.d_nb3 = d->nb[3];
    g.M = (int)s1->ne[1]; g.N = (int)s0->ne[1]; g.K = (int)s0->ne[0];
    g.ne12 = (int)s1->ne[2];
    g.r2 = (int)(s1->ne[2] / s0->ne[2]);
    g.r3 = (int)(s1->ne[3] / s0->ne[3]);
    Timed tg(timed ? ctx : nullptr, "gemm_f32");
    return hip_check(ctx, tg.done(launch_gemm_f32(g, (int)(s1->ne[2] * s1->ne[3]), ctx->stream)), "gemm_f32 launch");
}

}  // namespace

namespace mi355 {

int act_mode_for(int t) {
    switch (t) {
        case T_Q8_0:
        case T_Q4_0: return ACT_Q8;
        case T_Q4_1: return ACT_Q8S;
        case T_F16: return ACT_F16;
        default: return ACT_F32;
    }
}

int act_mode_for_weight(const mi355_tensor* w) {
    if (w->layout == MI355_LAYOUT_INT8) return w->type == T_Q4_1 ? ACT_I8S : ACT_I8;
    return act_mode_for(w->type);
}

// MUL_MAT of a prequantized operand with a fused epilogue in place of dst
// (dst [M][N] F32 is only a shape here: nothing is written to it).
mi355_status mul_mat_epi(mi355_context* ctx, const mi355_tensor* s0, const ActF16& a, const MmqEpi& e) {
    if (!s0) return fail(ctx, MI355_STATUS_INVALID_ARG, "mul_mat_epi: null weights");
    mi355_tensor d{};
    d.type = T_F32;
    d.ne[0] = s0->ne[1];
    d.ne[1] = a.M;
    d.ne[2] = d.ne[3] = 1;
    d.nb[0] = 4;
    d.nb[1] = 4 * d.ne[0];
    d.nb[2] = d.nb[3] = d.nb[1] * a.M;
    d.data = e.kind == MMQ_EPI_RESIDUAL ? static_cast<void*>(e.out) : static_cast<void*>(e.q);
    return mul_mat_act(ctx, s0, a, &d, &e);
}

// mul_mat_act for a prepared weight: the int8 kernel over an ACT_I8 / ACT_I8S operand.
mi355_status mul_mat_act_i8(mi355_context* ctx, const mi355_tensor* s0, const ActF16& a, const mi355_tensor* d,
                            const MmqEpi* epi) {
    const bool q41 = s0->type == T_Q4_1;
    if (!a.d || !a.dh || (q41 && !a.s) || a.dp != mmq_scale_pitch(a.K) || a.s1 != a.K)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "mul_mat_act: int8 operand scales missing or wrong pitch");
    mi355_tensor s1{};
    s1.type = T_F32;
    s1.ne[0] = a.K;
    s1.ne[1] = a.M;
    s1.ne[2] = s1.ne[3] = 1;
    s1.nb[0] = 4;
    s1.nb[1] = 4 * a.K;
    s1.nb[2] = s1.nb[3] = s1.nb[1] * a.M;
    s1.data = const_cast<void*>(a.q);
    mi355_status st = check_mul_mat(ctx, s0, &s1, d);
    if (st != MI355_STATUS_SUCCESS) return st;
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "mul_mat_act: null context");
    (void)hipSetDevice(ctx->device);
    const int64_t N = s0->ne[1];
    ActI8 a8;
    a8.q = a.q;
    a8.s1 = a.s1;
    a8.dl = static_cast<const uint32_t*>(a.d);
    a8.dh = static_cast<const uint32_t*>(a.dh);
    a8.s = q41 ? a.s : nullptr;
    a8.nst = a.dp / 2;
    a8.M = a.M;
    a8.K = a.K;
    const WRep wr = wrep_view(s0->type, N, a.K, s0->data);
    if (!mmq8_supported(wr, a8)) return fail(ctx, MI355_STATUS_UNSUPPORTED, "mul_mat_act: operands beyond the int8 kernel");
    const int ks = epi || dst_split_ok(d) ? mmq_ksplit(s0->type, a.M, N, a.K, 1, ctx->cus) : 1;
    const size_t part = ks > 1 ? align_up((size_t)ks * (size_t)a.M * (size_t)N * 4) : 0;
    if (part) {
        st = ensure_ws(ctx, part);
        if (st != MI355_STATUS_SUCCESS) return st;
    }
    MmqSplit sp{ks, ks > 1 ? static_cast<float*>(ctx->ws) : nullptr, ctx->skinny};
    sp.cus = ctx->cus;
    static const char* names[3][3] = {{"mmq8_q8_0", "mmq8_q8_0+residual", "mmq8_q8_0+qkv"},
                                      {"mmq8_q4_0", "mmq8_q4_0+residual", "mmq8_q4_0+qkv"},
                                      {"mmq8_q4_1", "mmq8_q4_1+residual", "mmq8_q4_1+qkv"}};
    const int ti = s0->type == T_Q8_0 ? 0 : s0->type == T_Q4_0 ? 1 : 2;
    Timed tq(ctx, names[ti][epi ? epi->kind : 0]);
    return hip_check(ctx, tq.done(launch_mmq8(wr, a8, matd_of(d), epi, sp, ctx->stream)), "mmq8 launch");
}

mi355_status mul_mat_act(mi355_context* ctx, const mi355_tensor* s0, const ActF16& a, const mi355_tensor* d,
                         const MmqEpi* epi) {
    if (!s0 || !a.q) return fail(ctx, MI355_STATUS_INVALID_ARG, "mul_mat_act: null operand");
    if (s0->layout == MI355_LAYOUT_INT8) return mul_mat_act_i8(ctx, s0, a, d, epi);
    if (s0->layout != MI355_LAYOUT_GGML) return fail(ctx, MI355_STATUS_INVALID_ARG, "mul_mat_act: unknown weight layout");
    const int mode = act_mode_for(s0->type);
    if (mode == ACT_F32) return fail(ctx, MI355_STATUS_UNSUPPORTED, "mul_mat_act: no prequantized path for type %d", s0->type);
    if (mode != ACT_F16 && (!a.d || (mode == ACT_Q8S && !a.s) || a.dp != mmq_scale_pitch(a.K)))
        return fail(ctx, MI355_STATUS_INVALID_ARG, "mul_mat_act: scales missing or wrong pitch");
    if (mode == ACT_F16 && a.K % 8 != 0)
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "mul_mat_act: F16 operands need K %% 8 == 0");
    // validate the weights and dst as mul_mat would see them with an F32 [K, M] src1
    mi355_tensor s1{};
    s1.type = T_F32;
    s1.ne[0] = a.K;
    s1.ne[1] = a.M;
    s1.ne[2] = s1.ne[3] = 1;
    s1.nb[0] = 4;
    s1.nb[1] = 4 * a.K;
    s1.nb[2] = s1.nb[3] = s1.nb[1] * a.M;
    s1.data = const_cast<void*>(a.q);
    mi355_status st = check_mul_mat(ctx, s0, &s1, d);
    if (st != MI355_STATUS_SUCCESS) return st;
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "mul_mat_act: null context");
    (void)hipSetDevice(ctx->device);
    const int64_t N = s0->ne[1];
    const size_t align = align_up(mmq_align_bytes(matw_of(s0), N, a.K));
    const int ks = epi || dst_split_ok(d) ? mmq_ksplit(s0->type, a.M, N, a.K, 1, ctx->cus) : 1;
    const size_t part = ks > 1 ? align_up((size_t)ks * (size_t)a.M * (size_t)N * 4) : 0;
    if (align + part) {
        st = ensure_ws(ctx, align + part);
        if (st != MI355_STATUS_SUCCESS) return st;
    }
    const MmqSplit sp{ks, ks > 1 ? reinterpret_cast<float*>(static_cast<char*>(ctx->ws) + align) : nullptr,
                      ctx->skinny};
    if (epi && epi->ln_next)
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "mul_mat_act: a LayerNorm hand-off needs int8-layout weights");
    static const char* names[4][3] = {{"mmq_f16", "mmq_f16+residual", "mmq_f16+qkv"},
                                      {"mmq_q8_0", "mmq_q8_0+residual", "mmq_q8_0+qkv"},
                                      {"mmq_q4_0", "mmq_q4_0+residual", "mmq_q4_0+qkv"},
                                      {"mmq_q4_1", "mmq_q4_1+residual", "mmq_q4_1+qkv"}};
    const int ti = s0->type == T_F16 ? 0 : s0->type == T_Q8_0 ? 1 : s0->type == T_Q4_0 ? 2 : 3;
    Timed tq(ctx, names[ti][epi ? epi->kind : 0]);
    if (epi)
        return hip_check(ctx, tq.done(launch_mmq_epi(matw_of(s0), a, N, *epi, align ? ctx->ws : nullptr, sp,
                                                     ctx->stream)),
                         "mmq launch");
    return hip_check(ctx, tq.done(launch_mmq(matw_of(s0), a, matd_of(d), N, 1, 1, nullptr, align ? ctx->ws : nullptr,
                                             sp, ctx->stream)),
                     "mmq launch");
}

// ggml_flash_attn_ext's shape rules plus what fattn_kernel implements.
mi355_status check_flash_attn(mi355_context* ctx, const mi355_tensor* q, const mi355_tensor* k, const mi355_tensor* v,
                              const mi355_tensor* mask, float max_bias, float logit_softcap, const mi355_tensor* dst) {
    if (!q || !k || !v || !dst || !q->data || !k->data || !v->data || !dst->data)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "flash_attn_ext: null argument");
    if (!dims_ok(q) || !dims_ok(k) || !dims_ok(v) || !dims_ok(dst))
        return fail(ctx, MI355_STATUS_INVALID_ARG, "flash_attn_ext: negative ne/nb or not the ggml layout");
    if (mask || max_bias != 0.0f || logit_softcap != 0.0f)
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "flash_attn_ext: mask, ALiBi and softcap not supported");
    // ggml_flash_attn_ext shape rules
    const int64_t D = q->ne[0];
    if (k->ne[0] != D || v->ne[1] != k->ne[1] || q->ne[3] != k->ne[3] || q->ne[3] != v->ne[3])
        return fail(ctx, MI355_STATUS_INVALID_ARG, "flash_attn_ext: q/k/v shapes do not match");
    if (k->ne[2] <= 0 || v->ne[2] <= 0 || q->ne[2] % k->ne[2] != 0 || q->ne[2] % v->ne[2] != 0)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "flash_attn_ext: heads not divisible by kv heads");
    if (dst->type != T_F32 || dst->ne[0] != v->ne[0] || dst->ne[1] != q->ne[2] || dst->ne[2] != q->ne[1] ||
        dst->ne[3] != q->ne[3])
        return fail(ctx, MI355_STATUS_INVALID_ARG, "flash_attn_ext: dst must be F32 [Dv, n_head, n_q, batch]");
    if (dst->nb[0] != 4 || dst->nb[1] != 4 * dst->ne[0] || dst->nb[2] != dst->nb[1] * dst->ne[1] ||
        dst->nb[3] != dst->nb[2] * dst->ne[2])
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "flash_attn_ext: dst must be contiguous");
    if (v->ne[0] != D || !(D == 64 || D == 96 || D == 128))
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "flash_attn_ext: head size %lld (supported: D = Dv in 64, 96, 128)",
                    (long long)D);
    const mi355_tensor* ops[3] = {q, k, v};
    for (const mi355_tensor* t : ops) {
        if (t->type != T_F32 && t->type != T_F16)
            return fail(ctx, MI355_STATUS_UNSUPPORTED, "flash_attn_ext: q/k/v must be F32 or F16");
        if (t->nb[0] != type_size(t->type))
            return fail(ctx, MI355_STATUS_UNSUPPORTED, "flash_attn_ext: rows must be contiguous (nb[0] = type size)");
        if (((reinterpret_cast<uintptr_t>(t->data) | (uintptr_t)t->nb[1] | (uintptr_t)t->nb[2] | (uintptr_t)t->nb[3]) &
             3) != 0)
            return fail(ctx, MI355_STATUS_UNSUPPORTED, "flash_attn_ext: rows must be 4-byte aligned");
    }
    if (k->type != v->type) return fail(ctx, MI355_STATUS_UNSUPPORTED, "flash_attn_ext: k and v must share a type");
    if (q->ne[1] > INT32_MAX || k->ne[1] > INT32_MAX || q->ne[2] > 65535 || q->ne[3] > 65535)
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "flash_attn_ext: sizes beyond the launch limits");
    return MI355_STATUS_SUCCESS;
}

mi355_status flash_attn_act(mi355_context* ctx, const mi355_tensor* q, const mi355_tensor* k, const mi355_tensor* v,
                            const mi355_tensor* mask, float scale, float max_bias, float logit_softcap,
                            const mi355_tensor* dst, const ActOut* op) {
    const mi355_status cs = check_flash_attn(ctx, q, k, v, mask, max_bias, logit_softcap, dst);
    if (cs != MI355_STATUS_SUCCESS) return cs;
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "flash_attn_ext: null context");
    const int64_t D = q->ne[0];
    FaArgs a;
    a.q = static_cast<const char*>(q->data);
    a.k = static_cast<const char*>(k->data);
    a.v = static_cast<const char*>(v->data);
    a.dst = static_cast<float*>(dst->data);
    a.q_nb1 = q->nb[1]; a.q_nb2 = q->nb[2]; a.q_nb3 = q->nb[3];
    a.k_nb1 = k->nb[1]; a.k_nb2 = k->nb[2]; a.k_nb3 = k->nb[3];
    a.v_nb1 = v->nb[1]; a.v_nb2 = v->nb[2]; a.v_nb3 = v->nb[3];
    a.nq = (int)q->ne[1];
    a.nkv = (int)k->ne[1];
    a.nh = (int)q->ne[2];
    a.rk2 = (int)(q->ne[2] / k->ne[2]);
    a.rv2 = (int)(q->ne[2] / v->ne[2]);
    const float c = fabsf(scale) * 1.44269504088896340736f;
    a.c = c > 1e-30f ? c : 1e-30f;  // keeps masked (-inf) scores at weight 0 when scale is 0
    a.negq = scale < 0.0f;
    a.out = ActOut{ACT_F32, nullptr, nullptr, nullptr, nullptr, 0};
    if (op) {
        const int64_t K = q->ne[2] * D;
        if (op->mode == ACT_F32 || !op->q ||
            (op->mode != ACT_F16 && (!op->d || (act_has_sums(op->mode) && !op->s) || (op->mode >= ACT_I8 && !op->dh) ||
                                     op->dp != mmq_scale_pitch(K))))
            return fail(ctx, MI355_STATUS_INVALID_ARG, "flash_attn_ext: bad operand output");
        a.out = *op;
    }
    (void)hipSetDevice(ctx->device);
    a.kv_split = fattn_kv_split(a.nq, a.nkv, a.nh, (int)q->ne[3], ctx->cus);
    a.kv_chunk = 0;
    a.part = nullptr;
    if (a.kv_split > 1) {
        const int ntile = (a.nkv + 63) / 64, per = (ntile + a.kv_split - 1) / a.kv_split;
        a.kv_chunk = per * 64;
        a.kv_split = (ntile + per - 1) / per;  // no empty range
        if (a.kv_split > 1) {
            const mi355_status s2 = ensure_ws(ctx, fattn_part_bytes((int)D, a.nq, a.nh, (int)q->ne[3], a.kv_split));
            if (s2 != MI355_STATUS_SUCCESS) return s2;
            a.part = static_cast<float*>(ctx->ws);
        }
    }
    if (a.kv_split <= 1) {
        a.kv_split = 1;
        a.kv_chunk = a.nkv;
    }
    Timed tf(ctx, "flash_attn_ext");
    return hip_check(ctx, tf.done(launch_fattn(a, (int)D, q->type == T_F32, k->type == T_F32, (int)q->ne[3], ctx->stream)),
                     "flash_attn_ext launch");
}

}  // namespace mi355

extern "C" {

const char* mi355_status_to_string(mi355_status s) {
    switch (s) {
        case MI355_STATUS_SUCCESS: return "GGML status: success";
        case MI355_STATUS_FAILED: return "GGML status: error (operation failed)";
        case MI355_STATUS_ALLOC_FAILED: return "GGML status: error (failed to allocate memory)";
        case MI355_STATUS_ABORTED: return "GGML status: warning (operation aborted)";
        case MI355_STATUS_UNSUPPORTED: return "MI355 status: error (operation not supported)";
        case MI355_STATUS_INVALID_ARG: return "MI355 status: error (invalid argument)";
        default: return "MI355 status: unknown";
    }
}

const char* mi355_last_error(const mi355_context* ctx) {
    return ctx ? ctx->last_error.c_str() : g_noctx_error.c_str();
}

int mi355_abi_version(void) { return MI355_ABI_VERSION; }

mi355_status mi355_context_create(int device, void* stream, mi355_context** out) {
    if (!out) return fail(nullptr, MI355_STATUS_INVALID_ARG, "context_create: out is null");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) return fail(nullptr, MI355_STATUS_FAILED, "no HIP device: %s", hipGetErrorString(e));
    if (device < 0 || device >= n) return fail(nullptr, MI355_STATUS_INVALID_ARG, "device %d out of range", device);
    e = hipSetDevice(device);
    if (e != hipSuccess) return fail(nullptr, MI355_STATUS_FAILED, "hipSetDevice: %s", hipGetErrorString(e));
    mi355_context* ctx = new mi355_context();
    ctx->device = device;
    ctx->stream = static_cast<hipStream_t>(stream);  // NULL: the device's default stream
    ctx->cus = device_cus(device);
    // the no-allocation entry point's fixed scratch on this device (resolved once per device)
    if (noalloc_scratch_init(ctx) != MI355_STATUS_SUCCESS) {
        ctx->scratch_error = ctx->last_error;
        ctx->last_error.clear();
    }
    *out = ctx;
    return MI355_STATUS_SUCCESS;
}

void mi355_context_free(mi355_context* ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    noalloc_release(ctx);
    mi355_profile_reset(ctx);
    if (ctx->ws) (void)hipFree(ctx->ws);
    if (ctx->enc) (void)hipFree(ctx->enc);
    if (ctx->neck) (void)hipFree(ctx->neck);
    delete ctx;
}

mi355_status mi355_synchronize(mi355_context* ctx) {
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "synchronize: null context");
    (void)hipSetDevice(ctx->device);
    return hip_check(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

mi355_status mi355_reserve_workspace(mi355_context* ctx, size_t bytes) {
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "reserve_workspace: null context");
    (void)hipSetDevice(ctx->device);
    return ensure_ws(ctx, bytes);
}

size_t mi355_mul_mat_workspace_size(const mi355_tensor* s0, const mi355_tensor* s1) {
    if (!s0 || !s1) return 0;
    if (s0->type != T_F32 && s0->type != T_F16 && s0->type != T_Q8_0 && s0->type != T_Q4_0 && s0->type != T_Q4_1)
        return 0;
    int dev = 0;
    (void)hipGetDevice(&dev);
    // the most any MUL_MAT route (mi355_context_set_mmq_kernel) needs
    const int cus = device_cus(dev);
    size_t bytes = 0;
    for (int k : {MI355_MMQ_F16, MI355_MMQ_INT8, MI355_MMQ_AUTO}) bytes = std::max(bytes, mm_plan(s0, s1, cus, true, k).total());
    return bytes;
}

size_t mi355_weight_prepared_nbytes(const mi355_tensor* w) {
    if (!w || !dims_ok(w) || !(w->type == T_Q8_0 || w->type == T_Q4_0 || w->type == T_Q4_1) || w->ne[2] != 1 ||
        w->ne[3] != 1 || w->ne[0] % 32 != 0)
        return 0;
    return wrep_bytes(w->type, w->ne[1], w->ne[0]);
}

mi355_status mi355_weight_prepare(mi355_context* ctx, const mi355_tensor* w, void* dst, size_t dst_size,
                                  mi355_tensor* out) {
    if (!w || !dst || !out) return fail(ctx, MI355_STATUS_INVALID_ARG, "weight_prepare: null argument");
    const size_t need = mi355_weight_prepared_nbytes(w);
    if (need == 0) return fail(ctx, MI355_STATUS_INVALID_ARG, "weight_prepare: not a 2-D Q8_0/Q4_0/Q4_1 ggml weight");
    if (!w->data) return fail(ctx, MI355_STATUS_INVALID_ARG, "weight_prepare: null weight data");
    if (w->nb[0] != type_size(w->type) || w->nb[1] < row_size(w->type, w->ne[0]) ||
        (reinterpret_cast<uintptr_t>(w->data) & 1) || (w->nb[1] & 1))
        return fail(ctx, MI355_STATUS_INVALID_ARG, "weight_prepare: rows must be contiguous and 2-byte aligned");
    if ((reinterpret_cast<uintptr_t>(dst) & 255) != 0)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "weight_prepare: dst must be 256-byte aligned");
    if (dst_size < need) return fail(ctx, MI355_STATUS_INVALID_ARG, "weight_prepare: dst holds %zu bytes, %zu needed", dst_size, need);
    const char* wb = static_cast<const char*>(w->data);
    const char* db = static_cast<const char*>(dst);
    const size_t wspan = (size_t)((w->ne[1] - 1) * w->nb[1] + row_size(w->type, w->ne[0]));
    if (w->ne[1] > 0 && db < wb + wspan && wb < db + need)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "weight_prepare: dst overlaps the weight");
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "weight_prepare: null context");
    (void)hipSetDevice(ctx->device);
    *out = *w;
    out->layout = MI355_LAYOUT_INT8;
    out->nb[1] = row_size(w->type, w->ne[0]);
    out->nb[2] = out->nb[3] = out->nb[1] * w->ne[1];
    out->data = dst;
    if (w->ne[0] == 0 || w->ne[1] == 0) return MI355_STATUS_SUCCESS;
    WRep wr;
    Timed t(ctx, "repack_weights");
    return hip_check(ctx, t.done(launch_repack_weights(matw_of(w), w->ne[1], w->ne[0], dst, &wr, ctx->stream)),
                     "repack_weights launch");
}

int mi355_supports_mul_mat(const mi355_tensor* s0, const mi355_tensor* s1, const mi355_tensor* d) {
    return check_mul_mat(nullptr, s0, s1, d) == MI355_STATUS_SUCCESS;
}

mi355_status mi355_mul_mat(mi355_context* ctx, const mi355_tensor* s0, const mi355_tensor* s1,
                           const mi355_tensor* d) {
    mi355_status st = check_mul_mat(ctx, s0, s1, d);
    if (st != MI355_STATUS_SUCCESS) return st;
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "mul_mat: null context");
    (void)hipSetDevice(ctx->device);
    if (s0->ne[0] == 0 || s0->ne[1] == 0 || s1->ne[1] == 0 || s1->ne[2] * s1->ne[3] == 0) return MI355_STATUS_SUCCESS;
    if (s0->type == T_F32) return mul_mat_f32(ctx, s0, s1, d, true);
    const MmPlan pl = mm_plan(s0, s1, ctx->cus, dst_split_ok(d), ctx->mmq_kernel);
    st = ensure_ws(ctx, pl.total());
    if (st != MI355_STATUS_SUCCESS) return st;
    return mul_mat_run(ctx, s0, s1, d, pl, static_cast<char*>(ctx->ws), true);
}

mi355_status mi355_mul_mat_noalloc(mi355_context* ctx, const mi355_tensor* s0, const mi355_tensor* s1,
                                   const mi355_tensor* d) {
    mi355_status st = check_mul_mat(ctx, s0, s1, d);
    if (st != MI355_STATUS_SUCCESS) return st;
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "mul_mat_noalloc: null context");
    (void)hipSetDevice(ctx->device);
    if (s0->ne[0] == 0 || s0->ne[1] == 0 || s1->ne[1] == 0 || s1->ne[2] * s1->ne[3] == 0) return MI355_STATUS_SUCCESS;
    if (s0->type == T_F32) return mul_mat_f32(ctx, s0, s1, d, false);
    if (!ctx->scratch)
        return fail(ctx, MI355_STATUS_FAILED, "mul_mat_noalloc: no static scratch on device %d (%s)", ctx->device,
                    ctx->scratch_error.c_str());
    const MmPlan pl = mm_plan(s0, s1, ctx->cus, dst_split_ok(d), ctx->mmq_kernel);
    if (pl.total() > MI355_NOALLOC_SCRATCH_BYTES)
        return fail(ctx, MI355_STATUS_UNSUPPORTED,
                    "mul_mat_noalloc: these operands need %zu bytes of scratch, the static scratch holds %zu",
                    pl.total(), (size_t)MI355_NOALLOC_SCRATCH_BYTES);
    return noalloc_run(ctx, [&] { return mul_mat_run(ctx, s0, s1, d, pl, static_cast<char*>(ctx->scratch), false); });
}

mi355_status mi355_mul_mat_block_dots(mi355_context* ctx, const mi355_tensor* s0, const mi355_tensor* s1,
                                      int32_t* isums) {
    if (!s0 || !s1 || !isums) return fail(ctx, MI355_STATUS_INVALID_ARG, "block_dots: null argument");
    if (s0->type == T_F16 || s0->type == T_F32)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "block_dots: src0 must be a block type");
    mi355_tensor d{};
    d.type = T_F32;
    d.ne[0] = s0->ne[1];
    d.ne[1] = s1->ne[1];
    d.ne[2] = s1->ne[2];
    d.ne[3] = s1->ne[3];
    d.nb[0] = 4;
    d.nb[1] = 4 * d.ne[0];
    d.nb[2] = d.nb[1] * d.ne[1];
    d.nb[3] = d.nb[2] * d.ne[2];
    d.data = isums;  // shape check only; the kernel writes isums
    mi355_status st = check_mul_mat(ctx, s0, s1, &d);
    if (st != MI355_STATUS_SUCCESS) return st;
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "block_dots: null context");
    (void)hipSetDevice(ctx->device);
    const MmPlan pl = mm_plan(s0, s1, ctx->cus, false, ctx->mmq_kernel);
    st = ensure_ws(ctx, pl.total());
    if (st != MI355_STATUS_SUCCESS) return st;
    if (pl.i8) {
        char* ws = static_cast<char*>(ctx->ws);
        const int64_t K = s0->ne[0], M = s1->ne[1];
        WRep wr = wrep_view(s0->type, s0->ne[1], K, s0->data);
        if (!pl.prep) {
            st = hip_check(ctx, launch_repack_weights(matw_of(s0), s0->ne[1], K, ws + pl.q + pl.d + pl.s, &wr,
                                                      ctx->stream),
                           "repack_weights launch");
            if (st != MI355_STATUS_SUCCESS) return st;
        }
        const ActI8 a8 = act_i8(ws, pl, s0->type, M, K);
        st = hip_check(ctx, launch_quantize_mmq_i8(view_of(s1), s0->type == T_Q4_1, K, 2 * a8.nst, reinterpret_cast<int8_t*>(ws),
                                                   reinterpret_cast<uint16_t*>(ws + pl.q),
                                                   reinterpret_cast<uint16_t*>(const_cast<void*>(a8.s)), ctx->stream),
                       "quantize_mmq_i8 launch");
        if (st != MI355_STATUS_SUCCESS) return st;
        return hip_check(ctx, launch_mmq8(wr, a8, MatD{nullptr, 0, 0, 0}, nullptr, MmqSplit{1, nullptr}, ctx->stream,
                                          isums),
                         "mmq8(dots) launch");
    }
    ActF16 a;
    st = prep_act_q8(ctx, s0, s1, pl, static_cast<char*>(ctx->ws), true, a);
    if (st != MI355_STATUS_SUCCESS) return st;
    void* align_buf = pl.align ? static_cast<char*>(ctx->ws) + pl.q + pl.d + pl.s : nullptr;
    return hip_check(ctx, launch_mmq(matw_of(s0), a, matd_of(&d), s0->ne[1], s1->ne[2], s1->ne[3], isums, align_buf,
                                     MmqSplit{1, nullptr}, ctx->stream),
                     "mmq(dots) launch");
}

mi355_status mi355_quantize_rows(mi355_context* ctx, int type, int variant, const mi355_tensor* src, void* dst) {
    if (!src || !src->data || !dst) return fail(ctx, MI355_STATUS_INVALID_ARG, "quantize_rows: null argument");
    if (!dims_ok(src)) return fail(ctx, MI355_STATUS_INVALID_ARG, "quantize_rows: negative ne/nb or not the ggml layout");
    if (src->type != T_F32) return fail(ctx, MI355_STATUS_UNSUPPORTED, "quantize_rows: src must be F32");
    if (!(type == T_Q8_0 || type == T_Q8_1 || type == T_F16))
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "quantize_rows: type %d not supported", type);
    if (variant != MI355_ACT_X86 && variant != MI355_ACT_REF)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "quantize_rows: bad variant %d", variant);
    if (src->ne[0] % blck(type) != 0)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "quantize_rows: ne0 not a multiple of the block size");
    if (type == T_Q8_1 && (reinterpret_cast<uintptr_t>(dst) & 3))
        return fail(ctx, MI355_STATUS_INVALID_ARG, "quantize_rows: q8_1 dst must be 4-byte aligned");
    if (reinterpret_cast<uintptr_t>(dst) & 1)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "quantize_rows: dst must be 2-byte aligned");
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "quantize_rows: null context");
    (void)hipSetDevice(ctx->device);
    Timed tq(ctx, "quantize_rows");
    return hip_check(ctx, tq.done(launch_quantize_ggml(view_of(src), type, variant == MI355_ACT_REF, dst, ctx->stream)),
                     "quantize launch");
}

mi355_status mi355_quantize_weights(mi355_context* ctx, int type, const mi355_tensor* src, void* dst) {
    if (!src || !src->data || !dst) return fail(ctx, MI355_STATUS_INVALID_ARG, "quantize_weights: null argument");
    if (!dims_ok(src)) return fail(ctx, MI355_STATUS_INVALID_ARG, "quantize_weights: negative ne/nb or not the ggml layout");
    if (src->type != T_F32 && src->type != T_F16)
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "quantize_weights: src must be F32 or F16");
    if (!(type == T_Q8_0 || type == T_Q4_0 || type == T_Q4_1))
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "quantize_weights: type %d not supported", type);
    if (src->ne[0] % 32 != 0)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "quantize_weights: ne0 not a multiple of the block size");
    const uintptr_t sa = reinterpret_cast<uintptr_t>(src->data) | (uintptr_t)src->nb[0] | (uintptr_t)src->nb[1] |
                         (uintptr_t)src->nb[2] | (uintptr_t)src->nb[3];
    if ((sa & (src->type == T_F32 ? 3 : 1)) || (reinterpret_cast<uintptr_t>(dst) & 1))
        return fail(ctx, MI355_STATUS_INVALID_ARG, "quantize_weights: src elements and dst must be naturally aligned");
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "quantize_weights: null context");
    (void)hipSetDevice(ctx->device);
    Timed tq(ctx, "quantize_weights");
    return hip_check(ctx, tq.done(launch_quantize_ggml(view_of(src), type, true, dst, ctx->stream)),
                     "quantize_weights launch");
}

int mi355_supports_flash_attn_ext(const mi355_tensor* q, const mi355_tensor* k, const mi355_tensor* v,
                                  const mi355_tensor* mask, float max_bias, float logit_softcap,
                                  const mi355_tensor* dst) {
    return mi355::check_flash_attn(nullptr, q, k, v, mask, max_bias, logit_softcap, dst) == MI355_STATUS_SUCCESS;
}

int mi355_supports_soft_max_ext(const mi355_tensor* src, const mi355_tensor* mask, float max_bias,
                                const mi355_tensor* dst) {
    return check_soft_max(nullptr, src, mask, max_bias, dst) == MI355_STATUS_SUCCESS;
}

mi355_status mi355_soft_max_ext(mi355_context* ctx, const mi355_tensor* src, const mi355_tensor* mask, float scale,
                                float max_bias, const mi355_tensor* dst) {
    const mi355_status cs = check_soft_max(ctx, src, mask, max_bias, dst);
    if (cs != MI355_STATUS_SUCCESS) return cs;
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "soft_max: null context");
    (void)hipSetDevice(ctx->device);
    Timed ts(ctx, "soft_max");
    return hip_check(ctx, ts.done(launch_soft_max(view_of(src), scale, static_cast<char*>(dst->data), dst->nb, ctx->stream)),
                     "soft_max launch");
}

mi355_status mi355_context_set_fusion(mi355_context* ctx, int enable) {
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "set_fusion: null context");
    ctx->fuse = enable != 0;
    return MI355_STATUS_SUCCESS;
}

mi355_status mi355_context_set_mmq_kernel(mi355_context* ctx, int kernel) {
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "set_mmq_kernel: null context");
    if (kernel != MI355_MMQ_F16 && kernel != MI355_MMQ_INT8 && kernel != MI355_MMQ_AUTO)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "set_mmq_kernel: unknown kernel %d", kernel);
    ctx->mmq_kernel = kernel;
    return MI355_STATUS_SUCCESS;
}

mi355_status mi355_context_set_skinny(mi355_context* ctx, int enable) {
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "set_skinny: null context");
    ctx->skinny = enable != 0;
    return MI355_STATUS_SUCCESS;
}

mi355_status mi355_profile_enable(mi355_context* ctx, int enable) {
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "profile_enable: null context");
    ctx->prof = enable != 0;
    return MI355_STATUS_SUCCESS;
}

int mi355_profile_collect(mi355_context* ctx) {
    if (!ctx) return (int)fail(nullptr, MI355_STATUS_INVALID_ARG, "profile_collect: null context");
    (void)hipSetDevice(ctx->device);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return (int)hip_check(ctx, e, "hipStreamSynchronize");
    for (auto& p : ctx->pending) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
            auto& t = ctx->totals[p.name];
            t.first += 1;
            t.second += ms;
        }
        (void)hipEventDestroy(p.a);
        (void)hipEventDestroy(p.b);
    }
    ctx->pending.clear();
    ctx->names.clear();
    for (auto& kv : ctx->totals) ctx->names.push_back(kv.first);
    return (int)ctx->names.size();
}

mi355_status mi355_profile_get(mi355_context* ctx, int index, const char** name, int* launches, double* total_ms) {
    if (!ctx || index < 0 || index >= (int)ctx->names.size())
        return fail(ctx, MI355_STATUS_INVALID_ARG, "profile_get: bad index %d", index);
    const auto& t = ctx->totals[ctx->names[index]];
    if (name) *name = ctx->names[index].c_str();
    if (launches) *launches = t.first;
    if (total_ms) *total_ms = t.second;
    return MI355_STATUS_SUCCESS;
}

void mi355_profile_reset(mi355_context* ctx) {
    if (!ctx) return;
    for (auto& p : ctx->pending) {
        (void)hipEventDestroy(p.a);
        (void)hipEventDestroy(p.b);
    }
    ctx->pending.clear();
    ctx->totals.clear();
    ctx->names.clear();
}

mi355_status mi355_flash_attn_ext(mi355_context* ctx, const mi355_tensor* q, const mi355_tensor* k,
                                  const mi355_tensor* v, const mi355_tensor* mask, float scale, float max_bias,
                                  float logit_softcap, const mi355_tensor* dst) {
    return mi355::flash_attn_act(ctx, q, k, v, mask, scale, max_bias, logit_softcap, dst, nullptr);
}

}  // extern "C"
