// SAM2 Hiera image encoder on the MI355X backend: the graph of
// sam2_build_hiera_graph (sam3.cpp:4466-4535) node group by node group.  Per
// block (sam2_hiera_block_forward, sam3.cpp:4299-4461):
//
//   xn   = LN1(x)  [window order over the zero-padded grid for windowed blocks]
//   sc   = x | maxpool(x) | [maxpool](mul_mat(dim_proj_w, LN1(x)) + dim_proj_b)
//   qkv  = mul_mat(qkv_w, xn)
//   q,k,v = split(qkv + qkv_b), q max-pooled 2x2 inside each window  -> fp16
//   attn = flash_attn_ext(q, k, v, 1/sqrt(HD))
//   x'   = sc + window_unpartition(mul_mat(proj_w, attn) + proj_b)
//   x'   = x' + (mul_mat(fc2_w, gelu(mul_mat(fc1_w, LN2(x')) + fc1_b)) + fc2_b)
//
// MUL_MAT and FLASH_ATTN_EXT go through the backend's own entry points; the
// memory-bound steps are the fused passes of hiera.hip.  For quantized and F16
// weights the passes feeding a MUL_MAT (LN1 -> qkv and dim_proj, LN2 -> fc1,
// bias+GELU -> fc2) write the GEMM's activation operand (Q8 quants + scales,
// or F16 rows) directly instead of f32 rows that MUL_MAT would quantize again.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "context.h"

using namespace mi355;

namespace {

struct Info {
    int dim_in, dim_out, heads, ws, qs, stage;
};

// sam2_precompute_hiera_metadata (sam3.cpp:1680-1746): the window size lags a
// block behind the stage (a stage's first block keeps the previous stage's
// window), and Q pooling happens at the first block of stages 1..q_pool.
bool block_infos(const mi355_hiera_hparams* hp, std::vector<Info>& out) {
    out.clear();
    int total = 0, ends[4];
    for (int s = 0; s < 4; ++s) {
        if (hp->stages[s] < 0) return false;
        total += hp->stages[s];
        ends[s] = total - 1;
    }
    std::vector<int> qpool_blocks;
    for (int s = 0; s < 3 && (int)qpool_blocks.size() < hp->q_pool; ++s) qpool_blocks.push_back(ends[s] + 1);
    int cur = 0, dim = hp->embed_dim, heads = hp->num_heads;
    for (int i = 0; i < total; ++i) {
        Info b;
        int ws = hp->window_spec[cur];
        for (int g = 0; g < hp->n_global && g < 8; ++g)
            if (hp->global_idx[g] == i) ws = 0;
        b.ws = ws;
        int dim_out = dim;
        if (i > 0 && i - 1 == ends[cur]) {
            dim_out = dim * 2;
            heads *= 2;
            ++cur;
        }
        b.stage = cur;
        b.dim_in = dim;
        b.dim_out = dim_out;
        b.heads = heads;
        b.qs = std::find(qpool_blocks.begin(), qpool_blocks.end(), i) != qpool_blocks.end();
        out.push_back(b);
        dim = dim_out;
    }
    return true;
}

int cdiv(int a, int b) { return (a + b - 1) / b; }

// activation buffers of one block (or their maxima over the backbone)
struct Sizes {
    size_t xw = 0, xn = 0, dp = 0, sc = 0, qkv = 0, q = 0, kv = 0, att = 0, p = 0, h = 0, f = 0, x = 0, cols = 0, w32 = 0,
           a0 = 0, a1 = 0, a2 = 0;
    static constexpr int kFields = 17;
    void max_with(const Sizes& o) {
        size_t* a = &xw;
        const size_t* b = &o.xw;
        for (int i = 0; i < kFields; ++i) a[i] = std::max(a[i], b[i]);
    }
};

// a GEMM activation operand of rows x K in one buffer: q [rows][K] fp16 (or
// int8), then the scales (fp16 [rows][dp], or the int8 operand's dl and dh
// dword arrays [rows][dp / 2] each), then s [rows][dp] fp16
struct Operand {
    uint16_t *q, *d, *s;
    uint32_t* dh;
};
size_t operand_bytes(size_t rows, size_t K, Operand* o = nullptr, char* base = nullptr) {
    const size_t dp = (size_t)mmq_scale_pitch((int64_t)K);
    const size_t qb = align_up(rows * K * 2), db = align_up(rows * dp * 4), sb = align_up(rows * dp * 2);
    if (o && base) {
        o->q = reinterpret_cast<uint16_t*>(base);
        o->d = reinterpret_cast<uint16_t*>(base + qb);
        o->dh = reinterpret_cast<uint32_t*>(base + qb) + rows * (dp / 2);
        o->s = reinterpret_cast<uint16_t*>(base + qb + db);
    }
    return qb + db + sb;
}

Sizes block_sizes(const Info& b, int S) {
    Sizes z;
    const size_t Cin = b.dim_in, Cout = b.dim_out;
    const int S2 = b.qs ? S / 2 : S;
    size_t rows = (size_t)S * S, nq = rows;
    if (b.ws > 0) {
        const size_t nw = (size_t)cdiv(S, b.ws) * cdiv(S, b.ws);
        rows = nw * b.ws * b.ws;
        nq = b.qs ? nw * (b.ws / 2) * (b.ws / 2) : rows;
        z.xw = rows * Cin * 4;
    }
    z.xn = (size_t)S * S * std::max(Cin, Cout) * 4;
    if (Cin != Cout) z.dp = (size_t)S * S * Cout * 4;
    if (Cin != Cout || b.qs) z.sc = (size_t)S2 * S2 * Cout * 4;
    z.qkv = rows * 3 * Cout * 4;
    z.q = nq * Cout * 2;
    z.kv = rows * Cout * 2;
    z.att = nq * Cout * 4;
    z.p = nq * Cout * 4;
    z.h = (size_t)S2 * S2 * 4 * Cout * 4;
    z.f = (size_t)S2 * S2 * Cout * 4;
    z.x = (size_t)S * S * std::max(Cin, Cout) * 4;
    // a0: LN1 in attention order, attention output and LN2 operands;
    // a1: LN1 in image order; a2: the GELU output (fc2's operand)
    z.a0 = std::max({operand_bytes(rows, Cin), operand_bytes(nq, Cout), operand_bytes((size_t)S2 * S2, Cout),
                     operand_bytes((size_t)S2 * S2, 4 * Cout)});
    z.a2 = operand_bytes((size_t)S2 * S2, 4 * Cout);
    if (Cin != Cout) {
        z.a1 = operand_bytes((size_t)S * S, Cin);
        z.xw = std::max(z.xw, (size_t)S * S * Cin * 4);  // dim_proj's f32 LN1 rows next to a fused qkv operand
    }
    return z;
}

struct Bufs {
    float *xw, *xn, *dp, *sc, *qkv, *att, *p, *h, *f, *x0, *x1, *cols, *w32;
    _Float16 *q, *k, *v;
    char *a0, *a1, *a2;
};

size_t layout(const Sizes& z, char* base, Bufs* b) {
    const size_t parts[19] = {z.xw, z.xn, z.dp, z.sc, z.qkv, z.att, z.p,  z.h,  z.f,  z.x,
                              z.x,  z.cols, z.w32, z.q, z.kv, z.kv, z.a0, z.a1, z.a2};
    size_t off[19], o = 0;
    for (int i = 0; i < 19; ++i) {
        off[i] = o;
        o += align_up(std::max(parts[i], (size_t)256));
    }
    if (b && base) {
        float** fp[13] = {&b->xw, &b->xn, &b->dp, &b->sc, &b->qkv, &b->att, &b->p, &b->h, &b->f, &b->x0, &b->x1, &b->cols, &b->w32};
        for (int i = 0; i < 13; ++i) *fp[i] = reinterpret_cast<float*>(base + off[i]);
        b->q = reinterpret_cast<_Float16*>(base + off[13]);
        b->k = reinterpret_cast<_Float16*>(base + off[14]);
        b->v = reinterpret_cast<_Float16*>(base + off[15]);
        b->a0 = base + off[16];
        b->a1 = base + off[17];
        b->a2 = base + off[18];
    }
    return o;
}

mi355_status check_hp(mi355_context* ctx, const mi355_hiera_hparams* hp, std::vector<Info>& infos) {
    if (!hp) return fail(ctx, MI355_STATUS_INVALID_ARG, "hiera: null hparams");
    if (hp->img_size <= 0 || hp->img_size % 4 != 0 || hp->embed_dim <= 0 || hp->num_heads <= 0 || hp->q_pool < 0 ||
        hp->n_global < 0 || hp->n_global > 8 || !(hp->eps >= 0.0f))
        return fail(ctx, MI355_STATUS_INVALID_ARG, "hiera: bad hparams");
    for (int s = 0; s < 4; ++s)
        if (hp->window_spec[s] < 0) return fail(ctx, MI355_STATUS_INVALID_ARG, "hiera: negative window size");
    if (!block_infos(hp, infos) || infos.empty()) return fail(ctx, MI355_STATUS_INVALID_ARG, "hiera: bad stage table");
    int S = hp->img_size / 4;
    for (size_t i = 0; i < infos.size(); ++i) {
        const Info& b = infos[i];
        if (b.dim_out % b.heads != 0) return fail(ctx, MI355_STATUS_INVALID_ARG, "hiera: width not divisible by heads");
        const int HD = b.dim_out / b.heads;
        if (!(HD == 64 || HD == 96 || HD == 128))
            return fail(ctx, MI355_STATUS_UNSUPPORTED, "hiera: head size %d (supported: 64, 96, 128)", HD);
        if (b.dim_in % 4 != 0 || b.dim_out % 4 != 0 || b.dim_out > 2048)
            return fail(ctx, MI355_STATUS_UNSUPPORTED, "hiera: widths must be multiples of 4, <= 2048");
        if (b.qs && (S % 2 != 0 || (b.ws > 0 && b.ws % 2 != 0)))
            return fail(ctx, MI355_STATUS_UNSUPPORTED, "hiera: Q pooling needs even grid and window");
        if (b.qs && b.ws == 0) return fail(ctx, MI355_STATUS_UNSUPPORTED, "hiera: Q pooling in a global block");
        if (b.qs) S /= 2;
    }
    return MI355_STATUS_SUCCESS;
}

// The patch embedding's 147 im2col columns (c, ky, kx) and weight rows at a zero-padded
// pitch of 148 floats: the fp32 MFMA GEMM then takes them in whole 16-byte chunks (the zero
// column adds exact zeros to every sum)
constexpr int PATCH_KP = 148;

Sizes all_sizes(const mi355_hiera_hparams* hp, const std::vector<Info>& infos) {
    Sizes z;
    int S = hp->img_size / 4;
    for (const Info& b : infos) {
        z.max_with(block_sizes(b, S));
        if (b.qs) S /= 2;
    }
    const size_t S0 = (size_t)(hp->img_size / 4);
    z.cols = S0 * S0 * PATCH_KP * 4;
    z.w32 = (size_t)PATCH_KP * hp->embed_dim * 4;
    z.x = std::max(z.x, S0 * S0 * (size_t)hp->embed_dim * 4);
    return z;
}

mi355_tensor tensor_on(const void* p, int type, int64_t ne0, int64_t ne1, int64_t ne2 = 1, int64_t ne3 = 1) {
    mi355_tensor t{};
    t.type = type;
    t.ne[0] = ne0;
    t.ne[1] = ne1;
    t.ne[2] = ne2;
    t.ne[3] = ne3;
    t.nb[0] = type == T_F32 ? 4 : 2;
    t.nb[1] = t.nb[0] * ne0;
    t.nb[2] = t.nb[1] * ne1;
    t.nb[3] = t.nb[2] * ne2;
    t.data = const_cast<void*>(p);
    return t;
}

mi355_status get_bufs(mi355_context* ctx, const mi355_hiera_hparams* hp, const std::vector<Info>& infos, Bufs* b) {
    const Sizes z = all_sizes(hp, infos);
    mi355_status st = ensure_buffer(ctx, &ctx->enc, &ctx->enc_size, layout(z, nullptr, nullptr));
    if (st != MI355_STATUS_SUCCESS) return st;
    layout(z, static_cast<char*>(ctx->enc), b);
    return MI355_STATUS_SUCCESS;
}

#define TRY(e)                                     \
    do {                                           \
        mi355_status st_ = (e);                    \
        if (st_ != MI355_STATUS_SUCCESS) return st_; \
    } while (0)

// the activation mode a producer writes for a GEMM over K inputs with weights W
int fused_mode(const mi355_context* ctx, const mi355_tensor& W, int64_t K) {
    return ctx->fuse && K % 32 == 0 ? act_mode_for_weight(&W) : ACT_F32;
}

ActOut act_out(char* base, int mode, int64_t rows, int64_t K) {
    Operand o;
    operand_bytes((size_t)rows, (size_t)K, &o, base);
    ActOut a{mode, nullptr, o.q, o.d, o.s, mmq_scale_pitch(K)};
    if (mode >= ACT_I8) a.dh = o.dh;
    return a;
}

ActF16 act_in(char* base, int mode, int64_t rows, int64_t K) {
    Operand o;
    operand_bytes((size_t)rows, (size_t)K, &o, base);
    ActF16 a;
    a.q = o.q;
    a.s1 = K;
    a.s2 = a.s3 = K * rows;
    a.d = mode == ACT_F16 ? nullptr : o.d;
    a.s = act_has_sums(mode) ? o.s : nullptr;
    if (mode >= ACT_I8) a.dh = o.dh;
    a.dp = mmq_scale_pitch(K);
    a.M = rows;
    a.K = K;
    return a;
}

mi355_status run_block(mi355_context* ctx, const mi355_hiera_hparams* hp, const Info& bi, const mi355_hiera_block* blk,
                       const float* x, int S, float* x_out, const Bufs& b) {
    const int Cin = bi.dim_in, Cout = bi.dim_out, NH = bi.heads, HD = Cout / NH, ws = bi.ws;
    const int S2 = bi.qs ? S / 2 : S;
    const bool dimch = Cin != Cout;
    const int nwh = ws > 0 ? cdiv(S, ws) : 1;
    const int nW = ws > 0 ? nwh * nwh : 1;
    const int Nkv = ws > 0 ? ws * ws : S * S;
    const int Nq = bi.qs ? (ws / 2) * (ws / 2) : Nkv;
    const int64_t rows = (int64_t)nW * Nkv;
    hipStream_t st = ctx->stream;
    if (!blk->norm1_w || !blk->norm1_b || !blk->qkv_b || !blk->proj_b || !blk->norm2_w || !blk->norm2_b || !blk->fc1_b ||
        !blk->fc2_b || (dimch && (!blk->dim_proj_w.data || !blk->dim_proj_b)))
        return fail(ctx, MI355_STATUS_INVALID_ARG, "hiera block: null weight pointer");

    // LN1: window order for the attention input; image order when dim_proj or
    // global attention reads it.  Each output is the operand its GEMM takes.
    const int64_t Mimg = (int64_t)S * S;
    const int mq = fused_mode(ctx, blk->qkv_w, Cin);
    const int md = dimch ? fused_mode(ctx, blk->dim_proj_w, Cin) : ACT_F32;
    {
        HieraLnArgs a{};
        a.x = x;
        a.w = blk->norm1_w;
        a.b = blk->norm1_b;
        a.C = Cin;
        a.W = a.H = S;
        a.eps = hp->eps;
        if (ws > 0) {
            a.out = mq == ACT_F32 ? ActOut{ACT_F32, b.xw, nullptr, nullptr, nullptr, 0} : act_out(b.a0, mq, rows, Cin);
            if (dimch)
                a.out_img = md == ACT_F32 ? ActOut{ACT_F32, b.xn, nullptr, nullptr, nullptr, 0}
                                          : act_out(b.a1, md, Mimg, Cin);
            a.rows_out = rows;
            a.ws = ws;
            a.nwh = nwh;
        } else {
            a.out = mq == ACT_F32 ? ActOut{ACT_F32, b.xn, nullptr, nullptr, nullptr, 0} : act_out(b.a0, mq, Mimg, Cin);
            a.rows_out = Mimg;
        }
        {
            Timed t(ctx, "hiera_ln");
            TRY(hip_check(ctx, t.done(launch_hiera_ln(a, st)), "hiera_ln launch"));
        }
        if (ws == 0 && dimch && md != mq) {  // a second image-order LN for dim_proj's operand
            a.out = md == ACT_F32 ? ActOut{ACT_F32, b.xw, nullptr, nullptr, nullptr, 0} : act_out(b.a1, md, Mimg, Cin);
            Timed t(ctx, "hiera_ln");
            TRY(hip_check(ctx, t.done(launch_hiera_ln(a, st)), "hiera_ln launch"));
        }
    }
    // shortcut
    const float* sc = x;
    if (dimch) {
        const mi355_tensor out = tensor_on(b.dp, T_F32, Cout, Mimg);
        if (ws == 0 && md == mq) {  // one image-order LN output serves both GEMMs
            if (md == ACT_F32) {
                const mi355_tensor in = tensor_on(b.xn, T_F32, Cin, Mimg);
                TRY(mi355_mul_mat(ctx, &blk->dim_proj_w, &in, &out));
            } else {
                TRY(mul_mat_act(ctx, &blk->dim_proj_w, act_in(b.a0, md, Mimg, Cin), &out));
            }
        } else if (md == ACT_F32) {
            const mi355_tensor in = tensor_on(ws > 0 ? b.xn : b.xw, T_F32, Cin, Mimg);
            TRY(mi355_mul_mat(ctx, &blk->dim_proj_w, &in, &out));
        } else {
            TRY(mul_mat_act(ctx, &blk->dim_proj_w, act_in(b.a1, md, Mimg, Cin), &out));
        }
        Timed t(ctx, "hiera_bias_maxpool");
        TRY(hip_check(ctx, t.done(launch_hiera_bias_maxpool(b.dp, blk->dim_proj_b, b.sc, Cout, S, S, bi.qs, st)),
                      "bias_maxpool launch"));
        sc = b.sc;
    } else if (bi.qs) {
        Timed t(ctx, "hiera_bias_maxpool");
        TRY(hip_check(ctx, t.done(launch_hiera_bias_maxpool(x, nullptr, b.sc, Cout, S, S, true, st)), "maxpool launch"));
        sc = b.sc;
    }
    // attention operands: q / k / v are the qkv rows split by head with the bias added,
    // rounded to fp16 ([window][head][token][HD]): the GEMM's qkv epilogue writes them
    // directly (the same fp32 add and rounding as hiera_qkv, no f32 round trip).  With Q
    // pooling the epilogue's unpooled q goes to the (then unused) qkv buffer and
    // hiera_qpool takes its 2x2 window max
    if (mq != ACT_F32) {
        MmqEpi e{};
        e.kind = MMQ_EPI_QKV;
        e.bias = blk->qkv_b;
        e.rope = nullptr;
        e.q = bi.qs ? reinterpret_cast<_Float16*>(b.qkv) : b.q;
        e.k = b.k;
        e.v = b.v;
        e.ntok = Nkv;
        e.nh = NH;
        e.hd = HD;
        TRY(mul_mat_epi(ctx, &blk->qkv_w, act_in(b.a0, mq, rows, Cin), e));
        if (bi.qs) {
            Timed t(ctx, "hiera_qkv");
            TRY(hip_check(ctx,
                          t.done(launch_hiera_qpool(reinterpret_cast<const _Float16*>(b.qkv), b.q, nW, NH, Nkv, Nq,
                                                    ws, HD, st)),
                          "hiera_qpool launch"));
        }
    } else {
        const mi355_tensor out = tensor_on(b.qkv, T_F32, 3 * Cout, rows);
        if (mq == ACT_F32) {
            const mi355_tensor in = tensor_on(ws > 0 ? b.xw : b.xn, T_F32, Cin, rows);
            TRY(mi355_mul_mat(ctx, &blk->qkv_w, &in, &out));
        } else {
            TRY(mul_mat_act(ctx, &blk->qkv_w, act_in(b.a0, mq, rows, Cin), &out));
        }
        HieraQkvArgs a{};
        a.qkv = b.qkv;
        a.bias = blk->qkv_b;
        a.q = b.q;
        a.k = b.k;
        a.v = b.v;
        a.B = nW;
        a.Nkv = Nkv;
        a.Nq = Nq;
        a.NH = NH;
        a.HD = HD;
        a.qpool = bi.qs;
        a.ws = ws;
        Timed t(ctx, "hiera_qkv");
        TRY(hip_check(ctx, t.done(launch_hiera_qkv(a, st)), "hiera_qkv launch"));
    }
    // attention; for quantized / F16 proj weights it writes the projection's operand
    const int mp = fused_mode(ctx, blk->proj_w, Cout);
    {
        const mi355_tensor q = tensor_on(b.q, T_F16, HD, Nq, NH, nW), k = tensor_on(b.k, T_F16, HD, Nkv, NH, nW),
                           v = tensor_on(b.v, T_F16, HD, Nkv, NH, nW), o = tensor_on(b.att, T_F32, HD, NH, Nq, nW);
        const ActOut op = act_out(b.a0, mp, (int64_t)Nq * nW, Cout);
        TRY(flash_attn_act(ctx, &q, &k, &v, nullptr, 1.0f / sqrtf((float)HD), 0.0f, 0.0f, &o,
                           mp == ACT_F32 ? nullptr : &op));
    }
    // proj (+ bias, window unpartition with crop, shortcut): fused into the
    // GEMM's epilogue for quantized / F16 weights
    {
        const int64_t Mo = (int64_t)Nq * nW;
        const int wso = ws > 0 ? (bi.qs ? ws / 2 : ws) : 0;
        const int nwh_o = wso > 0 ? cdiv(S2, wso) : 1;
        if (mp == ACT_F32) {
            const mi355_tensor in = tensor_on(b.att, T_F32, Cout, Mo), out = tensor_on(b.p, T_F32, Cout, Mo);
            TRY(mi355_mul_mat(ctx, &blk->proj_w, &in, &out));
            Timed t(ctx, "hiera_proj_residual");
            TRY(hip_check(ctx, t.done(launch_hiera_proj_residual(x_out, sc, b.p, blk->proj_b, Cout, S2, S2, wso, nwh_o, st)),
                          "proj_residual launch"));
        } else {
            MmqEpi e{};
            e.kind = MMQ_EPI_RESIDUAL;
            e.bias = blk->proj_b;
            e.res = sc;
            e.out = x_out;
            e.map = RowMap{wso > 0 ? ROWMAP_SAM2_UNPART : ROWMAP_IDENTITY, S2, S2, wso, nwh_o};
            TRY(mul_mat_epi(ctx, &blk->proj_w, act_in(b.a0, mp, Mo, Cout), e));
        }
    }
    // MLP
    const int64_t M2 = (int64_t)S2 * S2;
    const int MLP = 4 * Cout;
    const int m1 = fused_mode(ctx, blk->fc1_w, Cout);
    {
        HieraLnArgs a{};
        a.x = x_out;
        a.w = blk->norm2_w;
        a.b = blk->norm2_b;
        a.out = m1 == ACT_F32 ? ActOut{ACT_F32, b.xn, nullptr, nullptr, nullptr, 0} : act_out(b.a0, m1, M2, Cout);
        a.rows_out = M2;
        a.C = Cout;
        a.W = a.H = S2;
        a.eps = hp->eps;
        Timed t(ctx, "hiera_ln");
        TRY(hip_check(ctx, t.done(launch_hiera_ln(a, st)), "hiera_ln launch"));
    }
    // fc1, bias + GELU writing fc2's operand, fc2 (+ bias, residual: fused epilogue)
    const int m2 = fused_mode(ctx, blk->fc2_w, MLP);
    {
        const mi355_tensor out = tensor_on(b.h, T_F32, MLP, M2);
        if (m1 == ACT_F32) {
            const mi355_tensor in = tensor_on(b.xn, T_F32, Cout, M2);
            TRY(mi355_mul_mat(ctx, &blk->fc1_w, &in, &out));
        } else {
            TRY(mul_mat_act(ctx, &blk->fc1_w, act_in(b.a0, m1, M2, Cout), &out));
        }
        Timed t(ctx, "bias_gelu_tanh");
        if (m2 == ACT_F32)
            TRY(hip_check(ctx, t.done(launch_bias_gelu_tanh(b.h, blk->fc1_b, M2, MLP, st)), "bias_gelu_tanh launch"));
        else
            TRY(hip_check(ctx, t.done(launch_bias_gelu_tanh_act(b.h, blk->fc1_b, M2, MLP, act_out(b.a2, m2, M2, MLP), st)),
                          "bias_gelu_tanh launch"));
    }
    if (m2 == ACT_F32) {
        const mi355_tensor in = tensor_on(b.h, T_F32, MLP, M2), out = tensor_on(b.f, T_F32, Cout, M2);
        TRY(mi355_mul_mat(ctx, &blk->fc2_w, &in, &out));
        Timed t(ctx, "bias_residual");
        TRY(hip_check(ctx, t.done(launch_bias_residual(x_out, b.f, blk->fc2_b, M2, Cout, st)), "bias_residual launch"));
    } else {
        MmqEpi e{};
        e.kind = MMQ_EPI_RESIDUAL;
        e.bias = blk->fc2_b;
        e.res = x_out;
        e.out = x_out;
        e.map = RowMap{ROWMAP_IDENTITY, 0, 0, 0, 0};
        TRY(mul_mat_epi(ctx, &blk->fc2_w, act_in(b.a2, m2, M2, MLP), e));
    }
    return MI355_STATUS_SUCCESS;
}

mi355_status check_patch(mi355_context* ctx, const mi355_hiera_hparams* hp, const mi355_tensor* patch_w,
                         const char* what) {
    const int E = hp->embed_dim;
    if (patch_w->ne[0] != 7 || patch_w->ne[1] != 7 || patch_w->ne[2] != 3 || patch_w->ne[3] != E ||
        !(patch_w->type == T_F32 || patch_w->type == T_F16) || !patch_w->data)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "%s: patch weight must be F32/F16 [7, 7, 3, E]", what);
    if (patch_w->nb[0] != (patch_w->type == T_F32 ? 4 : 2) || patch_w->nb[3] != patch_w->nb[0] * 147)
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "%s: patch weight must be contiguous", what);
    return MI355_STATUS_SUCCESS;
}

// patch embedding (sam3.cpp:4473-4494): ggml_conv_2d(w, img, 4, 4, 3, 3, 1, 1) = im2col +
// F32 mul_mat, + bias, + pos_embed -> x [S0*S0][E]. With F16 weights the image columns are
// rounded to fp16 (ggml's F16 im2col) and the weights widened: the F16 kernel's products
// are exact in fp32. Bias and pos_embed are added in the GEMM's epilogue in the reference's
// order, (conv + b) + pe.
mi355_status patch_embed(mi355_context* ctx, const mi355_hiera_hparams* hp, const float* image,
                         const mi355_tensor* patch_w, const float* patch_b, const float* pos_embed, const Bufs& b,
                         float* x) {
    const int E = hp->embed_dim, IMG = hp->img_size, S0 = IMG / 4;
    hipStream_t st = ctx->stream;
    const bool w16 = patch_w->type == T_F16;
    {
        Timed t(ctx, "im2col");
        TRY(hip_check(ctx, t.done(launch_im2col_pad(image, b.cols, 3, IMG, IMG, 7, 7, 4, 3, S0, S0, PATCH_KP, w16, st)),
                      "im2col launch"));
    }
    TRY(hip_check(ctx, launch_pad_rows_f32(patch_w->data, w16, E, 147, PATCH_KP, b.w32, st), "patch weight pad"));
    GemmF32Args g;
    g.W = b.w32;
    g.w_nb1 = 4LL * PATCH_KP;
    g.w_nb2 = g.w_nb3 = g.w_nb1 * E;
    g.X = b.cols;
    g.x_nb1 = 4LL * PATCH_KP;
    g.x_nb2 = g.x_nb3 = g.x_nb1 * S0 * S0;
    g.D = x;
    g.d_nb1 = 4LL * E;
    g.d_nb2 = g.d_nb3 = g.d_nb1 * S0 * S0;
    g.M = S0 * S0;
    g.N = E;
    g.K = PATCH_KP;
    g.ne12 = g.r2 = g.r3 = 1;
    g.bias = patch_b;
    g.add = pos_embed;
    Timed t(ctx, "gemm_f32");
    return hip_check(ctx, t.done(launch_gemm_f32(g, 1, st)), "gemm_f32 launch");
}

}  // namespace

extern "C" {

mi355_status mi355_hiera_pos_embed(mi355_context* ctx, const float* bkg, int E, int bkg_h, int bkg_w, const float* win,
                                   int ws, int H, int W, float* out) {
    if (!bkg || !win || !out) return fail(ctx, MI355_STATUS_INVALID_ARG, "hiera_pos_embed: null pointer");
    if (E <= 0 || bkg_h <= 0 || bkg_w <= 0 || ws <= 0 || H <= 0 || W <= 0 || (int64_t)H * W * E >= ((int64_t)1 << 40))
        return fail(ctx, MI355_STATUS_INVALID_ARG, "hiera_pos_embed: bad sizes");
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "hiera_pos_embed: null context");
    (void)hipSetDevice(ctx->device);
    Timed t(ctx, "hiera_pos_embed");
    return hip_check(ctx, t.done(launch_hiera_pos_embed(bkg, E, bkg_h, bkg_w, win, ws, H, W, out, ctx->stream)),
                     "hiera_pos_embed launch");
}

int mi355_hiera_n_blocks(const mi355_hiera_hparams* hp) {
    std::vector<Info> infos;
    if (!hp || !block_infos(hp, infos)) return -1;
    return (int)infos.size();
}

mi355_status mi355_hiera_block_info_get(const mi355_hiera_hparams* hp, int block_index, mi355_hiera_block_info* out) {
    std::vector<Info> infos;
    if (!hp || !out || !block_infos(hp, infos)) return fail(nullptr, MI355_STATUS_INVALID_ARG, "hiera: bad hparams");
    if (block_index < 0 || block_index >= (int)infos.size())
        return fail(nullptr, MI355_STATUS_INVALID_ARG, "hiera: block index %d out of range", block_index);
    const Info& b = infos[block_index];
    out->dim_in = b.dim_in;
    out->dim_out = b.dim_out;
    out->num_heads = b.heads;
    out->window_size = b.ws;
    out->q_stride = b.qs;
    out->stage = b.stage;
    return MI355_STATUS_SUCCESS;
}

size_t mi355_hiera_workspace_size(const mi355_hiera_hparams* hp) {
    std::vector<Info> infos;
    if (check_hp(nullptr, hp, infos) != MI355_STATUS_SUCCESS) return 0;
    return layout(all_sizes(hp, infos), nullptr, nullptr);
}

mi355_status mi355_hiera_block_forward(mi355_context* ctx, const mi355_hiera_hparams* hp, int block_index,
                                       const mi355_hiera_block* blk, const float* x, int spatial, float* x_out) {
    std::vector<Info> infos;
    TRY(check_hp(ctx, hp, infos));
    if (!blk || !x || !x_out) return fail(ctx, MI355_STATUS_INVALID_ARG, "hiera_block: null pointer");
    if (block_index < 0 || block_index >= (int)infos.size())
        return fail(ctx, MI355_STATUS_INVALID_ARG, "hiera_block: block index %d out of range", block_index);
    const Info& bi = infos[block_index];
    if (spatial <= 0 || (bi.qs && spatial % 2 != 0))
        return fail(ctx, MI355_STATUS_INVALID_ARG, "hiera_block: bad spatial size %d", spatial);
    if (x == x_out) return fail(ctx, MI355_STATUS_INVALID_ARG, "hiera_block: x_out must not overlap x");
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "hiera_block: null context");
    (void)hipSetDevice(ctx->device);
    // buffers sized for this block at this spatial size (at least the backbone's)
    Sizes z = all_sizes(hp, infos);
    z.max_with(block_sizes(bi, spatial));
    TRY(ensure_buffer(ctx, &ctx->enc, &ctx->enc_size, layout(z, nullptr, nullptr)));
    Bufs b;
    layout(z, static_cast<char*>(ctx->enc), &b);
    return run_block(ctx, hp, bi, blk, x, spatial, x_out, b);
}

mi355_status mi355_hiera_prefix(mi355_context* ctx, const mi355_hiera_hparams* hp, const float* image,
                                const mi355_tensor* patch_w, const float* patch_b, const float* pos_embed, float* x) {
    std::vector<Info> infos;
    TRY(check_hp(ctx, hp, infos));
    if (!image || !patch_w || !patch_b || !pos_embed || !x) return fail(ctx, MI355_STATUS_INVALID_ARG, "hiera_prefix: null pointer");
    TRY(check_patch(ctx, hp, patch_w, "hiera_prefix"));
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "hiera_prefix: null context");
    (void)hipSetDevice(ctx->device);
    Bufs b;
    TRY(get_bufs(ctx, hp, infos, &b));
    return patch_embed(ctx, hp, image, patch_w, patch_b, pos_embed, b, x);
}

mi355_status mi355_hiera_encode(mi355_context* ctx, const mi355_hiera_hparams* hp, const float* image,
                                const mi355_tensor* patch_w, const float* patch_b, const float* pos_embed,
                                const mi355_hiera_block* blocks, int n_blocks, float* const stage_out[4]) {
    std::vector<Info> infos;
    TRY(check_hp(ctx, hp, infos));
    if (!image || !patch_w || !patch_b || !pos_embed || !blocks)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "hiera_encode: null pointer");
    if (n_blocks != (int)infos.size())
        return fail(ctx, MI355_STATUS_INVALID_ARG, "hiera_encode: %d blocks given, the stage table has %d", n_blocks,
                    (int)infos.size());
    TRY(check_patch(ctx, hp, patch_w, "hiera_encode"));
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "hiera_encode: null context");
    (void)hipSetDevice(ctx->device);
    Bufs b;
    TRY(get_bufs(ctx, hp, infos, &b));
    hipStream_t st = ctx->stream;
    const int S0 = hp->img_size / 4;
    TRY(patch_embed(ctx, hp, image, patch_w, patch_b, pos_embed, b, b.x0));
    float* cur = b.x0;
    float* nxt = b.x1;
    int S = S0, stage = 0;
    int ends[4], total = 0;
    for (int s = 0; s < 4; ++s) {
        total += hp->stages[s];
        ends[s] = total - 1;
    }
    // a stage's last block writes its output straight into the caller's stage map, which the
    // next block then reads (run_block only reads its input); the internal pair x0 / x1 takes
    // every other output, the one that is not the current input
    for (int i = 0; i < n_blocks; ++i) {
        while (stage < 4 && hp->stages[stage] == 0) ++stage;
        const bool last = stage < 4 && i == ends[stage];
        float* dst = last && stage_out && stage_out[stage] ? stage_out[stage] : nxt;
        TRY(run_block(ctx, hp, infos[i], &blocks[i], cur, S, dst, b));
        cur = dst;
        nxt = cur == b.x0 ? b.x1 : b.x0;
        if (infos[i].qs) S /= 2;
        if (last) ++stage;
    }
    return MI355_STATUS_SUCCESS;
}

}  // extern "C"
