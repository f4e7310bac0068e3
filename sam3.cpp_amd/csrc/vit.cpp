// SAM3 ViT image encoder on the MI355X backend: the graph of
// sam3_build_vit_graph (sam3.cpp:3836-3853) executed node group by node
// group.  MUL_MAT and FLASH_ATTN_EXT go through the same entry points a ggml
// graph would use; the memory-bound nodes between them run as the fused
// passes of glue.hip.  Per block (sam3_vit_block_forward, sam3.cpp:3714-3805):
//
//   xn   = LN1(x)                  [window order when windowed: win_part]
//   qkv  = mul_mat(qkv_w, xn)
//   q,k,v = split(qkv + qkv_b), RoPE(q), RoPE(k)    -> fp16
//   attn = flash_attn_ext(q, k, v, 1/sqrt(HD))      [E, M]
//   p    = mul_mat(proj_w, attn)
//   x    = x + win_unpart(p + proj_b)
//   xn   = LN2(x)
//   h    = gelu_erf(mul_mat(fc1_w, xn) + fc1_b)
//   x    = x + (mul_mat(fc2_w, h) + fc2_b)
//
// For quantized and F16 weights the passes that feed a MUL_MAT (LN1 -> qkv,
// LN2 -> fc1, bias+GELU -> fc2) write the GEMM's activation operand directly
// (Q8 quants + scales, or F16 rows), computed from the same fp32 values ggml
// would quantize, so the separate activation quantize pass and the f32 round
// trip disappear.  The activation buffers live in one device allocation owned
// by the context (mi355_vit_workspace_size); mul_mat keeps using the
// context's own scratch.
#include <cmath>

#include "context.h"

using namespace mi355;

namespace {

struct EncBufs {
    float* xn;      // [M][E]  LN output, projection output
    float* qkv;     // [M][3E]
    _Float16* q;    // [M][E] each, FLASH_ATTN_EXT layout
    _Float16* k;
    _Float16* v;
    float* attn;    // [M][E]  attention output, fc2 output
    float* big;     // [M][MLP] fc1 output (or im2col columns)
    uint16_t* aq;   // [M][E] activation operand of qkv / proj / fc1: Q8 quants or F16 rows
    uint16_t* ad;   // [M][dp(E)] block scales
    uint16_t* as;   // [M][dp(E)] Q8_1 sums
    uint16_t* hq;   // [M][MLP] operand of fc2 (fc1's epilogue output)
    uint16_t* hd;
    uint16_t* hs;
};

size_t enc_bytes(const mi355_vit_hparams* hp, EncBufs* b, char* base) {
    const size_t M = (size_t)hp->grid * hp->grid, E = (size_t)hp->embed_dim;
    const size_t kpatch = 3 * (size_t)hp->patch_size * hp->patch_size;
    const size_t big = M * std::max((size_t)hp->mlp_dim, kpatch) * 4;
    const size_t H = (size_t)hp->mlp_dim;
    const size_t dpe = (size_t)mmq_scale_pitch((int64_t)E), dph = (size_t)mmq_scale_pitch((int64_t)H);
    // operand scales: fp16 [M][dp], or the int8 operand's dl and dh dword arrays (4 bytes per block)
    const size_t sz[13] = {M * E * 4, M * 3 * E * 4, M * E * 2, M * E * 2, M * E * 2,   M * E * 4,  big,
                           M * E * 2, M * dpe * 4,   M * dpe * 2, M * H * 2, M * dph * 4, M * dph * 2};
    size_t off[13], o = 0;
    for (int i = 0; i < 13; ++i) {
        off[i] = o;
        o += align_up(sz[i]);
    }
    if (b && base) {
        b->xn = reinterpret_cast<float*>(base + off[0]);
        b->qkv = reinterpret_cast<float*>(base + off[1]);
        b->q = reinterpret_cast<_Float16*>(base + off[2]);
        b->k = reinterpret_cast<_Float16*>(base + off[3]);
        b->v = reinterpret_cast<_Float16*>(base + off[4]);
        b->attn = reinterpret_cast<float*>(base + off[5]);
        b->big = reinterpret_cast<float*>(base + off[6]);
        b->aq = reinterpret_cast<uint16_t*>(base + off[7]);
        b->ad = reinterpret_cast<uint16_t*>(base + off[8]);
        b->as = reinterpret_cast<uint16_t*>(base + off[9]);
        b->hq = reinterpret_cast<uint16_t*>(base + off[10]);
        b->hd = reinterpret_cast<uint16_t*>(base + off[11]);
        b->hs = reinterpret_cast<uint16_t*>(base + off[12]);
    }
    return o;
}

mi355_status check_hp(mi355_context* ctx, const mi355_vit_hparams* hp) {
    if (!hp) return fail(ctx, MI355_STATUS_INVALID_ARG, "vit: null hparams");
    const int E = hp->embed_dim, NH = hp->num_heads;
    if (E <= 0 || NH <= 0 || E % NH != 0 || hp->mlp_dim <= 0 || hp->grid <= 0 || hp->patch_size <= 0 ||
        hp->window_size < 0 || hp->pos_grid < 0 || !(hp->eps >= 0.0f))
        return fail(ctx, MI355_STATUS_INVALID_ARG, "vit: bad hparams");
    const int HD = E / NH;
    if (!(HD == 64 || HD == 96 || HD == 128))
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "vit: head size %d (supported: 64, 96, 128)", HD);
    if (E % 64 != 0 || E > 2048) return fail(ctx, MI355_STATUS_UNSUPPORTED, "vit: embed_dim must be a multiple of 64, <= 2048");
    if (hp->mlp_dim % 4 != 0) return fail(ctx, MI355_STATUS_UNSUPPORTED, "vit: mlp_dim must be a multiple of 4");
    if ((int64_t)hp->grid * hp->grid * std::max(3 * E, hp->mlp_dim) >= ((int64_t)1 << 31))
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "vit: activations beyond 2^31 elements");
    return MI355_STATUS_SUCCESS;
}

// contiguous F32 / F16 tensor over a device buffer
mi355_tensor dev_tensor(const void* p, int type, int64_t ne0, int64_t ne1, int64_t ne2 = 1, int64_t ne3 = 1) {
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

// a GEMM activation operand (q, d, s) with K inputs over M rows: the E-wide
// one (aq, ad, as) or fc2's (hq, hd, hs); the int8 operand's dh array follows
// dl in the scale buffer
ActOut act_out(const EncBufs& b, int mode, int64_t M, int64_t K, bool hidden = false) {
    ActOut o = hidden ? ActOut{mode, nullptr, b.hq, b.hd, b.hs, mmq_scale_pitch(K)}
                      : ActOut{mode, nullptr, b.aq, b.ad, b.as, mmq_scale_pitch(K)};
    if (mode >= ACT_I8) o.dh = reinterpret_cast<uint32_t*>(o.d) + M * (o.dp / 2);
    return o;
}
ActF16 act_in(const EncBufs& b, int mode, int64_t M, int64_t K, bool hidden = false) {
    ActF16 a;
    a.q = hidden ? b.hq : b.aq;
    a.s1 = K;
    a.s2 = a.s3 = K * M;
    a.d = mode == ACT_F16 ? nullptr : hidden ? b.hd : b.ad;
    a.s = act_has_sums(mode) ? (hidden ? b.hs : b.as) : nullptr;
    a.dp = mmq_scale_pitch(K);
    a.M = M;
    a.K = K;
    if (mode >= ACT_I8) a.dh = reinterpret_cast<const uint32_t*>(a.d) + M * (a.dp / 2);  // after dl, as act_out puts it
    return a;
}

mi355_status get_bufs(mi355_context* ctx, const mi355_vit_hparams* hp, EncBufs* b) {
    const size_t need = enc_bytes(hp, nullptr, nullptr);
    mi355_status st = ensure_buffer(ctx, &ctx->enc, &ctx->enc_size, need);
    if (st != MI355_STATUS_SUCCESS) return st;
    enc_bytes(hp, b, static_cast<char*>(ctx->enc));
    return MI355_STATUS_SUCCESS;
}

}  // namespace

extern "C" {

size_t mi355_vit_workspace_size(const mi355_vit_hparams* hp) {
    if (check_hp(nullptr, hp) != MI355_STATUS_SUCCESS) return 0;
    return enc_bytes(hp, nullptr, nullptr);
}

mi355_status mi355_vit_layer_norm(mi355_context* ctx, const float* x, const float* add, int add_grid, const float* w,
                                  const float* b, float* y, int64_t rows, int E, int grid, int window, float eps) {
    if (!x || !y) return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_layer_norm: null x/y");
    if (rows < 0 || E <= 0 || add_grid < 0 || window < 0 || !(eps >= 0.0f))
        return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_layer_norm: bad sizes");
    if (E % 64 != 0 || E > 2048) return fail(ctx, MI355_STATUS_UNSUPPORTED, "vit_layer_norm: E must be a multiple of 64, <= 2048");
    if ((window > 0 || (add && add_grid > 0)) && ((int64_t)grid * grid != rows || grid <= 0))
        return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_layer_norm: rows must be grid^2 for window / tiled add");
    if (window > 0 && grid % window != 0)
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "vit_layer_norm: grid %d not a multiple of the window %d", grid, window);
    if (x == y && window > 0) return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_layer_norm: window reorder cannot run in place");
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "vit_layer_norm: null context");
    LnArgs a;
    a.x = x;
    a.add = add;
    a.add_grid = add ? add_grid : 0;
    a.w = w;
    a.b = b;
    a.out = ActOut{ACT_F32, y, nullptr, nullptr, nullptr, 0};
    a.rows = rows;
    a.E = E;
    a.grid = grid;
    a.ws = window;
    a.eps = eps;
    (void)hipSetDevice(ctx->device);
    Timed t(ctx, "layer_norm");
    return hip_check(ctx, t.done(launch_layer_norm(a, ctx->stream)), "layer_norm launch");
}

mi355_status mi355_vit_qkv_rope(mi355_context* ctx, const float* qkv, const float* bias, const float* rope, void* q,
                                void* k, void* v, int64_t M, int N, int n_heads, int head_dim) {
    if (!qkv || !bias || !q || !k || !v) return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_qkv_rope: null pointer");
    if (M < 0 || N <= 0 || n_heads <= 0 || head_dim <= 0 || head_dim % 2 != 0 || M % N != 0)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_qkv_rope: bad sizes");
    if (((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) & 3) != 0)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_qkv_rope: q/k/v must be 4-byte aligned");
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "vit_qkv_rope: null context");
    QkvArgs a;
    a.qkv = qkv;
    a.bias = bias;
    a.rope = rope;
    a.q = static_cast<_Float16*>(q);
    a.k = static_cast<_Float16*>(k);
    a.v = static_cast<_Float16*>(v);
    a.M = M;
    a.N = N;
    a.NH = n_heads;
    a.HD = head_dim;
    (void)hipSetDevice(ctx->device);
    Timed t(ctx, "qkv_rope");
    return hip_check(ctx, t.done(launch_qkv_rope(a, ctx->stream)), "qkv_rope launch");
}

mi355_status mi355_vit_proj_residual(mi355_context* ctx, float* x, const float* p, const float* b, int64_t rows, int E,
                                     int grid, int window) {
    if (!x || !p || !b) return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_proj_residual: null pointer");
    if (rows < 0 || E <= 0 || E % 4 != 0 || window < 0) return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_proj_residual: bad sizes");
    if (window > 0 && (grid <= 0 || (int64_t)grid * grid != rows || grid % window != 0))
        return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_proj_residual: rows must be grid^2 with grid a multiple of the window");
    if (window > 0 && x == p) return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_proj_residual: window reorder cannot run in place");
    if (((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(p) | reinterpret_cast<uintptr_t>(b)) & 15) != 0)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_proj_residual: pointers must be 16-byte aligned");
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "vit_proj_residual: null context");
    (void)hipSetDevice(ctx->device);
    Timed t(ctx, "proj_residual");
    return hip_check(ctx, t.done(launch_proj_residual(x, p, b, rows, E, grid, window, ctx->stream)), "proj_residual launch");
}

mi355_status mi355_vit_bias_gelu(mi355_context* ctx, float* h, const float* b, int64_t rows, int n) {
    if (!h || !b) return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_bias_gelu: null pointer");
    if (rows < 0 || n <= 0 || n % 4 != 0) return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_bias_gelu: bad sizes (n %% 4 == 0)");
    if (((reinterpret_cast<uintptr_t>(h) | reinterpret_cast<uintptr_t>(b)) & 15) != 0)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_bias_gelu: pointers must be 16-byte aligned");
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "vit_bias_gelu: null context");
    (void)hipSetDevice(ctx->device);
    Timed t(ctx, "bias_gelu");
    return hip_check(ctx, t.done(launch_bias_gelu(h, b, rows, n, ctx->stream)), "bias_gelu launch");
}

mi355_status mi355_vit_bias_residual(mi355_context* ctx, float* x, const float* f, const float* b, int64_t rows, int n) {
    if (!x || !f || !b) return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_bias_residual: null pointer");
    if (rows < 0 || n <= 0 || n % 4 != 0) return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_bias_residual: bad sizes (n %% 4 == 0)");
    if (((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(f) | reinterpret_cast<uintptr_t>(b)) & 15) != 0)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_bias_residual: pointers must be 16-byte aligned");
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "vit_bias_residual: null context");
    (void)hipSetDevice(ctx->device);
    Timed t(ctx, "bias_residual");
    return hip_check(ctx, t.done(launch_bias_residual(x, f, b, rows, n, ctx->stream)), "bias_residual launch");
}

mi355_status mi355_vit_prefix(mi355_context* ctx, const mi355_vit_hparams* hp, const float* image,
                              const mi355_tensor* patch_w, const float* pos_embed, const float* ln_pre_w,
                              const float* ln_pre_b, float* x) {
    mi355_status st = check_hp(ctx, hp);
    if (st != MI355_STATUS_SUCCESS) return st;
    if (!image || !patch_w || !pos_embed || !ln_pre_w || !ln_pre_b || !x)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_prefix: null pointer");
    const int E = hp->embed_dim, P = hp->patch_size, G = hp->grid;
    const int64_t K = 3LL * P * P, M = (int64_t)G * G;
    if (patch_w->ne[0] != P || patch_w->ne[1] != P || patch_w->ne[2] != 3 || patch_w->ne[3] != E)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_prefix: patch weight must be [P, P, 3, E]");
    if (hp->pos_grid <= 0 || G % hp->pos_grid != 0)
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "vit_prefix: grid must be a multiple of pos_grid");
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "vit_prefix: null context");
    (void)hipSetDevice(ctx->device);
    EncBufs b;
    st = get_bufs(ctx, hp, &b);
    if (st != MI355_STATUS_SUCCESS) return st;
    {
        Timed t(ctx, "im2col");
        st = hip_check(ctx, t.done(launch_im2col(image, b.big, 3, G * P, G * P, P, G, ctx->stream)), "im2col launch");
        if (st != MI355_STATUS_SUCCESS) return st;
    }
    // conv weight [P, P, 3, E] viewed as ggml [K, E]
    mi355_tensor w = *patch_w;
    w.ne[0] = K;
    w.ne[1] = E;
    w.ne[2] = w.ne[3] = 1;
    w.nb[1] = patch_w->nb[3];
    w.nb[2] = w.nb[3] = w.nb[1] * E;
    const mi355_tensor cols = dev_tensor(b.big, T_F32, K, M);
    const mi355_tensor out = dev_tensor(b.xn, T_F32, E, M);
    st = mi355_mul_mat(ctx, &w, &cols, &out);
    if (st != MI355_STATUS_SUCCESS) return st;
    return mi355_vit_layer_norm(ctx, b.xn, pos_embed, hp->pos_grid, ln_pre_w, ln_pre_b, x, M, E, G, 0, hp->eps);
}

// One block.  next: the block that follows (or null); when it is given and the shapes allow,
// this block's fc2 also runs next's LN1 into the qkv operand (fused into the K-split
// reduction at E = 1024) and sets *ln_next_done.  ln1_ready: this block's LN1 already ran so.
static mi355_status block_forward(mi355_context* ctx, const mi355_vit_hparams* hp, const mi355_vit_block* blk, float* x,
                                  const mi355_vit_block* next, bool ln1_ready, bool* ln_next_done) {
    if (ln_next_done) *ln_next_done = false;
    mi355_status st = check_hp(ctx, hp);
    if (st != MI355_STATUS_SUCCESS) return st;
    if (!blk || !x || !blk->norm1_w || !blk->norm1_b || !blk->qkv_b || !blk->proj_b || !blk->norm2_w || !blk->norm2_b ||
        !blk->fc1_b || !blk->fc2_b)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_block: null pointer");
    const int E = hp->embed_dim, NH = hp->num_heads, HD = E / NH, MLP = hp->mlp_dim, G = hp->grid;
    const int WS = blk->is_global ? 0 : hp->window_size;
    if (!blk->is_global && (WS <= 0 || G % WS != 0))
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "vit_block: grid %d not a multiple of the window %d", G, WS);
    const int64_t M = (int64_t)G * G;
    const int N = WS > 0 ? WS * WS : (int)M;  // tokens per attention batch
    const int B = (int)(M / N);
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "vit_block: null context");
    (void)hipSetDevice(ctx->device);
    EncBufs b;
    st = get_bufs(ctx, hp, &b);
    if (st != MI355_STATUS_SUCCESS) return st;

#define TRY(e)                                   \
    do {                                         \
        st = (e);                                \
        if (st != MI355_STATUS_SUCCESS) return st; \
    } while (0)
    // LN -> the GEMM's activation operand (fused) or F32 rows
    auto ln_gemm = [&](const float* w, const float* bb, int ws, const mi355_tensor& W, float* out, int64_t N,
                       const MmqEpi* epi, bool ready = false) -> mi355_status {
        const int mode = ctx->fuse ? act_mode_for_weight(&W) : ACT_F32;
        if (mode == ACT_F32 && epi) return fail(ctx, MI355_STATUS_FAILED, "vit: epilogue without a fused operand");
        if (mode == ACT_F32 && ready) return fail(ctx, MI355_STATUS_FAILED, "vit: LayerNorm handed over without an operand");
        if (mode == ACT_F32) {
            mi355_status s1 = mi355_vit_layer_norm(ctx, x, nullptr, 0, w, bb, b.xn, M, E, G, ws, hp->eps);
            if (s1 != MI355_STATUS_SUCCESS) return s1;
            const mi355_tensor in = dev_tensor(b.xn, T_F32, E, M), o = dev_tensor(out, T_F32, N, M);
            return mi355_mul_mat(ctx, &W, &in, &o);
        }
        LnArgs a;
        a.x = x;
        a.add = nullptr;
        a.add_grid = 0;
        a.w = w;
        a.b = bb;
        a.out = act_out(b, mode, M, E);
        a.rows = M;
        a.E = E;
        a.grid = G;
        a.ws = ws;
        a.eps = hp->eps;
        if (!ready) {
            Timed t(ctx, "layer_norm");
            mi355_status s1 = hip_check(ctx, t.done(launch_layer_norm(a, ctx->stream)), "layer_norm launch");
            if (s1 != MI355_STATUS_SUCCESS) return s1;
        }
        if (epi) return mul_mat_epi(ctx, &W, act_in(b, mode, M, E), *epi);
        const mi355_tensor o = dev_tensor(out, T_F32, N, M);
        return mul_mat_act(ctx, &W, act_in(b, mode, M, E), &o);
    };
    // attention
    // LN1 -> qkv (+ bias, q/k/v split, RoPE, fp16: fused epilogue)
    if (ctx->fuse && act_mode_for_weight(&blk->qkv_w) != ACT_F32) {
        MmqEpi e{};
        e.kind = MMQ_EPI_QKV;
        e.bias = blk->qkv_b;
        e.rope = blk->freqs_cis;
        e.q = b.q;
        e.k = b.k;
        e.v = b.v;
        e.ntok = N;
        e.nh = NH;
        e.hd = HD;
        TRY(ln_gemm(blk->norm1_w, blk->norm1_b, WS, blk->qkv_w, nullptr, 3 * E, &e, ln1_ready));
    } else {
        TRY(ln_gemm(blk->norm1_w, blk->norm1_b, WS, blk->qkv_w, b.qkv, 3 * E, nullptr, ln1_ready));
        TRY(mi355_vit_qkv_rope(ctx, b.qkv, blk->qkv_b, blk->freqs_cis, b.q, b.k, b.v, M, N, NH, HD));
    }
    // attention; for quantized / F16 proj weights it writes the projection's operand
    const int mp = ctx->fuse ? act_mode_for_weight(&blk->proj_w) : ACT_F32;
    {
        const mi355_tensor q = dev_tensor(b.q, T_F16, HD, N, NH, B), k = dev_tensor(b.k, T_F16, HD, N, NH, B),
                           v = dev_tensor(b.v, T_F16, HD, N, NH, B), o = dev_tensor(b.attn, T_F32, HD, NH, N, B);
        const ActOut op = act_out(b, mp, M, E);
        TRY(flash_attn_act(ctx, &q, &k, &v, nullptr, 1.0f / sqrtf((float)HD), 0.0f, 0.0f, &o,
                           mp == ACT_F32 ? nullptr : &op));
    }
    // proj (+ bias, window unpartition, residual: fused into the GEMM's epilogue)
    if (mp == ACT_F32) {
        const mi355_tensor in = dev_tensor(b.attn, T_F32, E, M), out = dev_tensor(b.xn, T_F32, E, M);
        TRY(mi355_mul_mat(ctx, &blk->proj_w, &in, &out));
        TRY(mi355_vit_proj_residual(ctx, x, b.xn, blk->proj_b, M, E, G, WS));
    } else {
        MmqEpi e{};
        e.kind = MMQ_EPI_RESIDUAL;
        e.bias = blk->proj_b;
        e.res = x;
        e.out = x;
        e.map = RowMap{WS > 0 ? ROWMAP_WIN_UNPART : ROWMAP_IDENTITY, G, G, WS, 0};
        TRY(mul_mat_epi(ctx, &blk->proj_w, act_in(b, mp, M, E), e));
    }
    // MLP: fc1, bias + GELU writing fc2's operand, fc2 (+ bias, residual: fused epilogue)
    const int m2 = ctx->fuse && MLP % 32 == 0 ? act_mode_for_weight(&blk->fc2_w) : ACT_F32;
    TRY(ln_gemm(blk->norm2_w, blk->norm2_b, 0, blk->fc1_w, b.big, MLP, nullptr));
    if (m2 == ACT_F32) {
        TRY(mi355_vit_bias_gelu(ctx, b.big, blk->fc1_b, M, MLP));
    } else {
        Timed t(ctx, "bias_gelu");
        TRY(hip_check(ctx, t.done(launch_bias_gelu_act(b.big, blk->fc1_b, M, MLP, act_out(b, m2, M, MLP, true), ctx->stream)),
                      "bias_gelu launch"));
    }
    if (m2 == ACT_F32) {
        const mi355_tensor in = dev_tensor(b.big, T_F32, MLP, M), out = dev_tensor(b.attn, T_F32, E, M);
        TRY(mi355_mul_mat(ctx, &blk->fc2_w, &in, &out));
        TRY(mi355_vit_bias_residual(ctx, x, b.attn, blk->fc2_b, M, E));
    } else {
        MmqEpi e{};
        e.kind = MMQ_EPI_RESIDUAL;
        e.bias = blk->fc2_b;
        e.res = x;
        e.out = x;
        e.map = RowMap{ROWMAP_IDENTITY, 0, 0, 0, 0};
        // the next block's LN1 (its qkv operand) handed to the int8 route with this residual
        const int WSn = next ? (next->is_global ? 0 : hp->window_size) : 0;
        const int mn = next && ctx->fuse ? act_mode_for_weight(&next->qkv_w) : ACT_F32;
        LnArgs la;
        if (ln_next_done && mn != ACT_F32 && blk->fc2_w.layout == MI355_LAYOUT_INT8 && next->norm1_w &&
            next->norm1_b && (WSn == 0 || (WSn > 0 && G % WSn == 0))) {
            la.x = x;
            la.add = nullptr;
            la.add_grid = 0;
            la.w = next->norm1_w;
            la.b = next->norm1_b;
            la.out = act_out(b, mn, M, E);
            la.rows = M;
            la.E = E;
            la.grid = G;
            la.ws = WSn;
            la.eps = hp->eps;
            e.ln_next = &la;
        }
        TRY(mul_mat_epi(ctx, &blk->fc2_w, act_in(b, m2, M, MLP, true), e));
        if (e.ln_next) *ln_next_done = true;
    }
#undef TRY
    return MI355_STATUS_SUCCESS;
}

mi355_status mi355_vit_block_forward(mi355_context* ctx, const mi355_vit_hparams* hp, const mi355_vit_block* blk,
                                     float* x) {
    return block_forward(ctx, hp, blk, x, nullptr, false, nullptr);
}

mi355_status mi355_vit_encode(mi355_context* ctx, const mi355_vit_hparams* hp, const float* image,
                              const mi355_tensor* patch_w, const float* pos_embed, const float* ln_pre_w,
                              const float* ln_pre_b, const mi355_vit_block* blocks, int n_blocks, float* x) {
    if (n_blocks < 0 || (n_blocks > 0 && !blocks)) return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_encode: bad blocks");
    mi355_status st = mi355_vit_prefix(ctx, hp, image, patch_w, pos_embed, ln_pre_w, ln_pre_b, x);
    bool ready = false;  // block i's LN1 already ran in block i - 1's fc2
    for (int i = 0; i < n_blocks && st == MI355_STATUS_SUCCESS; ++i) {
        bool done = false;
        st = block_forward(ctx, hp, &blocks[i], x, i + 1 < n_blocks ? &blocks[i + 1] : nullptr, ready, &done);
        ready = done;
    }
    return st;
}

}  // extern "C"
