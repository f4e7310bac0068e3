// SAM3 SimpleFPN neck (sam3_build_neck_graph, sam3.cpp:3867-3925) on the
// MI355X backend.
//
// The reference permutes the ViT output to channel-planar [W, H, E], runs
// ggml's convolutions (im2col + MUL_MAT, and conv_transpose_2d), and permutes
// each result back to [C, W, H].  Here every activation stays token-major
// [H*W][C] (= ggml [C, W, H], the layout of its input and outputs), so each
// convolution is a MUL_MAT over pixels with no permutes:
//   - conv_transpose_2d_p0 (kernel 2, stride 2): the taps do not overlap, so
//     it is one F16 GEMM [pixels x Cin] x [Cin x 4*Cout] (kernel cast to F16
//     and repacked tap-major) whose columns are scattered to the 2x map, with
//     the bias (and the GELU of scale 0): in the fp16 implicit-GEMM kernel's
//     epilogue, or (maps with Cin % 32 != 0 or unaligned rows) as a MUL_MAT
//     and a scatter pass;
//   - conv_2d_sk_p0 1x1: a GEMM with the kernel rows as they are, the bias in
//     its epilogue (F32 kernels: the tiled fp32 GEMM; F16 kernels: the fp16
//     implicit-GEMM kernel below with one tap);
//   - conv_2d_s1_ph 3x3: an implicit GEMM over the map (the kernel repacked to
//     (tap, channel) rows, no im2col) on fp32 MFMA (F32 kernels) or fp16 MFMA
//     (F16 kernels, the map rounded to fp16 as it is loaded); maps with
//     Cin % 32 != 0 or rows not 16-byte aligned take im2col (K ordered as
//     ggml's, ic-major) or the plain map + MUL_MAT + bias;
//   - pool_2d MAX 2x2 / 2.
// Each op's numerics are ggml-cpu's: operands in the kernel's type (F16
// rounded to nearest even, or F32), f32 accumulation, f32 bias adds.
#include <algorithm>

#include "context.h"

using namespace mi355;

namespace {

mi355_tensor dev_t(const void* p, int type, int64_t ne0, int64_t ne1) {
    mi355_tensor t{};
    t.type = type;
    t.ne[0] = ne0;
    t.ne[1] = ne1;
    t.ne[2] = t.ne[3] = 1;
    t.nb[0] = type == T_F32 ? 4 : 2;
    t.nb[1] = t.nb[0] * ne0;
    t.nb[2] = t.nb[3] = t.nb[1] * ne1;
    t.data = const_cast<void*>(p);
    return t;
}

bool contiguous(const mi355_tensor* w) {
    const int64_t ts = w->type == T_F32 ? 4 : 2;
    return w->nb[0] == ts && w->nb[1] == ts * w->ne[0] && w->nb[2] == w->nb[1] * w->ne[1] &&
           w->nb[3] == w->nb[2] * w->ne[2];
}

mi355_status check_kernel(mi355_context* ctx, const mi355_tensor* w, const float* b, int k, const char* what) {
    if (!w || !w->data || !b) return fail(ctx, MI355_STATUS_INVALID_ARG, "%s: null kernel or bias", what);
    if (w->type != T_F32 && w->type != T_F16)
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "%s: kernel type %d (F32 or F16)", what, w->type);
    if (w->ne[0] != k || w->ne[1] != k || w->ne[2] <= 0 || w->ne[3] <= 0 || !contiguous(w))
        return fail(ctx, MI355_STATUS_INVALID_ARG, "%s: kernel must be a contiguous [%d, %d, C, C]", what, k, k);
    return MI355_STATUS_SUCCESS;
}

// scratch bytes of each op (the MUL_MAT's own workspace is the context's); the
// conv-transpose's GEMM output D is only written when the map takes the MUL_MAT path
size_t deconv_scratch(int64_t P, int64_t Cin, int64_t Cout) {
    return align_up((size_t)(4 * Cout * Cin * 2)) + align_up((size_t)(P * 4 * Cout * 4));
}
// the implicit-GEMM kernels take maps whose rows are 16-byte aligned with Cin % 32 == 0
bool implicit_ok(const float* x, int64_t Cin) { return (reinterpret_cast<uintptr_t>(x) & 15) == 0 && Cin % 32 == 0; }
// implicit 3x3: the kernel repacked to (tap, channel) rows; otherwise the im2col
// columns in the kernel's type (x_aligned: the map's rows are 16-byte aligned). The
// implicit-GEMM kernels' K-split partial sums follow (1x1 and 3x3).
size_t conv_scratch(int64_t P, int64_t Cin, int64_t Cout, int k, int wtype, bool x_aligned) {
    const bool implicit = x_aligned && Cin % 32 == 0;
    const size_t part = wtype == T_F32 ? gemm_f32_part_bytes(P, Cout, (int64_t)k * k * Cin)
                        : implicit     ? conv_f16_part_bytes(k * k, P, Cin, Cout)
                                       : 0;
    if (k == 1) return part;
    const int64_t es = wtype == T_F32 ? 4 : 2;
    if (x_aligned && Cin % 32 == 0) return align_up((size_t)(9 * Cin * Cout * es)) + part;
    return align_up((size_t)(P * 9 * Cin * es));
}

// conv_transpose_2d_p0(kernel [2, 2, Cout, Cin], stride 2) + bias (+ GELU):
// x [H*W][Cin] -> y [(2H)*(2W)][Cout]
// (x16 / y16: fp16 maps, the fused neck's intermediates; F16 kernels on the implicit path only)
mi355_status deconv(mi355_context* ctx, const mi355_tensor* w, const float* b, const void* xv, int H, int W, bool gelu,
                    void* yv, char* scratch, bool x16 = false, bool y16 = false) {
    const float* x = static_cast<const float*>(xv);
    float* y = static_cast<float*>(yv);
    mi355_status st = check_kernel(ctx, w, b, 2, "neck_deconv");
    if (st != MI355_STATUS_SUCCESS) return st;
    const int Cout = (int)w->ne[2], Cin = (int)w->ne[3];
    const int64_t P = (int64_t)H * W;
    if (Cout % 4 != 0) return fail(ctx, MI355_STATUS_UNSUPPORTED, "neck_deconv: Cout %% 4 != 0");
    uint16_t* packed = reinterpret_cast<uint16_t*>(scratch);
    float* D = reinterpret_cast<float*>(scratch + align_up((size_t)(4 * Cout * Cin * 2)));
    {
        Timed t(ctx, "neck_deconv_pack");
        st = hip_check(ctx, t.done(launch_deconv_pack(w->data, w->type, Cin, Cout, packed, ctx->stream)), "deconv pack");
        if (st != MI355_STATUS_SUCCESS) return st;
    }
    if (implicit_ok(x, Cin)) {
        // one fp16-MFMA GEMM whose epilogue adds the bias (+ GELU) and scatters to the 2x map
        Timed t(ctx, "neck_deconv_f16");
        return hip_check(ctx, t.done(launch_conv_f16(4, x, x16, packed, b, H, W, Cin, 4 * Cout, gelu, y, y16, ctx->stream)),
                         "deconv_f16 launch");
    }
    if (x16 || y16) return fail(ctx, MI355_STATUS_FAILED, "neck_deconv: fp16 maps off the implicit path");
    const mi355_tensor s0 = dev_t(packed, T_F16, Cin, 4LL * Cout), s1 = dev_t(x, T_F32, Cin, P),
                       d = dev_t(D, T_F32, 4LL * Cout, P);
    st = mi355_mul_mat(ctx, &s0, &s1, &d);
    if (st != MI355_STATUS_SUCCESS) return st;
    Timed t(ctx, "neck_deconv_scatter");
    return hip_check(ctx, t.done(launch_deconv_scatter(D, b, H, W, Cout, gelu, y, ctx->stream)), "deconv scatter");
}

// conv_2d_sk_p0 (1x1) or conv_2d_s1_ph (3x3) + bias: x [H*W][Cin] -> y [H*W][Cout]
mi355_status conv(mi355_context* ctx, const mi355_tensor* w, const float* b, const void* xv, int H, int W, void* yv,
                  char* scratch, bool x16 = false, bool y16 = false) {
    const float* x = static_cast<const float*>(xv);
    float* y = static_cast<float*>(yv);
    if (!w) return fail(ctx, MI355_STATUS_INVALID_ARG, "neck_conv: null kernel");
    const int k = (int)w->ne[0];
    if (k != 1 && k != 3) return fail(ctx, MI355_STATUS_UNSUPPORTED, "neck_conv: kernel size %d (1 or 3)", k);
    mi355_status st = check_kernel(ctx, w, b, k, "neck_conv");
    if (st != MI355_STATUS_SUCCESS) return st;
    const int Cin = (int)w->ne[2], Cout = (int)w->ne[3];
    const int64_t P = (int64_t)H * W, K = (int64_t)k * k * Cin;
    if (Cout % 4 != 0) return fail(ctx, MI355_STATUS_UNSUPPORTED, "neck_conv: Cout %% 4 != 0");
    // F32 kernels: the tiled fp32 MFMA GEMM with the bias in its epilogue, the 3x3 as an
    // implicit GEMM over the map (no im2col) with its kernel repacked to (tap, channel)
    // rows; maps whose rows are not 16-byte aligned (or a 3x3 with Cin % 32 != 0) take
    // im2col + MUL_MAT below
    const bool aligned = (reinterpret_cast<uintptr_t>(x) & 15) == 0 && Cin % 4 == 0;
    if ((x16 || y16) && !(w->type == T_F16 && implicit_ok(x, Cin) &&
                          (k == 3 || (reinterpret_cast<uintptr_t>(w->data) & 15) == 0)))
        return fail(ctx, MI355_STATUS_FAILED, "neck_conv: fp16 maps off the implicit F16 path");
    if (w->type == T_F32 && aligned && (k == 1 || implicit_ok(x, Cin))) {
        if (k == 3) {
            Timed t(ctx, "neck_conv3x3_pack");
            st = hip_check(ctx, t.done(launch_conv3x3_pack(static_cast<const float*>(w->data), Cin, Cout,
                                                           reinterpret_cast<float*>(scratch), ctx->stream)),
                           "conv3x3 pack");
            if (st != MI355_STATUS_SUCCESS) return st;
        }
        GemmF32Args g;
        g.W = k == 3 ? reinterpret_cast<const float*>(scratch) : static_cast<const float*>(w->data);
        // the K split's partial sums follow the repacked kernel
        g.part = reinterpret_cast<float*>(scratch + (k == 3 ? align_up((size_t)(K * Cout * 4)) : 0));
        g.part_bytes = gemm_f32_part_bytes(P, Cout, K);
        g.w_nb1 = 4 * K;
        g.w_nb2 = g.w_nb3 = 4 * K * Cout;
        g.X = x;
        g.x_nb1 = 4LL * Cin;
        g.x_nb2 = g.x_nb3 = 4LL * Cin * P;
        g.D = y;
        g.d_nb1 = 4LL * Cout;
        g.d_nb2 = g.d_nb3 = 4LL * Cout * P;
        g.M = (int)P;
        g.N = Cout;
        g.K = (int)K;
        g.ne12 = g.r2 = g.r3 = 1;
        g.bias = b;
        g.conv = k == 3 ? 1 : 0;
        g.H = H;
        g.Wd = W;
        g.C = Cin;
        Timed t(ctx, k == 3 ? "neck_conv3x3_f32" : "neck_conv1x1_f32");
        return hip_check(ctx, t.done(launch_gemm_f32(g, 1, ctx->stream)), "gemm_f32 launch");
    }
    if (w->type == T_F16 && implicit_ok(x, Cin) && (k == 3 || (reinterpret_cast<uintptr_t>(w->data) & 15) == 0)) {
        // F16 kernels: an implicit GEMM on fp16 MFMA (the map rounded to fp16 as it
        // is loaded), bias in its epilogue; the 3x3 kernel repacked to (tap, channel)
        if (k == 3) {
            Timed t(ctx, "neck_conv3x3_pack");
            st = hip_check(ctx, t.done(launch_conv3x3_pack_f16(static_cast<const uint16_t*>(w->data), Cin, Cout,
                                                               reinterpret_cast<uint16_t*>(scratch), ctx->stream)),
                           "conv3x3 pack");
            if (st != MI355_STATUS_SUCCESS) return st;
        }
        const uint16_t* wk = k == 3 ? reinterpret_cast<const uint16_t*>(scratch) : static_cast<const uint16_t*>(w->data);
        // the K split's partial sums follow the repacked kernel
        float* part = reinterpret_cast<float*>(scratch + (k == 3 ? align_up((size_t)(K * Cout * 2)) : 0));
        Timed t(ctx, k == 3 ? "neck_conv3x3_f16" : "neck_conv1x1_f16");
        return hip_check(ctx, t.done(launch_conv_f16(k * k, x, x16, wk, b, H, W, Cin, Cout, false, y, y16, ctx->stream,
                                                     part, conv_f16_part_bytes(k * k, P, Cin, Cout))),
                         "conv_f16 launch");
    }
    const mi355_tensor s0 = dev_t(w->data, w->type, K, Cout), d = dev_t(y, T_F32, Cout, P);
    mi355_tensor s1 = dev_t(x, T_F32, Cin, P);
    if (k == 3) {
        // im2col in the kernel's type: F16 columns feed the F16 MUL_MAT directly
        const bool f16 = w->type == T_F16;
        Timed t(ctx, "neck_im2col3x3");
        st = hip_check(ctx, t.done(launch_im2col3x3(x, H, W, Cin, f16, scratch, ctx->stream)), "im2col3x3");
        if (st != MI355_STATUS_SUCCESS) return st;
        s1 = dev_t(scratch, f16 ? T_F16 : T_F32, K, P);
    }
    st = mi355_mul_mat(ctx, &s0, &s1, &d);
    if (st != MI355_STATUS_SUCCESS) return st;
    Timed t(ctx, "neck_bias");
    return hip_check(ctx, t.done(launch_bias_rows(y, b, P, Cout, ctx->stream)), "bias");
}

mi355_status pool(mi355_context* ctx, const float* x, int H, int W, int C, float* y) {
    if (C % 4 != 0) return fail(ctx, MI355_STATUS_UNSUPPORTED, "neck_maxpool: C %% 4 != 0");
    Timed t(ctx, "neck_maxpool");
    return hip_check(ctx, t.done(launch_maxpool2(x, H, W, C, y, ctx->stream)), "maxpool");
}

mi355_status scratch_for(mi355_context* ctx, size_t bytes, char** p) {
    mi355_status st = ensure_buffer(ctx, &ctx->neck, &ctx->neck_size, std::max<size_t>(bytes, 256));
    *p = static_cast<char*>(ctx->neck);
    return st;
}

// The fused neck keeps its intermediate maps in fp16 when every kernel is F16 and every
// convolution takes the implicit path (16-byte aligned F32 input, channel counts % 32 == 0,
// 1x1 kernels on 16 bytes)
bool fp16_maps(const float* x, int E, const mi355_neck_scale* s) {
    auto f16 = [](const mi355_tensor* t) { return t->type == T_F16; };
    auto a16 = [](const mi355_tensor* t) { return (reinterpret_cast<uintptr_t>(t->data) & 15) == 0; };
    if (!implicit_ok(x, E)) return false;
    for (int i = 0; i < 4; ++i) {
        if (!f16(s[i].conv1x1_w) || !f16(s[i].conv3x3_w) || !a16(s[i].conv1x1_w)) return false;
        if (s[i].conv1x1_w->ne[2] % 32 != 0 || s[i].conv3x3_w->ne[2] % 32 != 0) return false;
        if (i < 2 && (!f16(s[i].deconv1_w) || s[i].deconv1_w->ne[3] % 32 != 0)) return false;
    }
    return f16(s[0].deconv2_w) && s[0].deconv2_w->ne[3] % 32 == 0;
}

// Buffer plan of the whole neck: two map buffers plus the largest op scratch.
struct NeckPlan {
    size_t map = 0, scratch = 0;
    size_t total() const { return 2 * map + scratch; }
};

bool neck_plan(int E, int G, const mi355_neck_scale* s, NeckPlan* pl) {
    auto ok = [](const mi355_tensor* t) { return t && t->ne[2] > 0 && t->ne[3] > 0; };
    for (int i = 0; i < 4; ++i)
        if (!ok(s[i].conv1x1_w) || !ok(s[i].conv3x3_w) || (i < 2 && !ok(s[i].deconv1_w)) || (i == 0 && !ok(s[0].deconv2_w)))
            return false;
    const int64_t G2 = (int64_t)G * G;
    auto mapb = [&](int64_t P, int64_t C) { pl->map = std::max(pl->map, align_up((size_t)(P * C * 4))); };
    auto scr = [&](size_t b) { pl->scratch = std::max(pl->scratch, b); };
    // scale 0: deconv E->C1 (2G), GELU, deconv C1->D (4G), 1x1, 3x3
    const int64_t C1 = s[0].deconv1_w->ne[2], D0 = s[0].deconv2_w->ne[2];
    mapb(4 * G2, C1);
    mapb(16 * G2, D0);
    mapb(16 * G2, s[0].conv1x1_w->ne[3]);
    scr(deconv_scratch(G2, E, C1));
    scr(deconv_scratch(4 * G2, C1, D0));
    scr(conv_scratch(16 * G2, s[0].conv1x1_w->ne[2], s[0].conv1x1_w->ne[3], 1, s[0].conv1x1_w->type, true));
    scr(conv_scratch(16 * G2, s[0].conv3x3_w->ne[2], s[0].conv3x3_w->ne[3], 3, s[0].conv3x3_w->type, true));
    // scale 1: deconv E->C1 (2G), 1x1, 3x3
    const int64_t C1b = s[1].deconv1_w->ne[2];
    mapb(4 * G2, C1b);
    mapb(4 * G2, s[1].conv1x1_w->ne[3]);
    scr(deconv_scratch(G2, E, C1b));
    scr(conv_scratch(4 * G2, s[1].conv1x1_w->ne[2], s[1].conv1x1_w->ne[3], 1, s[1].conv1x1_w->type, true));
    scr(conv_scratch(4 * G2, s[1].conv3x3_w->ne[2], s[1].conv3x3_w->ne[3], 3, s[1].conv3x3_w->type, true));
    // scale 2: 1x1, 3x3 at G; scale 3: pool, 1x1, 3x3 at G/2
    mapb(G2, s[2].conv1x1_w->ne[3]);
    scr(conv_scratch(G2, s[2].conv1x1_w->ne[2], s[2].conv1x1_w->ne[3], 1, s[2].conv1x1_w->type, true));
    scr(conv_scratch(G2, s[2].conv3x3_w->ne[2], s[2].conv3x3_w->ne[3], 3, s[2].conv3x3_w->type, true));
    mapb(G2 / 4, E);
    mapb(G2 / 4, s[3].conv1x1_w->ne[3]);
    scr(conv_scratch(G2 / 4, s[3].conv1x1_w->ne[2], s[3].conv1x1_w->ne[3], 1, s[3].conv1x1_w->type, true));
    scr(conv_scratch(G2 / 4, s[3].conv3x3_w->ne[2], s[3].conv3x3_w->ne[3], 3, s[3].conv3x3_w->type, true));
    return true;
}

}  // namespace

extern "C" {

mi355_status mi355_neck_deconv(mi355_context* ctx, const mi355_tensor* w, const float* b, const float* x, int H, int W,
                               int gelu, float* y) {
    if (!ctx || !x || !y) return fail(ctx, MI355_STATUS_INVALID_ARG, "neck_deconv: null argument");
    if (H <= 0 || W <= 0) return fail(ctx, MI355_STATUS_INVALID_ARG, "neck_deconv: bad size");
    mi355_status st = check_kernel(ctx, w, b, 2, "neck_deconv");
    if (st != MI355_STATUS_SUCCESS) return st;
    (void)hipSetDevice(ctx->device);
    char* scr = nullptr;
    st = scratch_for(ctx, deconv_scratch((int64_t)H * W, w->ne[3], w->ne[2]), &scr);
    if (st != MI355_STATUS_SUCCESS) return st;
    return deconv(ctx, w, b, x, H, W, gelu != 0, y, scr);
}

mi355_status mi355_neck_conv(mi355_context* ctx, const mi355_tensor* w, const float* b, const float* x, int H, int W,
                             float* y) {
    if (!ctx || !x || !y || !w) return fail(ctx, MI355_STATUS_INVALID_ARG, "neck_conv: null argument");
    if (H <= 0 || W <= 0) return fail(ctx, MI355_STATUS_INVALID_ARG, "neck_conv: bad size");
    (void)hipSetDevice(ctx->device);
    char* scr = nullptr;
    const int k = (int)w->ne[0];
    const size_t sb = conv_scratch((int64_t)H * W, w->ne[2], w->ne[3], k, w->type, implicit_ok(x, w->ne[2]));
    mi355_status st = scratch_for(ctx, sb, &scr);
    if (st != MI355_STATUS_SUCCESS) return st;
    return conv(ctx, w, b, x, H, W, y, scr);
}

mi355_status mi355_neck_maxpool(mi355_context* ctx, const float* x, int H, int W, int C, float* y) {
    if (!ctx || !x || !y) return fail(ctx, MI355_STATUS_INVALID_ARG, "neck_maxpool: null argument");
    if (H <= 1 || W <= 1 || C <= 0) return fail(ctx, MI355_STATUS_INVALID_ARG, "neck_maxpool: bad size");
    (void)hipSetDevice(ctx->device);
    return pool(ctx, x, H, W, C, y);
}

size_t mi355_neck_workspace_size(int E, int G, const mi355_neck_scale scales[4]) {
    NeckPlan pl;
    if (!scales || E <= 0 || G <= 0 || !neck_plan(E, G, scales, &pl)) return 0;
    return pl.total();
}

mi355_status mi355_sam3_neck(mi355_context* ctx, const float* x, int E, int G, const mi355_neck_scale scales[4],
                             float* const out[4]) {
    if (!ctx || !x || !scales || !out) return fail(ctx, MI355_STATUS_INVALID_ARG, "sam3_neck: null argument");
    for (int i = 0; i < 4; ++i)
        if (!out[i]) return fail(ctx, MI355_STATUS_INVALID_ARG, "sam3_neck: null output %d", i);
    if (E <= 0 || G <= 1 || G % 2 != 0) return fail(ctx, MI355_STATUS_INVALID_ARG, "sam3_neck: bad E or grid");
    NeckPlan pl;
    if (!neck_plan(E, G, scales, &pl)) return fail(ctx, MI355_STATUS_INVALID_ARG, "sam3_neck: missing kernels");
    // channel chain: each op's input channels are the previous op's outputs
    const mi355_neck_scale* s = scales;
    if (s[0].deconv1_w->ne[3] != E || s[0].deconv2_w->ne[3] != s[0].deconv1_w->ne[2] ||
        s[0].conv1x1_w->ne[2] != s[0].deconv2_w->ne[2] || s[1].deconv1_w->ne[3] != E ||
        s[1].conv1x1_w->ne[2] != s[1].deconv1_w->ne[2] || s[2].conv1x1_w->ne[2] != E || s[3].conv1x1_w->ne[2] != E)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "sam3_neck: kernel channels do not chain");
    for (int i = 0; i < 4; ++i)
        if (s[i].conv3x3_w->ne[2] != s[i].conv1x1_w->ne[3])
            return fail(ctx, MI355_STATUS_INVALID_ARG, "sam3_neck: scale %d 3x3 input channels", i);
    (void)hipSetDevice(ctx->device);
    mi355_status st = ensure_buffer(ctx, &ctx->neck, &ctx->neck_size, pl.total());
    if (st != MI355_STATUS_SUCCESS) return st;
    char* base = static_cast<char*>(ctx->neck);
    float* A = reinterpret_cast<float*>(base);
    float* B = reinterpret_cast<float*>(base + pl.map);
    char* scr = base + 2 * pl.map;
#define TRY(e)                                     \
    do {                                           \
        st = (e);                                  \
        if (st != MI355_STATUS_SUCCESS) return st; \
    } while (0)
    // F16 kernels throughout, on the implicit path: the maps between two convolutions are
    // stored as fp16, the values each consumer rounds its F32 input to (the same bits out);
    // the F32 ViT output, the pool output and the four outputs stay F32
    const bool h = fp16_maps(x, E, s);
    // the conv-transposes run F16 kernels whatever the weight type (ggml casts their kernels
    // and inputs to F16), so scale 0's first one hands the second an fp16 map whenever both
    // take the implicit path
    const bool hd = h || (implicit_ok(x, E) && s[0].deconv1_w->ne[2] % 32 == 0);
    // scale 0 (4x): deconv + GELU, deconv, 1x1, 3x3
    TRY(deconv(ctx, s[0].deconv1_w, s[0].deconv1_b, x, G, G, true, A, scr, false, hd));
    TRY(deconv(ctx, s[0].deconv2_w, s[0].deconv2_b, A, 2 * G, 2 * G, false, B, scr, hd, h));
    TRY(conv(ctx, s[0].conv1x1_w, s[0].conv1x1_b, B, 4 * G, 4 * G, A, scr, h, h));
    TRY(conv(ctx, s[0].conv3x3_w, s[0].conv3x3_b, A, 4 * G, 4 * G, out[0], scr, h, false));
    // scale 1 (2x): deconv, 1x1, 3x3
    TRY(deconv(ctx, s[1].deconv1_w, s[1].deconv1_b, x, G, G, false, A, scr, false, h));
    TRY(conv(ctx, s[1].conv1x1_w, s[1].conv1x1_b, A, 2 * G, 2 * G, B, scr, h, h));
    TRY(conv(ctx, s[1].conv3x3_w, s[1].conv3x3_b, B, 2 * G, 2 * G, out[1], scr, h, false));
    // scale 2 (1x): 1x1, 3x3
    TRY(conv(ctx, s[2].conv1x1_w, s[2].conv1x1_b, x, G, G, A, scr, false, h));
    TRY(conv(ctx, s[2].conv3x3_w, s[2].conv3x3_b, A, G, G, out[2], scr, h, false));
    // scale 3 (0.5x): max-pool, 1x1, 3x3
    TRY(pool(ctx, x, G, G, E, B));
    TRY(conv(ctx, s[3].conv1x1_w, s[3].conv1x1_b, B, G / 2, G / 2, A, scr, false, h));
    TRY(conv(ctx, s[3].conv3x3_w, s[3].conv3x3_b, A, G / 2, G / 2, out[3], scr, h, false));
#undef TRY
    return MI355_STATUS_SUCCESS;
}

}  // extern "C"
