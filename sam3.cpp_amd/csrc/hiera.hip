// Memory-bound ops of the SAM2 Hiera image encoder (sam2_hiera_block_forward,
// sam3.cpp:4299-4461, and the patch embedding of sam2_build_hiera_graph,
// sam3.cpp:4473-4496), each fusing the ggml nodes that touch one tensor.
// Token layouts: image order t = h*W + w (ggml [C, W, H]); window order of
// sam2_window_partition: window n = wh + nW_h*ww over the zero-padded grid,
// token lh*ws + lw inside it.  Every ggml node rounds to fp32 and so does
// each fused step: no FMA contraction in this file.
#pragma clang fp contract(off)
#include <algorithm>

#include "common.cuh"
#include "kernels.h"

namespace mi355 {

__device__ __forceinline__ double wave_sum_dh(double v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// ggml_norm(eps) -> mul(w) -> add(b) over rows of C, G lanes per row (C =
// 4*G*V), float4 loads.  ws > 0: output rows in window order (padding rows
// zero) and, when out_img is set, the same rows also in image order.
// MODE >= 0: the output mode of out (and out_img when used) fixed at compile time
template <int V, int MODE = -1>
__global__ __launch_bounds__(256) void hiera_ln_group_kernel(HieraLnArgs a, int G) {
    if (MODE >= 0) a.out.mode = a.out_img.mode = MODE;
    const int64_t r = (int64_t)blockIdx.x * (256 / G) + threadIdx.x / G;
    if (r >= a.rows_out) return;
    const int l = threadIdx.x & (G - 1), C = a.C;
    const int64_t src = a.ws > 0 ? hwin_src(r, a.W, a.H, a.ws, a.nwh) : r;
    v4f x[V];
    if (src < 0) {  // padding token: a zero row
#pragma unroll
        for (int v = 0; v < V; ++v) act_store_chunk(a.out, r, C, v * G + l, v4f{0.0f, 0.0f, 0.0f, 0.0f});
        return;
    }
    const float* xr = a.x + src * C;
#pragma unroll
    for (int v = 0; v < V; ++v) x[v] = *reinterpret_cast<const v4f*>(xr + 4 * (v * G + l));
    ln_group<V>(x, l, G, C, a.w, a.b, a.eps);
    const bool img = a.ws > 0 && (a.out_img.y || a.out_img.q);
#pragma unroll
    for (int v = 0; v < V; ++v) {
        act_store_chunk(a.out, r, C, v * G + l, x[v]);
        if (img) act_store_chunk(a.out_img, src, C, v * G + l, x[v]);
    }
}

// One wavefront per output row, for rows the grouped form does not fit
// (C <= 2048).
__global__ __launch_bounds__(256) void hiera_ln_kernel(const HieraLnArgs a) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= a.rows_out) return;
    const int lane = threadIdx.x & 63, C = a.C;
    const int per = (C + 63) / 64;
    const int64_t src = a.ws > 0 ? hwin_src(r, a.W, a.H, a.ws, a.nwh) : r;
    const bool img = a.ws > 0 && src >= 0 && (a.out_img.y || a.out_img.q);
    if (src < 0) {  // padding token: a zero row
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            const int e = j * 64 + lane;
            if (j < per) act_store_lane32(a.out, r, C, e, 0.0f, e < C);
        }
        return;
    }
    const float* xr = a.x + src * C;
    float v[32];
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const int e = j * 64 + lane;
        if (j < per && e < C) {
            v[j] = xr[e];
            s += (double)v[j];
        }
    }
    s = wave_sum_dh(s);
    const float mean = (float)(s / (double)C);
    double s2 = 0.0;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const int e = j * 64 + lane;
        if (j < per && e < C) {
            const float t = v[j] - mean;
            v[j] = t;
            s2 += (double)(t * t);
        }
    }
    s2 = wave_sum_dh(s2);
    const float var = (float)(s2 / (double)C);
    const float scale = 1.0f / sqrtf(var + a.eps);
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        if (j < per) {
            const int e = j * 64 + lane;
            const bool valid = e < C;
            float t = 0.0f;
            if (valid) {
                t = v[j] * scale;
                t = t * a.w[e];
                t = t + a.b[e];
            }
            act_store_lane32(a.out, r, C, e, t, valid);
            if (img) act_store_lane32(a.out_img, src, C, e, t, valid);
        }
    }
}

// K, V: thread per (attention batch bw, token t, head h, element pair i)
__global__ __launch_bounds__(256) void hiera_kv_kernel(const HieraQkvArgs a) {
    const int half = a.HD / 2, C = a.NH * a.HD;
    const int64_t tix = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = (int64_t)a.B * a.Nkv * a.NH * half;
    if (tix >= total) return;
    const int i = (int)(tix % half);
    const int h = (int)((tix / half) % a.NH);
    const int64_t t = (tix / ((int64_t)half * a.NH)) % a.Nkv;
    const int64_t bw = tix / ((int64_t)half * a.NH * a.Nkv);
    const int e = h * a.HD + 2 * i;
    const float* row = a.qkv + (bw * a.Nkv + t) * (int64_t)(3 * C);
    const float k0 = row[C + e] + a.bias[C + e], k1 = row[C + e + 1] + a.bias[C + e + 1];
    const float v0 = row[2 * C + e] + a.bias[2 * C + e], v1 = row[2 * C + e + 1] + a.bias[2 * C + e + 1];
    const int64_t o = ((bw * a.NH + h) * a.Nkv + t) * a.HD + 2 * i;
    *reinterpret_cast<uint32_t*>(a.k + o) = (uint32_t)f2h(k0) | ((uint32_t)f2h(k1) << 16);
    *reinterpret_cast<uint32_t*>(a.v + o) = (uint32_t)f2h(v0) | ((uint32_t)f2h(v1) << 16);
}

// Q: thread per (bw, query tq, head h, pair i); with q_pool, the 2x2 max of the
// window's (ws x ws) token grid (sam2_maxpool_2d inside each window)
__global__ __launch_bounds__(256) void hiera_q_kernel(const HieraQkvArgs a) {
    const int half = a.HD / 2, C = a.NH * a.HD;
    const int64_t tix = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = (int64_t)a.B * a.Nq * a.NH * half;
    if (tix >= total) return;
    const int i = (int)(tix % half);
    const int h = (int)((tix / half) % a.NH);
    const int64_t tq = (tix / ((int64_t)half * a.NH)) % a.Nq;
    const int64_t bw = tix / ((int64_t)half * a.NH * a.Nq);
    const int e = h * a.HD + 2 * i;
    const float b0 = a.bias[e], b1 = a.bias[e + 1];
    float q0, q1;
    if (a.qpool) {
        const int wo = a.ws / 2;
        const int ph = (int)(tq / wo), pw = (int)(tq % wo);
        q0 = q1 = -__builtin_inff();
#pragma unroll
        for (int dy = 0; dy < 2; ++dy)
#pragma unroll
            for (int dx = 0; dx < 2; ++dx) {
                const int64_t t = (int64_t)(2 * ph + dy) * a.ws + 2 * pw + dx;
                const float* row = a.qkv + (bw * a.Nkv + t) * (int64_t)(3 * C);
                q0 = fmaxf(q0, row[e] + b0);
                q1 = fmaxf(q1, row[e + 1] + b1);
            }
    } else {
        const float* row = a.qkv + (bw * a.Nkv + tq) * (int64_t)(3 * C);
        q0 = row[e] + b0;
        q1 = row[e + 1] + b1;
    }
    const int64_t o = ((bw * a.NH + h) * a.Nq + tq) * a.HD + 2 * i;
    *reinterpret_cast<uint32_t*>(a.q + o) = (uint32_t)f2h(q0) | ((uint32_t)f2h(q1) << 16);
}

// Q of a pooled block from the unpooled fp16 q [B][NH][Nkv][HD] (q + bias rounded, as the
// GEMM's qkv epilogue writes it): the 2x2 max inside each window's ws x ws token grid
// (sam2_maxpool_2d) into [B][NH][Nq][HD].  Rounding to fp16 is monotonic, so the max of the
// rounded values is the rounded max: the same bits as pooling in fp32 and rounding once
// (hiera_q_kernel).  Thread per (bw, head h, query tq, pair i).
__global__ __launch_bounds__(256) void hiera_qpool_kernel(const _Float16* __restrict__ qf, _Float16* __restrict__ q,
                                                          int64_t B, int NH, int Nkv, int Nq, int ws, int HD) {
    const int half = HD / 2;
    const int64_t tix = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (tix >= B * NH * Nq * half) return;
    const int i = (int)(tix % half);
    const int tq = (int)((tix / half) % Nq);
    const int64_t bh = tix / ((int64_t)half * Nq);  // bw * NH + h
    const int wo = ws / 2, ph = tq / wo, pw = tq - ph * wo;
    float q0 = -__builtin_inff(), q1 = -__builtin_inff();
#pragma unroll
    for (int dy = 0; dy < 2; ++dy)
#pragma unroll
        for (int dx = 0; dx < 2; ++dx) {
            const int t = (2 * ph + dy) * ws + 2 * pw + dx;
            const uint32_t w = *reinterpret_cast<const uint32_t*>(qf + (bh * Nkv + t) * HD + 2 * i);
            q0 = fmaxf(q0, h2f((uint16_t)(w & 0xffffu)));
            q1 = fmaxf(q1, h2f((uint16_t)(w >> 16)));
        }
    *reinterpret_cast<uint32_t*>(q + (bh * Nq + tq) * HD + 2 * i) = (uint32_t)f2h(q0) | ((uint32_t)f2h(q1) << 16);
}

// pool: out[h2][w2] = max over 2x2 of (p[t] (+ b)); else out[t] = p[t] (+ b); rows of C
__global__ __launch_bounds__(256) void hiera_bias_maxpool_kernel(const float* __restrict__ p, const float* __restrict__ b,
                                                                 float* __restrict__ out, int C, int W, int H, int pool) {
    if (!pool) {
        const int64_t tix = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
        if (tix >= (int64_t)W * H * C) return;
        out[tix] = b ? p[tix] + b[tix % C] : p[tix];
        return;
    }
    const int W2 = W / 2, H2 = H / 2;
    const int64_t tix = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (tix >= (int64_t)W2 * H2 * C) return;
    const int c = (int)(tix % C);
    const int64_t t2 = tix / C;
    const int w2 = (int)(t2 % W2), h2 = (int)(t2 / W2);
    const float bc = b ? b[c] : 0.0f;
    float m = -__builtin_inff();
#pragma unroll
    for (int dy = 0; dy < 2; ++dy)
#pragma unroll
        for (int dx = 0; dx < 2; ++dx) {
            float v = p[((int64_t)(2 * h2 + dy) * W + 2 * w2 + dx) * C + c];
            if (b) v = v + bc;
            m = fmaxf(m, v);
        }
    out[tix] = m;
}

// x[t] = shortcut[t] + (p[row(t)] + b) over the image grid W x H (rows of C);
// row(t) = window-order row for windows of ws (grid padded to a multiple of
// ws, nwh windows along H), or t when ws == 0
__global__ __launch_bounds__(256) void hiera_proj_residual_kernel(float* x, const float* shortcut,
                                                                  const float* __restrict__ p,
                                                                  const float* __restrict__ b, int C, int W, int H,
                                                                  int ws, int nwh) {
    const int64_t tix = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (tix >= (int64_t)W * H * C) return;
    const int c = (int)(tix % C);
    const int64_t t = tix / C;
    int64_t r = t;
    if (ws > 0) {
        const int w = (int)(t % W), h = (int)(t / W);
        const int64_t n = h / ws + (int64_t)nwh * (w / ws);
        r = (n * ws + h % ws) * ws + w % ws;
    }
    const float u = p[r * C + c] + b[c];
    x[tix] = shortcut[tix] + u;
}

// h = ggml_gelu(h + b) with ggml-cpu's fp16-table semantics (GGML_GELU_FP16):
// 0 for x <= -10, x for x >= 10, else f16(gelu_f32(f16(x))).
__global__ __launch_bounds__(256) void bias_gelu_tanh_kernel(float* __restrict__ h, const float* __restrict__ b,
                                                             int64_t rows, int n) {
    const int64_t tix = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (tix >= rows * n) return;
    const int c = (int)(tix % n);
    const float y = gelu_tanh_table(h[tix] + b[c]);
    h[tix] = y;
}

// h + b -> ggml_gelu -> the next MUL_MAT's operand; one thread per 4 values
// (n % 32 == 0, so the 8 threads of a block are lanes of one wavefront)
__global__ __launch_bounds__(256) void bias_gelu_tanh_act_kernel(const float* __restrict__ h, const float* __restrict__ b,
                                                                 int64_t rows, int n, const ActOut o) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int n4 = n / 4;
    if (t >= rows * n4) return;
    const int64_t r = t / n4;
    const int c = (int)(t - r * n4);
    const v4f hv = *reinterpret_cast<const v4f*>(h + r * n + 4 * c);
    const v4f bv = *reinterpret_cast<const v4f*>(b + 4 * c);
    v4f x;
#pragma unroll
    for (int k = 0; k < 4; ++k) x[k] = gelu_tanh_table(hv[k] + bv[k]);
    act_store_chunk(o, r, n, c, x);
}

// conv2d columns with stride / zero padding: cols[m][k], m = oy*OW + ox,
// k = (c*KH + ky)*KW + kx, rows of pitch kp >= K = C*KH*KW floats with the columns past K
// zero (a pitch the fp32 GEMM's 16-byte chunks take whole); optionally rounded to fp16
// (F16 kernels, ggml_im2col F16). Grid-stride over the n = OH OW K elements, consecutive
// threads on consecutive columns so the stores coalesce (a thread per kernel row writing
// KW columns was slower: 47 against 32 us at 1024^2); rc = {1/K, 1/(KH KW), 1/KW, 1/OW}
// when n plus the grid stays below 2^31: the indices then come from div_rcp instead of
// 64- and 32-bit divisions; else rc.k = 0.
struct Im2colRcp {
    double k, kk, kw, ow;
};
__global__ __launch_bounds__(256) void im2col_pad_kernel(const float* __restrict__ img, float* __restrict__ cols, int C,
                                                         int Hin, int Win, int KH, int KW, int stride, int pad, int OH,
                                                         int OW, int kp, int round16, Im2colRcp rc) {
    const int K = C * KH * KW;
    const int64_t n = (int64_t)OH * OW * K, step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t tix = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; tix < n; tix += step) {
        int k, kx, ky, c, ox, oy;
        int64_t m;
        if (rc.k != 0.0) {
            int r;
            m = div_rcp((int)tix, K, rc.k, k);
            c = div_rcp(k, KH * KW, rc.kk, r);
            ky = div_rcp(r, KW, rc.kw, kx);
            oy = div_rcp((int)m, OW, rc.ow, ox);
        } else {
            k = (int)(tix % K);
            m = tix / K;
            kx = k % KW;
            ky = (k / KW) % KH;
            c = k / (KW * KH);
            ox = (int)(m % OW);
            oy = (int)(m / OW);
        }
        const int y = oy * stride - pad + ky, xx = ox * stride - pad + kx;
        float v = (y >= 0 && y < Hin && xx >= 0 && xx < Win) ? img[((int64_t)c * Hin + y) * Win + xx] : 0.0f;
        if (round16) v = h2f(f2h(v));
        cols[m * kp + k] = v;
        if (k == K - 1)
            for (int j = K; j < kp; ++j) cols[m * kp + j] = 0.0f;
    }
}

// dst[r][k] = src[r][k] (F32, or F16 widened) for k < K, 0 for K <= k < kp: a weight
// matrix at the zero-padded pitch of the im2col columns
__global__ __launch_bounds__(256) void pad_rows_f32_kernel(const void* __restrict__ src, int f16, int64_t rows, int K,
                                                           int kp, float* __restrict__ dst) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= rows * kp) return;
    const int64_t r = t / kp;
    const int k = (int)(t - r * kp);
    float v = 0.0f;
    if (k < K) v = f16 ? h2f(static_cast<const uint16_t*>(src)[r * K + k]) : static_cast<const float*>(src)[r * K + k];
    dst[t] = v;
}

static unsigned nblk(int64_t n) { return (unsigned)((n + 255) / 256); }

hipError_t launch_hiera_ln(const HieraLnArgs& a, hipStream_t st) {
    if (a.rows_out <= 0) return hipSuccess;
    if (a.C <= 0 || a.C > 2048) return hipErrorInvalidValue;
    const bool q8 = a.out.mode >= ACT_Q8 || (a.ws > 0 && a.out_img.mode >= ACT_Q8 && (a.out_img.y || a.out_img.q));
    if (q8 && a.C % 32 != 0) return hipErrorInvalidValue;
    int G, V;
    ln_shape(a.C, &G, &V);
    const unsigned nb = (unsigned)((a.rows_out + 256 / G - 1) / (256 / G));
    switch (V) {
        case 1: hiera_ln_group_kernel<1><<<nb, 256, 0, st>>>(a, G); break;
        case 2: hiera_ln_group_kernel<2><<<nb, 256, 0, st>>>(a, G); break;
        case 3: {
            // the encoders' operands (int8 or F16), out_img unused or in the same mode
            const int m = a.out.mode;
            const bool one = !(a.ws > 0 && (a.out_img.y || a.out_img.q)) || a.out_img.mode == m;
            if (one && m == ACT_I8) hiera_ln_group_kernel<3, ACT_I8><<<nb, 256, 0, st>>>(a, G);
            else if (one && m == ACT_F16) hiera_ln_group_kernel<3, ACT_F16><<<nb, 256, 0, st>>>(a, G);
            else hiera_ln_group_kernel<3><<<nb, 256, 0, st>>>(a, G);
            break;
        }
        case 4: hiera_ln_group_kernel<4><<<nb, 256, 0, st>>>(a, G); break;
        case 5: hiera_ln_group_kernel<5><<<nb, 256, 0, st>>>(a, G); break;
        case 6: hiera_ln_group_kernel<6><<<nb, 256, 0, st>>>(a, G); break;
        case 7: hiera_ln_group_kernel<7><<<nb, 256, 0, st>>>(a, G); break;
        case 8: hiera_ln_group_kernel<8><<<nb, 256, 0, st>>>(a, G); break;
        default: hiera_ln_kernel<<<(unsigned)((a.rows_out + 3) / 4), 256, 0, st>>>(a); break;
    }
    return hipGetLastError();
}
hipError_t launch_hiera_qpool(const _Float16* qf, _Float16* q, int64_t B, int NH, int Nkv, int Nq, int ws, int HD,
                              hipStream_t st) {
    if (HD % 2 || ws % 2 || Nkv != ws * ws || Nq * 4 != Nkv) return hipErrorInvalidValue;
    const int64_t n = B * NH * Nq * (HD / 2);
    if (n > 0) hiera_qpool_kernel<<<nblk(n), 256, 0, st>>>(qf, q, B, NH, Nkv, Nq, ws, HD);
    return hipGetLastError();
}
hipError_t launch_hiera_qkv(const HieraQkvArgs& a, hipStream_t st) {
    const int half = a.HD / 2;
    const int64_t nkv = (int64_t)a.B * a.Nkv * a.NH * half, nq = (int64_t)a.B * a.Nq * a.NH * half;
    if (nkv > 0) hiera_kv_kernel<<<nblk(nkv), 256, 0, st>>>(a);
    if (nq > 0) hiera_q_kernel<<<nblk(nq), 256, 0, st>>>(a);
    return hipGetLastError();
}
hipError_t launch_hiera_bias_maxpool(const float* p, const float* b, float* out, int C, int W, int H, bool pool,
                                     hipStream_t st) {
    const int64_t n = pool ? (int64_t)(W / 2) * (H / 2) * C : (int64_t)W * H * C;
    if (n > 0) hiera_bias_maxpool_kernel<<<nblk(n), 256, 0, st>>>(p, b, out, C, W, H, pool ? 1 : 0);
    return hipGetLastError();
}
hipError_t launch_hiera_proj_residual(float* x, const float* shortcut, const float* p, const float* b, int C, int W,
                                      int H, int ws, int nwh, hipStream_t st) {
    const int64_t n = (int64_t)W * H * C;
    if (n > 0) hiera_proj_residual_kernel<<<nblk(n), 256, 0, st>>>(x, shortcut, p, b, C, W, H, ws, nwh);
    return hipGetLastError();
}
hipError_t launch_bias_gelu_tanh(float* h, const float* b, int64_t rows, int n, hipStream_t st) {
    if (rows * n > 0) bias_gelu_tanh_kernel<<<nblk(rows * n), 256, 0, st>>>(h, b, rows, n);
    return hipGetLastError();
}
hipError_t launch_bias_gelu_tanh_act(const float* h, const float* b, int64_t rows, int n, const ActOut& o,
                                     hipStream_t st) {
    if (n % 32) return hipErrorInvalidValue;
    if (o.mode >= ACT_I8 && rows * (n / 16) < (int64_t)1 << 30) return launch_bias_act_i8(1, h, b, rows, n, o, st);
    if (rows * (n / 4) > 0) bias_gelu_tanh_act_kernel<<<nblk(rows * (n / 4)), 256, 0, st>>>(h, b, rows, n, o);
    return hipGetLastError();
}
hipError_t launch_im2col_pad(const float* img, float* cols, int C, int Hin, int Win, int KH, int KW, int stride, int pad,
                             int OH, int OW, int kp, bool round16, hipStream_t st) {
    const int64_t K = (int64_t)C * KH * KW, n = (int64_t)OH * OW * K;
    if (n <= 0) return hipSuccess;
    if (kp < K) return hipErrorInvalidValue;
    // about eight elements per thread
    const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>(nblk(n), (nblk(n) + 7) / 8));
    Im2colRcp rc{0.0, 0.0, 0.0, 0.0};
    if (n + (int64_t)grid * 256 < ((int64_t)1 << 31) && K > 0 && OW > 0)
        rc = Im2colRcp{1.0 / (double)K, 1.0 / (double)(KH * KW), 1.0 / (double)KW, 1.0 / (double)OW};
    im2col_pad_kernel<<<grid, 256, 0, st>>>(img, cols, C, Hin, Win, KH, KW, stride, pad, OH, OW, kp, round16 ? 1 : 0, rc);
    return hipGetLastError();
}
// sam2_compute_pos_embed (sam3.cpp:4076-4157): Keys cubic convolution
// (a = -0.75) of the background table at half-pixel source coordinates, taps
// clamped to the border and summed rows-outer as val += wy*wx*src, plus the
// window table tiled modulo ws.  One thread per output value, channel
// fastest, so the token-major rows are written contiguously; the source
// tables are a few KB and stay in cache.  No contraction: the same roundings
// as the reference's C loop.
__device__ __forceinline__ float keys_cubic(float x) {
#pragma clang fp contract(off)
    x = fabsf(x);
    if (x < 1.0f) return (1.25f * x - 2.25f) * x * x + 1.0f;
    if (x < 2.0f) return ((-0.75f * x + 3.75f) * x - 6.0f) * x + 3.0f;
    return 0.0f;
}

__global__ __launch_bounds__(256) void hiera_pos_embed_kernel(const float* __restrict__ bkg, int E, int bh, int bw,
                                                              const float* __restrict__ win, int ws, int H, int W,
                                                              float* __restrict__ out) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)H * W * E) return;
    const int e = (int)(i % E);
    const int64_t tok = i / E;
    const int y = (int)(tok / W), x = (int)(tok % W);
    const float fy = ((float)y + 0.5f) * (float)bh / (float)H - 0.5f;
    const int iy = (int)floorf(fy);
    const float dy = fy - (float)iy;
    const float fx = ((float)x + 0.5f) * (float)bw / (float)W - 0.5f;
    const int ix = (int)floorf(fx);
    const float dx = fx - (float)ix;
    const float* src = bkg + (int64_t)e * bh * bw;
    float val = 0.0f;
#pragma unroll
    for (int jj = -1; jj <= 2; ++jj) {
        const float wy = keys_cubic(dy - (float)jj);
        const int sy = min(max(iy + jj, 0), bh - 1);
#pragma unroll
        for (int ii = -1; ii <= 2; ++ii) {
            const float wx = keys_cubic(dx - (float)ii);
            const int sx = min(max(ix + ii, 0), bw - 1);
            val += wy * wx * src[sy * bw + sx];
        }
    }
    out[i] = val + win[((int64_t)e * ws + y % ws) * ws + x % ws];
}

hipError_t launch_hiera_pos_embed(const float* bkg, int E, int bh, int bw, const float* win, int ws, int H, int W,
                                  float* out, hipStream_t st) {
    const int64_t n = (int64_t)H * W * E;
    if (n > 0) hiera_pos_embed_kernel<<<nblk(n), 256, 0, st>>>(bkg, E, bh, bw, win, ws, H, W, out);
    return hipGetLastError();
}
hipError_t launch_pad_rows_f32(const void* src, bool f16, int64_t rows, int K, int kp, float* dst, hipStream_t st) {
    if (kp < K) return hipErrorInvalidValue;
    if (rows * kp > 0) pad_rows_f32_kernel<<<nblk(rows * kp), 256, 0, st>>>(src, f16 ? 1 : 0, rows, K, kp, dst);
    return hipGetLastError();
}

}  // namespace mi355
