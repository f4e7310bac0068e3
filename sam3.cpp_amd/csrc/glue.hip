// Memory-bound ops of the SAM3 ViT image encoder around the MUL_MAT and
// FLASH_ATTN_EXT nodes, each fusing the ggml nodes that touch the same
// tensor once.  Every ggml node rounds its result to fp32, so each fused
// step keeps that rounding: no FMA contraction in this file.
//   ln_kernel          ggml_norm(eps) -> mul(w) -> add(b) (sam3_layer_norm,
//                      sam3.cpp:1041-1051), with an optional preceding add
//                      (patch + tiled pos_embed, sam3.cpp:3820-3826) and the
//                      ggml_win_part token order on output (sam3.cpp:3734)
//   qkv_rope_kernel    add(qkv_b), Q/K/V split + permute (sam3.cpp:3742-3767),
//                      sam3_apply_rope on Q and K (sam3.cpp:3671-3710); writes
//                      fp16 Q/K/V [B][NH][N][HD] for FLASH_ATTN_EXT
//   proj_residual_kernel  add(proj_b) -> ggml_win_unpart -> add(shortcut)
//                      (sam3.cpp:3783-3791)
//   bias_gelu_kernel   add(fc1_b) -> ggml_gelu_erf (sam3.cpp:3796-3797)
//   bias_residual_kernel  add(fc2_b) -> add(shortcut) (sam3.cpp:3799-3802)
//   im2col_kernel      ggml_conv_2d_sk_p0 input columns (sam3.cpp:3815)
#pragma clang fp contract(off)
#include <algorithm>

#include "common.cuh"
#include "kernels.h"

namespace mi355 {

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// token r of a grid x grid image (row-major, r = y*grid + x) -> its row in
// ggml_win_part order (window (y/ws, x/ws) row-major, then y%ws, x%ws)
__device__ __forceinline__ int64_t win_row(int64_t r, int grid, int ws) {
    const int y = (int)(r / grid), x = (int)(r % grid);
    const int nwx = grid / ws;
    return (((int64_t)(y / ws) * nwx + x / ws) * ws + y % ws) * ws + x % ws;
}

// Row r's addend row: the same row, or the pos_embed [pg x pg] table tiled
// over the grid x grid image
__device__ __forceinline__ const float* ln_addend(const LnArgs& a, int64_t r) {
    if (!a.add) return nullptr;
    int64_t pr = r;
    if (a.add_grid > 0) {
        const int y = (int)(r / a.grid), x = (int)(r % a.grid);
        pr = (int64_t)(y % a.add_grid) * a.add_grid + x % a.add_grid;
    }
    return a.add + pr * a.E;
}

// ln_group_kernel at E = 1024: one wavefront per row, lane l holding the 16 consecutive
// values 16l .. 16l + 15 (half a 32-block), so the operand's blocks are quantized by lane
// pairs (act_store_half16) instead of groups of eight lanes.  MODE >= 0 fixes the output
// mode at compile time (the int8 and F16 operands of the encoders), -1 reads a.out.mode.
template <int MODE>
__global__ __launch_bounds__(256) void ln1024_kernel(LnArgs a) {
    if (MODE >= 0) a.out.mode = MODE;
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= a.rows) return;
    const int l = threadIdx.x & 63;
    const float* xr = a.x + r * 1024;
    const float* ar = ln_addend(a, r);
    v4f x[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int c = l * 4 + v;
        x[v] = *reinterpret_cast<const v4f*>(xr + 4 * c);
        if (ar) x[v] = x[v] + *reinterpret_cast<const v4f*>(ar + 4 * c);
    }
    ln_group<4, true>(x, l, 64, 1024, a.w, a.b, a.eps);
    const int64_t orow = a.ws > 0 ? win_row(r, a.grid, a.ws) : r;
    float y[16];
#pragma unroll
    for (int v = 0; v < 4; ++v)
#pragma unroll
        for (int i = 0; i < 4; ++i) y[4 * v + i] = x[v][i];
    act_store_half16(a.out, orow, 1024, l, y);
}

// The K-split reduction of a 1024-wide residual GEMM followed by the next LayerNorm, in one
// pass: one wavefront per row, lane l holding columns 16l .. 16l + 15.  x = x + ((p_0 + ... +
// p_{ks-1}) + bias) with mmq_reduce_kernel's adds in its order, written back, then that row's
// LayerNorm into a.out as ln1024_kernel computes it (a.x is this x, no addend): the bits of
// the two passes, without reading x back.
template <int KS, int MODE>
__global__ __launch_bounds__(256) void reduce_residual_ln1024_kernel(const float* __restrict__ part,
                                                                     const float* __restrict__ bias, float* x,
                                                                     LnArgs a) {
    if (MODE >= 0) a.out.mode = MODE;
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= a.rows) return;
    const int l = threadIdx.x & 63;
    const int64_t mn = a.rows * 1024;
    float* xr = x + r * 1024;
    // every load of the row issued before the first add
    v4f pv[KS][4], bv[4], xv[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int c = 4 * (l * 4 + v);
#pragma unroll
        for (int s = 0; s < KS; ++s) pv[s][v] = *reinterpret_cast<const v4f*>(part + s * mn + r * 1024 + c);
        bv[v] = *reinterpret_cast<const v4f*>(bias + c);
        xv[v] = *reinterpret_cast<const v4f*>(xr + c);
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        v4f f = pv[0][v];
#pragma unroll
        for (int s = 1; s < KS; ++s) f = f + pv[s][v];
        const v4f u = f + bv[v];
        xv[v] = xv[v] + u;
        *reinterpret_cast<v4f*>(xr + 4 * (l * 4 + v)) = xv[v];
    }
    ln_group<4, true>(xv, l, 64, 1024, a.w, a.b, a.eps);
    const int64_t orow = a.ws > 0 ? win_row(r, a.grid, a.ws) : r;
    float y[16];
#pragma unroll
    for (int v = 0; v < 4; ++v)
#pragma unroll
        for (int i = 0; i < 4; ++i) y[4 * v + i] = xv[v][i];
    act_store_half16(a.out, orow, 1024, l, y);
}

// G lanes per row (E = 4*G*V), 256/G rows per workgroup, float4 loads
template <int V>
__global__ __launch_bounds__(256) void ln_group_kernel(const LnArgs a, int G) {
    const int64_t r = (int64_t)blockIdx.x * (256 / G) + threadIdx.x / G;
    if (r >= a.rows) return;
    const int l = threadIdx.x & (G - 1), E = a.E;
    const float* xr = a.x + r * E;
    const float* ar = ln_addend(a, r);
    v4f x[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
        const int c = v * G + l;
        x[v] = *reinterpret_cast<const v4f*>(xr + 4 * c);
        if (ar) x[v] = x[v] + *reinterpret_cast<const v4f*>(ar + 4 * c);
    }
    ln_group<V>(x, l, G, E, a.w, a.b, a.eps);
    const int64_t orow = a.ws > 0 ? win_row(r, a.grid, a.ws) : r;
#pragma unroll
    for (int v = 0; v < V; ++v) act_store_chunk(a.out, orow, E, v * G + l, x[v]);
}

// One wavefront per row of E (E % 64 == 0, E <= 2048): rows the grouped form
// does not fit.
__global__ __launch_bounds__(256) void ln_kernel(const LnArgs a) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= a.rows) return;
    const int lane = threadIdx.x & 63, E = a.E, per = E / 64;
    const float* xr = a.x + r * E;
    const float* ar = ln_addend(a, r);
    float v[32];
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        if (j < per) {
            float t = xr[j * 64 + lane];
            if (ar) t = t + ar[j * 64 + lane];
            v[j] = t;
            s += (double)t;
        }
    }
    s = wave_sum_d(s);
    const float mean = (float)(s / (double)E);
    double s2 = 0.0;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        if (j < per) {
            const float t = v[j] - mean;
            v[j] = t;
            s2 += (double)(t * t);
        }
    }
    s2 = wave_sum_d(s2);
    const float var = (float)(s2 / (double)E);
    const float scale = 1.0f / sqrtf(var + a.eps);
    const int64_t orow = a.ws > 0 ? win_row(r, a.grid, a.ws) : r;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        if (j < per) {
            const int e = j * 64 + lane;
            float t = v[j] * scale;
            if (a.w) t = t * a.w[e];
            if (a.b) t = t + a.b[e];
            act_store_lane32(a.out, orow, E, e, t, true);
        }
    }
}

// thread per (token row m, head h, pair i): rows m of qkv are [q | k | v] of E each
__global__ __launch_bounds__(256) void qkv_rope_kernel(const QkvArgs a) {
    const int half = a.HD / 2;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = (int64_t)a.M * a.NH * half;
    if (t >= total) return;
    const int i = (int)(t % half);
    const int h = (int)((t / half) % a.NH);
    const int64_t m = t / ((int64_t)half * a.NH);
    const int E = a.NH * a.HD;
    const int64_t bwin = m / a.N, n = m % a.N;
    const int e = h * a.HD + 2 * i;
    const float* row = a.qkv + m * (int64_t)(3 * E);
    float q0 = row[e] + a.bias[e], q1 = row[e + 1] + a.bias[e + 1];
    float k0 = row[E + e] + a.bias[E + e], k1 = row[E + e + 1] + a.bias[E + e + 1];
    const float v0 = row[2 * E + e] + a.bias[2 * E + e], v1 = row[2 * E + e + 1] + a.bias[2 * E + e + 1];
    if (a.rope) {
        const float c = a.rope[n * a.HD + 2 * i], s = a.rope[n * a.HD + 2 * i + 1];
        rope_pair(q0, q1, c, s);
        rope_pair(k0, k1, c, s);
    }
    const int64_t o = ((bwin * a.NH + h) * a.N + n) * a.HD + 2 * i;
    *reinterpret_cast<uint32_t*>(a.q + o) = (uint32_t)f2h(q0) | ((uint32_t)f2h(q1) << 16);
    *reinterpret_cast<uint32_t*>(a.k + o) = (uint32_t)f2h(k0) | ((uint32_t)f2h(k1) << 16);
    *reinterpret_cast<uint32_t*>(a.v + o) = (uint32_t)f2h(v0) | ((uint32_t)f2h(v1) << 16);
}

// x[r] = x[r] + (p[row(r)] + b), 4 elements per thread; row(r) = win_part row or r
__global__ __launch_bounds__(256) void proj_residual_kernel(float* __restrict__ x, const float* __restrict__ p,
                                                            const float* __restrict__ b, int64_t rows, int E, int grid,
                                                            int ws) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int E4 = E / 4;
    if (t >= rows * E4) return;
    const int64_t r = t / E4;
    const int e = (int)(t % E4) * 4;
    const int64_t pr = ws > 0 ? win_row(r, grid, ws) : r;
    const v4f pv = *reinterpret_cast<const v4f*>(p + pr * E + e);
    const v4f bv = *reinterpret_cast<const v4f*>(b + e);
    v4f xv = *reinterpret_cast<const v4f*>(x + r * E + e);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float u = pv[j] + bv[j];
        xv[j] = xv[j] + u;
    }
    *reinterpret_cast<v4f*>(x + r * E + e) = xv;
}

// h = gelu_erf(h + b) in place over rows of n (ggml_vec_gelu_erf_f32: 0.5*x*(1 + erf(x/sqrt(2))))
__global__ __launch_bounds__(256) void bias_gelu_kernel(float* __restrict__ h, const float* __restrict__ b, int64_t rows,
                                                        int n) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int n4 = n / 4;
    if (t >= rows * n4) return;
    const int64_t r = t / n4;
    const int c = (int)(t % n4) * 4;
    v4f hv = *reinterpret_cast<const v4f*>(h + r * n + c);
    const v4f bv = *reinterpret_cast<const v4f*>(b + c);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        hv[j] = gelu_erf(hv[j] + bv[j]);
    }
    *reinterpret_cast<v4f*>(h + r * n + c) = hv;
}

// h + b -> gelu_erf -> the next MUL_MAT's operand; one thread per 4 values
// (n % 32 == 0, so the 8 threads of a block are lanes of one wavefront)
__global__ __launch_bounds__(256) void bias_gelu_act_kernel(const float* __restrict__ h, const float* __restrict__ b,
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
    for (int k = 0; k < 4; ++k) {
        x[k] = gelu_erf(hv[k] + bv[k]);
    }
    act_store_chunk(o, r, n, c, x);
}

// h + b -> activation -> the int8 operand (ACT_I8 / ACT_I8S) of the next MUL_MAT.  Two
// lanes per 32-value block, 16 consecutive values each: one DPP swap of the adjacent lane
// gives the block max, the two divisions serve 16 values, and the quants leave as one
// 16-byte store per lane.  A grid-stride loop issues the next half-block's loads before
// this one's arithmetic, so loads stay in flight through the activation and the quantize.
// The block's d, id and quants are those of act_store_chunk (same formulas and rounding).
// ACT 0: gelu_erf (ggml_gelu_erf); 1: gelu_tanh_table (ggml_gelu, fp16-table semantics).
// total = rows * n / 16 half-blocks (< 2^30, even since n % 32 == 0), lanes 2k and 2k+1
// hold the two halves of one block and run the same iterations.
template <int ACT, int MODE = -1>  // MODE >= 0: o.mode fixed at compile time
__global__ __launch_bounds__(256) void bias_act_i8_kernel(const float* __restrict__ h, const float* __restrict__ b,
                                                          int rows, int n, ActOut o) {
    if (MODE >= 0) o.mode = MODE;
    const int hb = n / 16, total = rows * hb, step = (int)(gridDim.x * blockDim.x);
    int t = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (t >= total) return;
    v4f hv[4], bv[4];
    {
        const int r = t / hb, j = t - r * hb;
        const float* hr = h + (int64_t)r * n + 16 * j;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            hv[i] = *reinterpret_cast<const v4f*>(hr + 4 * i);
            bv[i] = *reinterpret_cast<const v4f*>(b + 16 * j + 4 * i);
        }
    }
    for (; t < total; t += step) {
        const int r = t / hb, j = t - r * hb;
        // the next half-block's loads, issued unconditionally (the last iteration reloads its own
        // half-block): the compiler then counts them, and its waits for this iteration's data
        // leave them in flight (a conditional load would make it wait for them too)
        const int tn = t + step < total ? t + step : t;
        v4f hn[4], bn[4];
        {
            const int rn = tn / hb, jn = tn - rn * hb;
            const float* hr = h + (int64_t)rn * n + 16 * jn;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                hn[i] = *reinterpret_cast<const v4f*>(hr + 4 * i);
                bn[i] = *reinterpret_cast<const v4f*>(b + 16 * jn + 4 * i);
            }
        }
        float x[16], amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float u = hv[i][k] + bv[i][k];
                x[4 * i + k] = ACT == 0 ? gelu_erf(u) : gelu_tanh_table(u);
                amax = fmaxf(amax, fabsf(x[4 * i + k]));
            }
        // the adjacent lane holds the other half of this block
        amax = fmaxf(amax, lane_swap_f<1>(amax));
        const float d = amax / 127.0f;
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        uint32_t w[4];
        int isum = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q0 = (int)rintf(x[4 * i] * id), q1 = (int)rintf(x[4 * i + 1] * id);
            const int q2 = (int)rintf(x[4 * i + 2] * id), q3 = (int)rintf(x[4 * i + 3] * id);
            isum += q0 + q1 + q2 + q3;
            w[i] = (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) | ((uint32_t)(q2 & 0xff) << 16) |
                   ((uint32_t)(q3 & 0xff) << 24);
        }
        if (o.mode == ACT_I8S) isum += lane_swap<1>(isum);
        *reinterpret_cast<uint4*>(reinterpret_cast<int8_t*>(o.q) + (int64_t)r * n + 16 * j) =
            make_uint4(w[0], w[1], w[2], w[3]);
        if ((j & 1) == 0) act_store_scale(o, r, n, j >> 1, d, isum);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            hv[i] = hn[i];
            bv[i] = bn[i];
        }
    }
}

hipError_t launch_bias_act_i8(int act, const float* h, const float* b, int64_t rows, int n, const ActOut& o,
                              hipStream_t st) {
    // the kernel's 32-bit index t + step stays below 2^31: total < 2^30 and step <= total / 4 + 2^18
    if (n % 32 || o.mode < ACT_I8 || rows < 0 || rows * (n / 16) >= (int64_t)1 << 30) return hipErrorInvalidValue;
    const int64_t total = rows * (n / 16);
    if (total == 0) return hipSuccess;
    // about four half-blocks per thread, but at least 1024 workgroups while there is work for them
    const int64_t wgs = (total + 255) / 256;
    const unsigned grid = (unsigned)std::max<int64_t>(std::min<int64_t>(wgs, 1024), (wgs + 3) / 4);
    if (act == 0 && o.mode == ACT_I8) bias_act_i8_kernel<0, ACT_I8><<<grid, 256, 0, st>>>(h, b, (int)rows, n, o);
    else if (act == 0) bias_act_i8_kernel<0><<<grid, 256, 0, st>>>(h, b, (int)rows, n, o);
    else if (o.mode == ACT_I8) bias_act_i8_kernel<1, ACT_I8><<<grid, 256, 0, st>>>(h, b, (int)rows, n, o);
    else bias_act_i8_kernel<1><<<grid, 256, 0, st>>>(h, b, (int)rows, n, o);
    return hipGetLastError();
}

// x = x + (f + b) over rows of n
__global__ __launch_bounds__(256) void bias_residual_kernel(float* __restrict__ x, const float* __restrict__ f,
                                                            const float* __restrict__ b, int64_t rows, int n) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int n4 = n / 4;
    if (t >= rows * n4) return;
    const int64_t r = t / n4;
    const int c = (int)(t % n4) * 4;
    v4f xv = *reinterpret_cast<const v4f*>(x + r * n + c);
    const v4f fv = *reinterpret_cast<const v4f*>(f + r * n + c);
    const v4f bv = *reinterpret_cast<const v4f*>(b + c);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float u = fv[j] + bv[j];
        xv[j] = xv[j] + u;
    }
    *reinterpret_cast<v4f*>(x + r * n + c) = xv;
}

// cols[m][k], m = py*grid + px, k = (c*P + ky)*P + kx  <-  img[c][py*P + ky][px*P + kx]
__global__ __launch_bounds__(256) void im2col_kernel(const float* __restrict__ img, float* __restrict__ cols, int C,
                                                     int Himg, int Wimg, int P, int grid) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int K = C * P * P;
    const int64_t total = (int64_t)grid * grid * K;
    if (t >= total) return;
    const int k = (int)(t % K);
    const int64_t m = t / K;
    const int kx = k % P, ky = (k / P) % P, c = k / (P * P);
    const int px = (int)(m % grid), py = (int)(m / grid);
    const int y = py * P + ky, x = px * P + kx;
    cols[t] = (y < Himg && x < Wimg) ? img[((int64_t)c * Himg + y) * Wimg + x] : 0.0f;
}

static unsigned blocks_for(int64_t n, int per_block = 256) { return (unsigned)((n + per_block - 1) / per_block); }

hipError_t launch_reduce_residual_ln1024(const float* part, int ks, const float* bias, float* x, const LnArgs& a,
                                        hipStream_t st) {
    if (a.rows <= 0) return hipSuccess;
    if (a.E != 1024 || a.x != x || a.add || ks < 2 || ks > 4 || !part || !bias) return hipErrorInvalidValue;
    const unsigned g = blocks_for(a.rows, 4);
    const int m = a.out.mode;
    if (ks == 3 && m == ACT_I8) reduce_residual_ln1024_kernel<3, ACT_I8><<<g, 256, 0, st>>>(part, bias, x, a);
    else if (ks == 3 && m == ACT_F16) reduce_residual_ln1024_kernel<3, ACT_F16><<<g, 256, 0, st>>>(part, bias, x, a);
    else if (ks == 2) reduce_residual_ln1024_kernel<2, -1><<<g, 256, 0, st>>>(part, bias, x, a);
    else if (ks == 3) reduce_residual_ln1024_kernel<3, -1><<<g, 256, 0, st>>>(part, bias, x, a);
    else reduce_residual_ln1024_kernel<4, -1><<<g, 256, 0, st>>>(part, bias, x, a);
    return hipGetLastError();
}

hipError_t launch_layer_norm(const LnArgs& a, hipStream_t st) {
    if (a.rows <= 0) return hipSuccess;
    if (a.E % 64 != 0 || a.E > 2048) return hipErrorInvalidValue;
    if (a.E == 1024) {
        const unsigned g = blocks_for(a.rows, 4);
        if (a.out.mode == ACT_I8) ln1024_kernel<ACT_I8><<<g, 256, 0, st>>>(a);
        else if (a.out.mode == ACT_F16) ln1024_kernel<ACT_F16><<<g, 256, 0, st>>>(a);
        else ln1024_kernel<-1><<<g, 256, 0, st>>>(a);
        return hipGetLastError();
    }
    int G, V;  // E % 64 == 0: G >= 16, so each 32-block's 8 lanes share a row
    ln_shape(a.E, &G, &V);
    const unsigned nb = blocks_for(a.rows, 256 / G);
    switch (V) {
        case 1: ln_group_kernel<1><<<nb, 256, 0, st>>>(a, G); break;
        case 2: ln_group_kernel<2><<<nb, 256, 0, st>>>(a, G); break;
        case 3: ln_group_kernel<3><<<nb, 256, 0, st>>>(a, G); break;
        case 4: ln_group_kernel<4><<<nb, 256, 0, st>>>(a, G); break;
        case 5: ln_group_kernel<5><<<nb, 256, 0, st>>>(a, G); break;
        case 6: ln_group_kernel<6><<<nb, 256, 0, st>>>(a, G); break;
        case 7: ln_group_kernel<7><<<nb, 256, 0, st>>>(a, G); break;
        case 8: ln_group_kernel<8><<<nb, 256, 0, st>>>(a, G); break;
        default: ln_kernel<<<blocks_for(a.rows, 4), 256, 0, st>>>(a); break;
    }
    return hipGetLastError();
}

hipError_t launch_qkv_rope(const QkvArgs& a, hipStream_t st) {
    const int64_t total = (int64_t)a.M * a.NH * (a.HD / 2);
    if (total <= 0) return hipSuccess;
    qkv_rope_kernel<<<blocks_for(total), 256, 0, st>>>(a);
    return hipGetLastError();
}

hipError_t launch_proj_residual(float* x, const float* p, const float* b, int64_t rows, int E, int grid, int ws,
                                hipStream_t st) {
    if (E % 4) return hipErrorInvalidValue;
    proj_residual_kernel<<<blocks_for(rows * (E / 4)), 256, 0, st>>>(x, p, b, rows, E, grid, ws);
    return hipGetLastError();
}

hipError_t launch_bias_gelu(float* h, const float* b, int64_t rows, int n, hipStream_t st) {
    if (n % 4) return hipErrorInvalidValue;
    bias_gelu_kernel<<<blocks_for(rows * (n / 4)), 256, 0, st>>>(h, b, rows, n);
    return hipGetLastError();
}

hipError_t launch_bias_gelu_act(const float* h, const float* b, int64_t rows, int n, const ActOut& o, hipStream_t st) {
    if (n % 32) return hipErrorInvalidValue;
    if (o.mode >= ACT_I8 && rows * (n / 16) < (int64_t)1 << 30) return launch_bias_act_i8(0, h, b, rows, n, o, st);
    bias_gelu_act_kernel<<<blocks_for(rows * (n / 4)), 256, 0, st>>>(h, b, rows, n, o);
    return hipGetLastError();
}

hipError_t launch_bias_residual(float* x, const float* f, const float* b, int64_t rows, int n, hipStream_t st) {
    if (n % 4) return hipErrorInvalidValue;
    bias_residual_kernel<<<blocks_for(rows * (n / 4)), 256, 0, st>>>(x, f, b, rows, n);
    return hipGetLastError();
}

hipError_t launch_im2col(const float* img, float* cols, int C, int Himg, int Wimg, int P, int grid, hipStream_t st) {
    const int64_t total = (int64_t)grid * grid * C * P * P;
    im2col_kernel<<<blocks_for(total), 256, 0, st>>>(img, cols, C, Himg, Wimg, P, grid);
    return hipGetLastError();
}

}  // namespace mi355
