// SAM3 SimpleFPN neck kernels (sam3_build_neck_graph, sam3.cpp:3867-3925) on
// token-major activations [H*W][C] (ggml [C, W, H]).  The convolutions
// themselves run as MUL_MATs (mmq.hip / gemm_f32.hip); these are the passes
// around them, all HBM-bound: the conv-transpose kernel repack + F16 cast,
// the scatter of the 2x2 / stride-2 transposed convolution with its bias
// (and GELU), the F32 3x3 kernel repack for the implicit GEMM, im2col of the
// F16 3x3 / pad-1 convolution, bias adds and the 2x2 max-pool.
#include "common.cuh"
#include "kernels.h"

namespace mi355 {

namespace {
unsigned nblk(int64_t n) { return (unsigned)((n + 255) / 256); }
}

// ggml conv-transpose kernel [kW=2, kH=2, Cout, Cin] (memory [ci][co][kh][kw]),
// F32 or F16, -> F16 MUL_MAT weight rows [4*Cout][Cin], row n = (kh*2 + kw)*Cout + co.
// The F32 -> F16 cast rounds to nearest even, as ggml_cast does
// (sam3_conv_transpose_weight, sam3.cpp:1087-1090).
__global__ __launch_bounds__(256) void deconv_pack_kernel(const void* __restrict__ w, int wtype, int Cin, int Cout,
                                                          uint16_t* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= 4LL * Cout * Cin) return;
    const int ci = (int)(i % Cin);
    const int n = (int)(i / Cin), t = n / Cout, co = n % Cout;
    const int64_t src = (((int64_t)ci * Cout + co) * 2 + (t >> 1)) * 2 + (t & 1);
    out[i] = wtype == T_F16 ? static_cast<const uint16_t*>(w)[src] : f2h(static_cast<const float*>(w)[src]);
}

// y[(2py + kh)(2W) + 2px + kw][co] = D[py*W + px][(kh*2 + kw)*Cout + co] + b[co]
// (then GELU-erf, or not).  Four channels per thread; Cout % 4 == 0.
__global__ __launch_bounds__(256) void deconv_scatter_kernel(const float* __restrict__ D, const float* __restrict__ b,
                                                             int H, int W, int Cout, int gelu, float* __restrict__ y) {
    const int c4 = Cout / 4;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= 4LL * H * W * c4) return;
    const int co = (int)(i % c4) * 4;
    const int64_t pix = i / c4;
    const int W2 = 2 * W;
    const int oy = (int)(pix / W2), ox = (int)(pix % W2);
    const int64_t p = (int64_t)(oy >> 1) * W + (ox >> 1);
    const int t = (oy & 1) * 2 + (ox & 1);
    v4f v = *reinterpret_cast<const v4f*>(&D[p * 4 * Cout + (int64_t)t * Cout + co]);
    const v4f bb = *reinterpret_cast<const v4f*>(&b[co]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float s = v[j] + bb[j];
        v[j] = gelu ? gelu_erf(s) : s;
    }
    *reinterpret_cast<v4f*>(&y[pix * Cout + co]) = v;
}

// ggml_im2col for a 3x3 / stride 1 / pad 1 convolution on token-major input:
// cols[p][(ic*3 + kh)*3 + kw] = x[(oy + kh - 1)*W + ox + kw - 1][ic], zero
// outside the image; F32, or F16 rounded to nearest even (im2col in the
// kernel's type).
template <bool F16>
__global__ __launch_bounds__(256) void im2col3x3_kernel(const float* __restrict__ x, int H, int W, int C,
                                                        void* __restrict__ cols) {
    const int64_t K = 9LL * C;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)H * W * K) return;
    const int64_t p = i / K;
    const int k = (int)(i - p * K);
    const int ic = k / 9, tap = k - ic * 9;
    const int oy = (int)(p / W) + tap / 3 - 1, ox = (int)(p % W) + tap % 3 - 1;
    const float v = oy >= 0 && oy < H && ox >= 0 && ox < W ? x[((int64_t)oy * W + ox) * C + ic] : 0.0f;
    if (F16) static_cast<uint16_t*>(cols)[i] = f2h(v);
    else static_cast<float*>(cols)[i] = v;
}

// F32 3x3 kernel [Cout][Cin][3][3] (ggml [3, 3, Cin, Cout]) -> rows [Cout][tap][Cin],
// tap = kh*3 + kw: the K order of the implicit-GEMM convolution
__global__ __launch_bounds__(256) void conv3x3_pack_kernel(const float* __restrict__ w, int Cin, int Cout,
                                                           float* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= 9LL * Cin * Cout) return;
    const int ci = (int)(i % Cin);
    const int64_t r = i / Cin;
    const int tap = (int)(r % 9), co = (int)(r / 9);
    out[i] = w[((int64_t)co * Cin + ci) * 9 + tap];
}

// y[r][c] += b[c], four channels per thread (C % 4 == 0)
__global__ __launch_bounds__(256) void bias_rows_kernel(float* __restrict__ y, const float* __restrict__ b, int64_t rows,
                                                        int C) {
    const int c4 = C / 4;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * c4) return;
    const int c = (int)(i % c4) * 4;
    v4f v = *reinterpret_cast<const v4f*>(&y[i * 4]);
    const v4f bb = *reinterpret_cast<const v4f*>(&b[c]);
    *reinterpret_cast<v4f*>(&y[i * 4]) = v + bb;
}

// ggml_pool_2d MAX, 2x2 window, stride 2, no padding: four channels per thread
__global__ __launch_bounds__(256) void maxpool2_kernel(const float* __restrict__ x, int H, int W, int C,
                                                       float* __restrict__ y) {
    const int c4 = C / 4, H2 = H / 2, W2 = W / 2;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)H2 * W2 * c4) return;
    const int c = (int)(i % c4) * 4;
    const int64_t q = i / c4;
    const int py = (int)(q / W2), px = (int)(q % W2);
    const float* s = x + ((int64_t)(2 * py) * W + 2 * px) * C + c;
    const v4f a = *reinterpret_cast<const v4f*>(s), b = *reinterpret_cast<const v4f*>(s + C);
    const v4f d = *reinterpret_cast<const v4f*>(s + (int64_t)W * C), e = *reinterpret_cast<const v4f*>(s + (int64_t)W * C + C);
    v4f m;
#pragma unroll
    for (int j = 0; j < 4; ++j) m[j] = fmaxf(fmaxf(a[j], b[j]), fmaxf(d[j], e[j]));
    *reinterpret_cast<v4f*>(&y[q * C + c]) = m;
}

hipError_t launch_deconv_pack(const void* w, int wtype, int Cin, int Cout, uint16_t* out, hipStream_t st) {
    const int64_t n = 4LL * Cout * Cin;
    if (n > 0) deconv_pack_kernel<<<nblk(n), 256, 0, st>>>(w, wtype, Cin, Cout, out);
    return hipGetLastError();
}

hipError_t launch_deconv_scatter(const float* D, const float* b, int H, int W, int Cout, bool gelu, float* y,
                                 hipStream_t st) {
    if (Cout % 4 != 0) return hipErrorInvalidValue;
    const int64_t n = 4LL * H * W * (Cout / 4);
    if (n > 0) deconv_scatter_kernel<<<nblk(n), 256, 0, st>>>(D, b, H, W, Cout, gelu ? 1 : 0, y);
    return hipGetLastError();
}

hipError_t launch_im2col3x3(const float* x, int H, int W, int C, bool f16, void* cols, hipStream_t st) {
    const int64_t n = (int64_t)H * W * 9 * C;
    if (n <= 0) return hipSuccess;
    if (f16) im2col3x3_kernel<true><<<nblk(n), 256, 0, st>>>(x, H, W, C, cols);
    else im2col3x3_kernel<false><<<nblk(n), 256, 0, st>>>(x, H, W, C, cols);
    return hipGetLastError();
}

hipError_t launch_conv3x3_pack(const float* w, int Cin, int Cout, float* out, hipStream_t st) {
    const int64_t n = 9LL * Cin * Cout;
    if (n > 0) conv3x3_pack_kernel<<<nblk(n), 256, 0, st>>>(w, Cin, Cout, out);
    return hipGetLastError();
}

hipError_t launch_bias_rows(float* y, const float* b, int64_t rows, int C, hipStream_t st) {
    if (C % 4 != 0) return hipErrorInvalidValue;
    const int64_t n = rows * (C / 4);
    if (n > 0) bias_rows_kernel<<<nblk(n), 256, 0, st>>>(y, b, rows, C);
    return hipGetLastError();
}

hipError_t launch_maxpool2(const float* x, int H, int W, int C, float* y, hipStream_t st) {
    if (C % 4 != 0) return hipErrorInvalidValue;
    const int64_t n = (int64_t)(H / 2) * (W / 2) * (C / 4);
    if (n > 0) maxpool2_kernel<<<nblk(n), 256, 0, st>>>(x, H, W, C, y);
    return hipGetLastError();
}

}  // namespace mi355
