// Host-side launchers of the gfx950 kernels (one .hip file each).  The C-ABI
// layer (capi.cpp) validates ggml semantics and calls these; each returns
// the hipError_t of its launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mi355 {

// enum ggml_type ids used on this path.
enum : int { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q8_0 = 8, T_Q8_1 = 9 };

// Strided view of an F32/F16 source tensor with rows over ne[1..3].
struct SrcView {
    const char* data;
    int type;  // 0 = F32, 1 = F16
    int64_t ne[4];
    int64_t nb[4];
};

// Quantized-activation layout consumed by the MMQ kernel: for z in
// [0, Z), rows m in [0, M): qs[(z*M + m)*K + k] int8, scale
// d[(z*nb + b)*M + m] fp32 (the fp16 d widened), and for Q8_1 the block sum
// term s[(z*nb + b)*M + m] fp32 (the fp16 s widened).
struct ActQ8 {
    int8_t* qs;
    float* d;
    float* s;
    int64_t M, K, Z;
};

// ggml from_float into contiguous ggml rows: type 8 (Q8_0), 9 (Q8_1), 1 (F16).
hipError_t launch_quantize_ggml(const SrcView& src, int type, bool ref_variant, void* dst, hipStream_t st);
// from_float into the MMQ layout (q8_0 semantics; with_sum adds the Q8_1 s).
hipError_t launch_quantize_mmq(const SrcView& src, bool with_sum, const ActQ8& out, hipStream_t st);
// F32/F16 strided rows -> contiguous F16 rows [rows][ne0] (round to nearest even).
hipError_t launch_convert_f16(const SrcView& src, uint16_t* dst, hipStream_t st);

struct MatW {  // src0 (weights), ggml layout
    const uint8_t* data;
    int type;
    int64_t nb1, nb2, nb3;  // bytes
    int64_t ne2, ne3;
};
struct MatD {  // dst F32
    float* data;
    int64_t nb1, nb2, nb3;  // bytes
};

// dst = W^T . act for quantized W (Q8_0 / Q4_0 / Q4_1); ne12/ne13 batch dims.
// When dots != nullptr the kernel writes the per-block int32 dots instead.
hipError_t launch_mmq(const MatW& w, const ActQ8& a, const MatD& d, int64_t N, int64_t ne12, int64_t ne13,
                      int32_t* dots, hipStream_t st);

// dst = W^T . A for F16 W and F16 activations A (rows of K halves with
// element strides a_nb1/a_nb2/a_nb3, in halves).
hipError_t launch_gemm_f16(const MatW& w, const uint16_t* a, int64_t a_s1, int64_t a_s2, int64_t a_s3,
                           const MatD& d, int64_t M, int64_t N, int64_t K, int64_t ne12, int64_t ne13, hipStream_t st);

// Row softmax of scale*x (F32, strided rows) into dst (F32, strided rows).
hipError_t launch_soft_max(const SrcView& src, float scale, char* dst, const int64_t dnb[4], hipStream_t st);

}  // namespace mi355
