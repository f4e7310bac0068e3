/*
 * ggml_oracle.h -- CPU restatement of ggml's CPU arithmetic for the quantized
 * mul_mat / activation-quantize / attention path of sam3.cpp.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product path (libsam3mi355.so) never links, calls or falls back to it.
 *
 * The reference (Sanzentyo/sam3.cpp) calls into ggml for all of this
 * arithmetic (sam3.cpp:1019-1030 graph compute; ggml_mul_mat at
 * sam3.cpp:3742,3783,3796,3799; ggml_flash_attn_ext at sam3.cpp:3778).  ggml
 * is an un-vendored submodule (.gitmodules:1-3, PABannier/ggml, commit not
 * recorded) and is absent, so this is a restatement of ggml's published CPU
 * algorithm:
 *   - block formats  block_q8_0 / q8_1 / q4_0 / q4_1 (ggml-common.h)
 *   - weight quantizers quantize_row_*_ref (ggml-quants.c), as called by
 *     ggml_quantize_chunk from examples/quantize.cpp:244-245
 *   - activation quantizers: the x86 AVX2 quantize_row_q8_0/q8_1
 *     (id = 127/amax, round-half-even) and the scalar _ref variant
 *     (id = 1/d, roundf half-away)
 *   - vec_dot for Q8_0xQ8_0, Q4_0xQ8_0, Q4_1xQ8_1, F16xF16 in the x86 AVX2 /
 *     llamafile tinyBLAS summation order, and a plain sequential order
 *   - ggml_compute_forward_mul_mat: src1 -> vec_dot_type, then vec_dot per
 *     (row, col) with ne2/ne3 broadcast
 *   - ggml_compute_forward_soft_max (ext, no mask) and the CPU
 *     flash_attn_ext online-softmax loop (f32 V and f16-accumulated V)
 *   - the SAM3 ViT block glue (ggml_norm, gelu_erf, RoPE of
 *     sam3.cpp:3671-3710, axial cis of sam3.cpp:3559-3590, win_part/unpart)
 *
 * Every function here is pinned by at least one check in tests/ that a
 * plausible transcription mistake would fail (known-answer blocks, numpy
 * float16, brute force in long double, invariants).  See the per-function
 * comments in ggml_oracle.c for the anchor of each.
 */
#ifndef SAM3_GGML_ORACLE_H
#define SAM3_GGML_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml_type ids (sam3.cpp:3246-3252 maps ftype {0,1,2,3,8} to these). */
enum {
    ORC_TYPE_F32  = 0,
    ORC_TYPE_F16  = 1,
    ORC_TYPE_Q4_0 = 2,
    ORC_TYPE_Q4_1 = 3,
    ORC_TYPE_Q8_0 = 8,
    ORC_TYPE_Q8_1 = 9,
};

/* Activation quantizer variant. */
enum {
    ORC_ACT_X86 = 0, /* AVX2 quantize_row_q8_0/q8_1: id = 127/amax, rint */
    ORC_ACT_REF = 1, /* quantize_row_q8_0_ref: id = 1/(amax/127), roundf */
};

/* Float-combine order of the dot products. */
enum {
    ORC_ORDER_X86 = 0, /* 8-lane fma accumulators + hsum_float_8 (AVX2) */
    ORC_ORDER_SEQ = 1, /* ggml generic C: sumf += isum*(dx*dy) per block */
};

/* ggml-shaped tensor view: ne[0] is the contiguous dimension, nb[] in bytes. */
typedef struct {
    int32_t type;
    int32_t pad_;
    int64_t ne[4];
    int64_t nb[4];
    void*   data;
} orc_tensor;

#define ORC_QK 32

/* fp16 <-> fp32, IEEE binary16 round-to-nearest-even. */
uint16_t orc_fp32_to_fp16(float f);
float    orc_fp16_to_fp32(uint16_t h);
void     orc_fp32_to_fp16_row(const float* x, uint16_t* y, int64_t n);
void     orc_fp16_to_fp32_row(const uint16_t* x, float* y, int64_t n);

/* Deterministic inputs: SplitMix64(seed, stream) counter stream. */
uint64_t orc_splitmix64(uint64_t* state);
void orc_fill_normal(float* out, int64_t n, uint64_t seed, uint64_t stream, float mean, float stddev);
void orc_fill_uniform(float* out, int64_t n, uint64_t seed, uint64_t stream, float lo, float hi);

/* Type traits. */
int     orc_blck_size(int type);
int64_t orc_type_size(int type);
int64_t orc_row_size(int type, int64_t ne0);
int     orc_vec_dot_type(int type);

/* Quantizers.  k must be a multiple of 32 for the block types. */
void orc_quantize_row_q8_0_ref(const float* x, void* y, int64_t k);
void orc_quantize_row_q8_0_x86(const float* x, void* y, int64_t k);
void orc_quantize_row_q8_1_ref(const float* x, void* y, int64_t k);
void orc_quantize_row_q8_1_x86(const float* x, void* y, int64_t k);
void orc_quantize_row_q4_0_ref(const float* x, void* y, int64_t k);
void orc_quantize_row_q4_1_ref(const float* x, void* y, int64_t k);
/* ggml_quantize_chunk(type, src, dst, start, nrows, n_per_row, imatrix=NULL):
 * reference weight quantizers; returns bytes written. */
int64_t orc_quantize_chunk(int type, const float* src, void* dst, int64_t start,
                           int64_t nrows, int64_t n_per_row);
/* from_float of the activation side (vec_dot_type rows). */
int orc_from_float(int type, int act_variant, const float* x, void* y, int64_t k);
/* to_float. */
int orc_dequantize_row(int type, const void* x, float* y, int64_t k);

/* Dot products.  x is a src0 row (type), y a vec_dot_type row. */
float  orc_vec_dot(int type, int64_t n, const void* x, const void* y, int order);
/* Exact integer block dots: out[b] = sum_j qx[b][j]*qy[b][j] (Q4_0: qx-8;
 * Q4_1: raw nibble).  Only for the block types. */
int    orc_block_isums(int type, int64_t n, const void* x, const void* y, int32_t* out);
/* The same dot in long double over the quantized values (no summation error). */
double orc_vec_dot_exact(int type, int64_t n, const void* x, const void* y);
/* Sum of |elementwise terms|: sum_b |d_x*d_y| * sum_j |qx_j*qy_j|
 * (+|m_x*s_y| for Q4_1).  It bounds the rounding error of any summation
 * order, so relative-error tolerances are stated against it. */
double orc_vec_dot_absterm(int type, int64_t n, const void* x, const void* y);

/* ggml_compute_forward_mul_mat: dst = src0^T . src1 per batch, broadcast over
 * ne2/ne3.  src1 is F32 (or F16 with F16 src0); dst F32.  Returns 0 on
 * success, <0 when the combination is unsupported. */
int orc_mul_mat(const orc_tensor* src0, const orc_tensor* src1, const orc_tensor* dst,
                int act_variant, int order, int n_threads);
/* Same shapes, long-double over dequantized src0 and quantized src1 rows.
 * Writes dst (rounded to float) and optionally the absterm per element
 * (as orc_vec_dot_absterm). */
int orc_mul_mat_exact(const orc_tensor* src0, const orc_tensor* src1, const orc_tensor* dst,
                      float* absterm, int act_variant, int n_threads);

/* ggml_soft_max_ext(a, mask=NULL, scale, max_bias=0) over rows of ne0. */
int orc_soft_max_ext(const orc_tensor* src, const orc_tensor* dst, float scale, int n_threads);

/* ggml_flash_attn_ext(q, k, v, mask=NULL, scale, max_bias=0, softcap).
 * q [D, n_q, n_head, batch] F32/F16; k [D, n_kv, n_head_kv, batch] F32/F16;
 * v [Dv, n_kv, n_head_kv, batch] F32/F16 (any strides); dst [Dv, n_head,
 * n_q, batch] F32 contiguous.  V=F16 accumulates in f16 like ggml-cpu. */
int orc_flash_attn_ext(const orc_tensor* q, const orc_tensor* k, const orc_tensor* v,
                       const orc_tensor* dst, float scale, float softcap, int n_threads);
/* Textbook softmax(scale*Q K^T) V in long double (same I/O conventions). */
int orc_attn_exact(const orc_tensor* q, const orc_tensor* k, const orc_tensor* v,
                   const orc_tensor* dst, float scale, int n_threads);

/* ViT glue (sam3.cpp:1041-1051, 3559-3590, 3671-3710, 3714-3805). */
void orc_norm_rows(const float* x, float* y, int64_t nrows, int64_t ne0, float eps);
void orc_gelu_erf(const float* x, float* y, int64_t n);
void orc_gelu_tanh(const float* x, float* y, int64_t n); /* ggml_gelu, fp16-table semantics */
void orc_hiera_win_part(const float* x, float* y, int64_t C, int64_t W, int64_t H, int ws);
void orc_hiera_win_unpart(const float* x, float* y, int64_t C, int64_t W, int64_t H, int ws);
void orc_maxpool2(const float* x, float* y, int64_t C, int64_t W, int64_t H, int64_t B);
/* sam2_compute_pos_embed (sam3.cpp:4076-4157): bicubic(bkg) + tiled window
 * table; bkg [E][bh][bw], win [E][ws][ws] CHW; out [H*W][E]. */
void orc_sam2_pos_embed(const float* bkg, int E, int bh, int bw, const float* win, int ws, int H, int W, float* out);
void orc_compute_axial_cis(float* out, int dim, int end_x, int end_y, float theta, float scale_pos);
/* x [hd, N, nh] rows; freqs [hd/2 pairs (cos,sin)] per token, [N][hd]. */
void orc_apply_rope(float* x, const float* freqs, int64_t hd, int64_t n_tok, int64_t n_rows3);
void orc_win_part(const float* src, float* dst, int64_t C, int64_t W, int64_t H, int w);
void orc_win_unpart(const float* src, float* dst, int64_t C, int64_t W, int64_t H, int w);

/* Host ISA path used by the fast dot kernels: 0 scalar, 1 AVX2, 2 AVX2 with AVX512-VNNI
 * for the quantized dots (bit-identical to 1 and to the scalar x86 order). */
int orc_isa_path(void);
void orc_set_isa(int path);

#ifdef __cplusplus
}
#endif
#endif
