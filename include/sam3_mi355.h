/*
 * sam3_mi355.h -- C-ABI of the MI355X (gfx950) backend for sam3.cpp's
 * quantized-matmul hot path.
 *
 * sam3.cpp builds ggml graphs and hands them to a backend
 * (sam3_graph_compute -> ggml_backend_graph_compute, sam3.cpp:1019-1030).
 * The nodes on the image-encoder hot path are MUL_MAT with F16/Q8_0/Q4_0/Q4_1
 * weights against F32 activations (sam3.cpp:3742,3783,3796,3799 for the SAM3
 * ViT; 4321,4349,4406,4451,4454 for SAM2 Hiera), FLASH_ATTN_EXT
 * (sam3.cpp:3778, 4399) and, for the explicit attention form, MUL_MAT(K,Q) /
 * SOFT_MAX / MUL_MAT(V^T,KQ) (sam3.cpp:8584-8589).  This header exposes one
 * entry point per such node, taking the ggml tensor layout fields (type, ne,
 * nb, data) so a ggml backend's graph_compute can forward node->src[i] and
 * the node itself unchanged.
 *
 * Conventions (ggml's): ne[0] is the contiguous dimension, nb[] are byte
 * strides, quantized rows are ne[0]/32 consecutive blocks.  All data pointers
 * are device pointers owned by the caller.  Calls enqueue work on the
 * context's HIP stream and return without waiting, like a backend's async
 * graph compute; mi355_synchronize() waits.  Nothing aborts: errors come back
 * as mi355_status values (the reference style, CLAUDE.md:62).
 */
#ifndef SAM3_MI355_H
#define SAM3_MI355_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* enum ggml_type ids used on this path (sam3.cpp:3246-3252). */
typedef enum {
    MI355_TYPE_F32 = 0,
    MI355_TYPE_F16 = 1,
    MI355_TYPE_Q4_0 = 2,
    MI355_TYPE_Q4_1 = 3,
    MI355_TYPE_Q8_0 = 8,
    MI355_TYPE_Q8_1 = 9,
} mi355_type;

/* enum ggml_status values, plus two refinements of FAILED. */
typedef enum {
    MI355_STATUS_INVALID_ARG = -4, /* shape/stride/pointer the op definition rejects */
    MI355_STATUS_UNSUPPORTED = -3, /* valid ggml op this backend does not implement */
    MI355_STATUS_ALLOC_FAILED = -2,
    MI355_STATUS_FAILED = -1,      /* a HIP runtime error */
    MI355_STATUS_SUCCESS = 0,
    MI355_STATUS_ABORTED = 1,
} mi355_status;

/* Activation-quantizer variant: ggml-cpu's from_float for Q8_0/Q8_1 exists as
 * the x86 SIMD routine (id = 127/amax, round half to even) and the scalar
 * _ref routine (id = 1/(amax/127), round half away).  mul_mat uses X86. */
typedef enum {
    MI355_ACT_X86 = 0,
    MI355_ACT_REF = 1,
} mi355_act_variant;

/* The layout fields of a ggml_tensor (ggml.h struct ggml_tensor: type, ne,
 * nb, data).  data is a device pointer. */
typedef struct mi355_tensor {
    int32_t type;
    int32_t pad_;
    int64_t ne[4];
    int64_t nb[4];
    void* data;
} mi355_tensor;

typedef struct mi355_context mi355_context;

/* Backend init: replaces ggml_backend_metal_init()/ggml_backend_cpu_init()
 * at sam3.cpp:3278-3292.  stream is a hipStream_t owned by the caller, or
 * NULL for the device's default (null) stream. */
mi355_status mi355_context_create(int device, void* stream, mi355_context** out);
void mi355_context_free(mi355_context* ctx);
/* Blocks until all work enqueued on the context's stream is done
 * (ggml_backend_synchronize). */
mi355_status mi355_synchronize(mi355_context* ctx);
/* ggml_status_to_string, used by sam3_graph_compute (sam3.cpp:1025-1027). */
const char* mi355_status_to_string(mi355_status status);
/* Text of the last error seen by this context ("" if none). */
const char* mi355_last_error(const mi355_context* ctx);
/* Reserve the context's scratch workspace (bytes); mul_mat grows it on
 * demand otherwise.  Replaces ggml-cpu's per-graph wdata buffer. */
mi355_status mi355_reserve_workspace(mi355_context* ctx, size_t bytes);
/* Workspace bytes mul_mat needs for these operands. */
size_t mi355_mul_mat_workspace_size(const mi355_tensor* src0, const mi355_tensor* src1);

/* ---- MUL_MAT (ggml_mul_mat, sam3.cpp:3742,3783,3796,3799) ----------------
 * dst[N, M, b2, b3] = src0[K, N, a2, a3]^T . src1[K, M, b2, b3], with
 * b2 % a2 == 0, b3 % a3 == 0 (src0 broadcast by the ratio).
 * src0: F16, Q8_0, Q4_0 or Q4_1, rows contiguous (nb[0] = type size).
 * src1: F32 (any strides) or, with F16 src0, F16.  dst: F32, nb[0] = 4.
 * Q8_0/Q4_0 quantize src1 to Q8_0 and Q4_1 to Q8_1 (x86 variant) exactly as
 * ggml-cpu's from_float, then combine exact int32 block dots in fp32.  F16
 * converts src1 to F16 (round to nearest even) and accumulates in fp32. */
int mi355_supports_mul_mat(const mi355_tensor* src0, const mi355_tensor* src1, const mi355_tensor* dst);
mi355_status mi355_mul_mat(mi355_context* ctx, const mi355_tensor* src0, const mi355_tensor* src1,
                           const mi355_tensor* dst);

/* ---- activation quantize (ggml-cpu type_traits[vec_dot_type].from_float,
 * the src1 conversion step of MUL_MAT; quantize_row_q8_0/q8_1, F16 convert).
 * Converts every row (ne[0] elements, rows over ne[1..3]) of the F32 tensor
 * src into dst as contiguous ggml rows of type (Q8_0, Q8_1 or F16): row r at
 * dst + r*row_size.  variant selects the from_float flavour. */
mi355_status mi355_quantize_rows(mi355_context* ctx, int type, int variant, const mi355_tensor* src, void* dst);

/* ---- Block-dot inspection (no ggml counterpart; test hook) ---------------
 * isums[b2][b3..][m][n][blk] = exact int32 block dots of the quantized
 * operands that mi355_mul_mat would combine, computed by the same MFMA
 * kernel.  src0 Q8_0/Q4_0/Q4_1; isums is a device buffer of
 * M*N*(K/32)*b2*b3 int32. */
mi355_status mi355_mul_mat_block_dots(mi355_context* ctx, const mi355_tensor* src0, const mi355_tensor* src1,
                                      int32_t* isums);

/* ---- SOFT_MAX (ggml_soft_max_ext(a, NULL, scale, 0.0f), sam3.cpp:8586) ----
 * Row-wise softmax of scale*src over ne[0]; F32 in/out, any row strides. */
mi355_status mi355_soft_max_ext(mi355_context* ctx, const mi355_tensor* src, const mi355_tensor* mask,
                                float scale, float max_bias, const mi355_tensor* dst);

/* ---- FLASH_ATTN_EXT (ggml_flash_attn_ext(q,k,v,NULL,scale,0,0),
 * sam3.cpp:3778 ViT, 4399 Hiera) --------------------------------------------
 * q [D, n_q, n_head, B], k [D, n_kv, n_head_kv, B], v [Dv, n_kv, n_head_kv, B]
 * (F32 or F16, any strides: the ViT passes V as a permuted view,
 * sam3.cpp:3767); dst [Dv, n_head, n_q, B] F32 contiguous.  D = Dv in
 * {64, 96, 128}.  mask must be NULL, max_bias and logit_softcap 0. */
mi355_status mi355_flash_attn_ext(mi355_context* ctx, const mi355_tensor* q, const mi355_tensor* k,
                                  const mi355_tensor* v, const mi355_tensor* mask, float scale, float max_bias,
                                  float logit_softcap, const mi355_tensor* dst);

/* ---- Kernel timing --------------------------------------------------------
 * The device-side counterpart of the reference's timing around graph compute
 * (std::chrono, sam3.cpp:6122-6135) and of its per-op micro-bench
 * (tests/test_metal_profile.cpp:22-69).  While enabled, every kernel launch
 * of the context is bracketed by HIP events on its stream;
 * mi355_profile_collect waits for them and folds the elapsed times into
 * per-kernel totals, returning the number of distinct kernels (or <0). */
mi355_status mi355_profile_enable(mi355_context* ctx, int enable);
int mi355_profile_collect(mi355_context* ctx);
mi355_status mi355_profile_get(mi355_context* ctx, int index, const char** name, int* launches, double* total_ms);
void mi355_profile_reset(mi355_context* ctx);

#ifdef __cplusplus
}
#endif
#endif /* SAM3_MI355_H */
