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

/* Version of this interface: 2 added the layout field of mi355_tensor (the
 * former padding word, which callers must now set to 0, e.g. by
 * zero-initializing the struct) and prepared weights.  A binding compiled
 * against one version checks mi355_abi_version() at load. */
#define MI355_ABI_VERSION 2
int mi355_abi_version(void);

/* The layout fields of a ggml_tensor (ggml.h struct ggml_tensor: type, ne,
 * nb, data).  data is a device pointer.  layout is MI355_LAYOUT_GGML (0, the
 * bytes ggml defines for type/ne/nb) except for a weight prepared by
 * mi355_weight_prepare (MI355_LAYOUT_INT8); any other value is rejected
 * (MI355_STATUS_INVALID_ARG) by every entry point. */
typedef enum {
    MI355_LAYOUT_GGML = 0,
    MI355_LAYOUT_INT8 = 1,
} mi355_layout;
typedef struct mi355_tensor {
    int32_t type;
    int32_t layout;
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
/* Workspace bytes mul_mat needs for these operands: the most over the
 * MUL_MAT routes (mi355_context_set_mmq_kernel). */
size_t mi355_mul_mat_workspace_size(const mi355_tensor* src0, const mi355_tensor* src1);

/* ---- Device buffers (the ggml-backend buffer calls around a graph) ---------
 * A buffer is one device allocation on the context's device, owned by the
 * caller until mi355_buffer_free.  It stands in for
 * ggml_backend_alloc_ctx_tensors (sam3.cpp:3320, the model's weights) and for
 * the graph allocator's buffer (ggml_gallocr_alloc_graph, sam3.cpp:6101-6115);
 * mi355_buffer_place puts a tensor at an offset in it (ggml_tallocr_alloc),
 * offsets being multiples of mi355_buffer_alignment().  The byte layouts are
 * ggml's, so tensor bytes read from a .ggml file or written by ggml-cpu are
 * used as they are. */
typedef struct mi355_buffer mi355_buffer;
size_t mi355_buffer_alignment(void);
mi355_status mi355_buffer_alloc(mi355_context* ctx, size_t size, mi355_buffer** out);
/* ggml_backend_buffer_free: waits for the device's work before freeing. */
void mi355_buffer_free(mi355_buffer* buf);
void* mi355_buffer_base(const mi355_buffer* buf);
size_t mi355_buffer_size(const mi355_buffer* buf);
/* Sets t->data = base + offset after checking that ggml_nbytes(t) bytes fit. */
mi355_status mi355_buffer_place(const mi355_buffer* buf, size_t offset, mi355_tensor* t);
/* ggml_nbytes of t's layout (0 for an empty tensor or an unknown type); for
 * a prepared weight (MI355_LAYOUT_INT8) the bytes of its prepared form. */
size_t mi355_tensor_nbytes(const mi355_tensor* t);
/* ggml_backend_buffer_clear. */
mi355_status mi355_buffer_clear(mi355_context* ctx, mi355_buffer* buf, uint8_t value);
/* ggml_backend_tensor_set / _get / _memset (sam3.cpp:3156-3179, 6117): bytes
 * [offset, offset + size) of the tensor's data, bounds-checked against
 * ggml_nbytes(t); ordered after the work already on the context's stream, and
 * returning when the host side is done (set: data may be reused; get: data
 * has arrived). */
mi355_status mi355_tensor_set(mi355_context* ctx, const mi355_tensor* t, const void* data, size_t offset, size_t size);
mi355_status mi355_tensor_get(mi355_context* ctx, const mi355_tensor* t, void* data, size_t offset, size_t size);
mi355_status mi355_tensor_memset(mi355_context* ctx, const mi355_tensor* t, uint8_t value, size_t offset, size_t size);

/* ---- MUL_MAT (ggml_mul_mat, sam3.cpp:3742,3783,3796,3799) ----------------
 * dst[N, M, b2, b3] = src0[K, N, a2, a3]^T . src1[K, M, b2, b3], with
 * b2 % a2 == 0, b3 % a3 == 0 (src0 broadcast by the ratio).
 * src0: F16, Q8_0, Q4_0 or Q4_1, rows contiguous (nb[0] = type size).
 * src1: F32 (any strides) or, with F16 src0, F16.  dst: F32, nb[0] = 4.
 * Q8_0/Q4_0 quantize src1 to Q8_0 and Q4_1 to Q8_1 (x86 variant) exactly as
 * ggml-cpu's from_float, then combine exact int32 block dots in fp32.  F16
 * converts src1 to F16 (round to nearest even) and accumulates in fp32. */
/* The mi355_supports_* queries are ggml_backend_supports_op for each node
 * kind: 1 when the entry point accepts these operands (no GPU work, no
 * context), 0 otherwise.  sam3.cpp runs each graph on a single backend
 * (sam3.cpp:3278-3292), so a graph builder checks every node before
 * choosing this one. */
int mi355_supports_mul_mat(const mi355_tensor* src0, const mi355_tensor* src1, const mi355_tensor* dst);
mi355_status mi355_mul_mat(mi355_context* ctx, const mi355_tensor* src0, const mi355_tensor* src1,
                           const mi355_tensor* dst);

/* ---- Prepared weights (the counterpart of ggml's "extra" buffer types, such
 * as ggml-cpu's, which repack Q4_0 weights into an interleaved layout when
 * ggml_backend_tensor_set uploads them; sam3.cpp uploads each weight once,
 * sam3.cpp:3156-3179).  A 2-D Q8_0 / Q4_0 / Q4_1 weight is repacked once into
 * the int8 MUL_MAT layout (quants as int8 rows, block scales in separate
 * arrays), so MUL_MATs with it skip the per-call repack.
 * mi355_weight_prepared_nbytes: bytes of the prepared form of w (0: w is not
 *   a 2-D Q8_0 / Q4_0 / Q4_1 weight with K % 32 == 0).
 * mi355_weight_prepare: repacks w (ggml layout, device data) into dst
 *   (256-byte aligned, dst_size >= the prepared bytes, not overlapping w) on
 *   the context's stream, and describes the result in *out: w's type and ne,
 *   layout MI355_LAYOUT_INT8, nb of a contiguous ggml tensor, data = dst.
 *   mi355_mul_mat and mi355_mul_mat_noalloc take *out as src0 and give the
 *   same bits as with w; the buffer and tensor calls copy it as bytes; every
 *   other op rejects it (MI355_STATUS_INVALID_ARG). */
size_t mi355_weight_prepared_nbytes(const mi355_tensor* w);
mi355_status mi355_weight_prepare(mi355_context* ctx, const mi355_tensor* w, void* dst, size_t dst_size,
                                  mi355_tensor* out);

/* ---- MUL_MAT without allocation (no counterpart in the reference; for
 * callers that cannot allocate device memory: code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc) ----------------------
 * The same operation, checks and kernels as mi355_mul_mat, with the same
 * results.  Its scratch (the converted src1, split-K partial sums, the
 * 4-byte-pitch weight copy) lives in a fixed device array of
 * MI355_NOALLOC_SCRATCH_BYTES per GPU, held from library load until the
 * process ends, instead of the context's workspace; the call allocates and
 * frees nothing and records no timing events.  Operands whose plan on the
 * context's current route (mi355_context_set_mmq_kernel) needs more scratch
 * than that are rejected with MI355_STATUS_UNSUPPORTED; the most any route
 * needs, mi355_mul_mat_workspace_size, bounds it from above.  Every call on
 * one GPU uses that GPU's one array: calls through one context serialize on
 * its stream, and a call through another context first makes its stream
 * wait on an event the device's previous call recorded (each context creates
 * its event when it is created).  Under stream capture no event is waited on
 * or recorded: the caller orders the launches of captured graphs.  Host
 * threads sharing one context must serialize their calls. */
#define MI355_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
mi355_status mi355_mul_mat_noalloc(mi355_context* ctx, const mi355_tensor* src0, const mi355_tensor* src1,
                                   const mi355_tensor* dst);

/* ---- activation quantize (ggml-cpu type_traits[vec_dot_type].from_float,
 * the src1 conversion step of MUL_MAT; quantize_row_q8_0/q8_1, F16 convert).
 * Converts every row (ne[0] elements, rows over ne[1..3]) of the F32 tensor
 * src into dst as contiguous ggml rows of type (Q8_0, Q8_1 or F16): row r at
 * dst + r*row_size.  variant selects the from_float flavour. */
mi355_status mi355_quantize_rows(mi355_context* ctx, int type, int variant, const mi355_tensor* src, void* dst);

/* ---- weight quantize (ggml_quantize_chunk(type, src, dst, 0, nrows,
 * n_per_row, NULL), examples/quantize.cpp:244-245: the _ref row quantizers
 * quantize_row_q8_0_ref / q4_0_ref / q4_1_ref).  Every row of the F32 or F16
 * tensor src (F16 widened to F32 exactly first, as sam3_quantize_model does
 * at quantize.cpp:227-237) -> dst as contiguous ggml rows of type (Q8_0, Q4_0
 * or Q4_1), row r at dst + r*row_size; dst 2-byte aligned. */
mi355_status mi355_quantize_weights(mi355_context* ctx, int type, const mi355_tensor* src, void* dst);

/* ---- Block-dot inspection (no ggml counterpart; test hook) ---------------
 * isums[b2][b3..][m][n][blk] = exact int32 block dots of the quantized
 * operands that mi355_mul_mat would combine, computed by the same MFMA
 * kernel.  src0 Q8_0/Q4_0/Q4_1; isums is a device buffer of
 * M*N*(K/32)*b2*b3 int32. */
mi355_status mi355_mul_mat_block_dots(mi355_context* ctx, const mi355_tensor* src0, const mi355_tensor* src1,
                                      int32_t* isums);

/* ---- SOFT_MAX (ggml_soft_max_ext(a, NULL, scale, 0.0f), sam3.cpp:8586) ----
 * Row-wise softmax of scale*src over ne[0]; F32 in/out, any row strides. */
int mi355_supports_soft_max_ext(const mi355_tensor* src, const mi355_tensor* mask, float max_bias,
                                const mi355_tensor* dst);
mi355_status mi355_soft_max_ext(mi355_context* ctx, const mi355_tensor* src, const mi355_tensor* mask,
                                float scale, float max_bias, const mi355_tensor* dst);

/* ---- FLASH_ATTN_EXT (ggml_flash_attn_ext(q,k,v,NULL,scale,0,0),
 * sam3.cpp:3778 ViT, 4399 Hiera) --------------------------------------------
 * q [D, n_q, n_head, B], k [D, n_kv, n_head_kv, B], v [Dv, n_kv, n_head_kv, B]
 * (F32 or F16, any strides: the ViT passes V as a permuted view,
 * sam3.cpp:3767); dst [Dv, n_head, n_q, B] F32 contiguous.  D = Dv in
 * {64, 96, 128}.  mask must be NULL, max_bias and logit_softcap 0. */
int mi355_supports_flash_attn_ext(const mi355_tensor* q, const mi355_tensor* k, const mi355_tensor* v,
                                  const mi355_tensor* mask, float max_bias, float logit_softcap,
                                  const mi355_tensor* dst);
mi355_status mi355_flash_attn_ext(mi355_context* ctx, const mi355_tensor* q, const mi355_tensor* k,
                                  const mi355_tensor* v, const mi355_tensor* mask, float scale, float max_bias,
                                  float logit_softcap, const mi355_tensor* dst);

/* ---- SAM3 ViT image encoder ----------------------------------------------
 * The graph sam3_build_vit_graph builds (sam3.cpp:3836-3853) run on this
 * backend: the prefix (patch embedding, tiled pos_embed, ln_pre;
 * sam3.cpp:3810-3834) and sam3_vit_block_forward (sam3.cpp:3714-3805), with
 * the memory-bound ggml nodes around each MUL_MAT / FLASH_ATTN_EXT fused
 * into single passes that keep ggml's per-node fp32 rounding.
 * Activations x are device F32 [grid*grid][E] in image token order
 * (ggml [E, W, H, 1]).  All weight pointers are device pointers. */
typedef struct mi355_vit_hparams {
    int32_t embed_dim;   /* E (1024) */
    int32_t num_heads;   /* 16; head size E / num_heads in {64, 96, 128} */
    int32_t mlp_dim;     /* 4736 */
    int32_t window_size; /* 24 */
    int32_t grid;        /* tokens per image side: img_size / patch_size (72) */
    int32_t patch_size;  /* 14 */
    int32_t pos_grid;    /* side of pos_embed at pretrained resolution (24), tiled over the grid */
    float eps;           /* LayerNorm eps (1e-5) */
} mi355_vit_hparams;

typedef struct mi355_vit_block {
    /* linear weights [in, out] (ggml ne), F16 / Q8_0 / Q4_0 / Q4_1 (or F32) */
    mi355_tensor qkv_w, proj_w, fc1_w, fc2_w;
    const float* norm1_w;
    const float* norm1_b;
    const float* qkv_b;
    const float* proj_b;
    const float* norm2_w;
    const float* norm2_b;
    const float* fc1_b;
    const float* fc2_b;
    const float* freqs_cis; /* [N][head_dim/2][2] (cos, sin); N = window_size^2, or grid^2 if global; NULL: no RoPE */
    int32_t is_global;      /* 0: attention inside window_size^2 windows (ggml_win_part) */
} mi355_vit_block;

/* Device bytes the encoder keeps for its activations (allocated on first use). */
size_t mi355_vit_workspace_size(const mi355_vit_hparams* hp);
/* x = ln_pre(conv2d_p(image) + tile(pos_embed)): image device F32 [3][H][W]
 * with H = W = grid * patch_size; patch_w [P, P, 3, E] F32 or F16. */
mi355_status mi355_vit_prefix(mi355_context* ctx, const mi355_vit_hparams* hp, const float* image,
                              const mi355_tensor* patch_w, const float* pos_embed, const float* ln_pre_w,
                              const float* ln_pre_b, float* x);
/* x = sam3_vit_block_forward(x) in place. */
mi355_status mi355_vit_block_forward(mi355_context* ctx, const mi355_vit_hparams* hp, const mi355_vit_block* blk,
                                     float* x);
/* The whole encoder: prefix, then n_blocks blocks; x: [grid*grid][E] output. */
mi355_status mi355_vit_encode(mi355_context* ctx, const mi355_vit_hparams* hp, const float* image,
                              const mi355_tensor* patch_w, const float* pos_embed, const float* ln_pre_w,
                              const float* ln_pre_b, const mi355_vit_block* blocks, int n_blocks, float* x);

/* The fused node groups the encoder runs, for use by other graph builders
 * and for testing each against ggml's node sequence:
 * - layer_norm: y[row(r)] = ggml_add(ggml_mul(ggml_norm(x[r] (+ add[r']), eps), w), b)
 *   (sam3_layer_norm, sam3.cpp:1041-1051); add (optional) is added first,
 *   row r' = r, or (y%add_grid)*add_grid + x%add_grid when add_grid > 0
 *   (ggml_repeat of pos_embed, sam3.cpp:3820-3826); row(r) is r, or its
 *   ggml_win_part row when window > 0 (sam3.cpp:3734).  w, b may be NULL. */
mi355_status mi355_vit_layer_norm(mi355_context* ctx, const float* x, const float* add, int add_grid, const float* w,
                                  const float* b, float* y, int64_t rows, int E, int grid, int window, float eps);
/* qkv [M][3E] (+ bias) -> Q, K (RoPE applied, sam3_apply_rope) and V as
 * fp16 [M/N][NH][N][HD] (the FLASH_ATTN_EXT operand layout of
 * sam3.cpp:3742-3778); rope [N][HD/2][2] or NULL. */
mi355_status mi355_vit_qkv_rope(mi355_context* ctx, const float* qkv, const float* bias, const float* rope, void* q,
                                void* k, void* v, int64_t M, int N, int n_heads, int head_dim);
/* x[r] = x[r] + (p[row(r)] + b): proj bias, ggml_win_unpart (window > 0) and
 * the residual add (sam3.cpp:3783-3791). */
mi355_status mi355_vit_proj_residual(mi355_context* ctx, float* x, const float* p, const float* b, int64_t rows, int E,
                                     int grid, int window);
/* h = ggml_gelu_erf(h + b) over rows of n (sam3.cpp:3796-3797). */
mi355_status mi355_vit_bias_gelu(mi355_context* ctx, float* h, const float* b, int64_t rows, int n);
/* x = x + (f + b) over rows of n (sam3.cpp:3799-3802). */
mi355_status mi355_vit_bias_residual(mi355_context* ctx, float* x, const float* f, const float* b, int64_t rows, int n);

/* ---- SAM2 Hiera image encoder ---------------------------------------------
 * sam2_build_hiera_graph (sam3.cpp:4466-4535) on this backend: patch
 * embedding (conv 7x7, stride 4, pad 3, + bias) + pos_embed, then the blocks
 * of sam2_hiera_block_forward (sam3.cpp:4299-4461) with the per-block
 * metadata of sam2_precompute_hiera_metadata (sam3.cpp:1680-1746).
 * Activations are device F32 [S*S][C] in image token order (ggml [C, S, S]). */
typedef struct mi355_hiera_hparams {
    int32_t img_size;       /* 1024 */
    int32_t embed_dim;      /* 96 for Hiera-tiny */
    int32_t num_heads;      /* 1 */
    int32_t stages[4];      /* blocks per stage {1, 2, 7, 2} */
    int32_t q_pool;         /* stage transitions with Q pooling (3) */
    int32_t window_spec[4]; /* {8, 4, 14, 7} */
    int32_t global_idx[8];  /* blocks with global attention {5, 7, 9} */
    int32_t n_global;
    float eps;              /* LayerNorm eps (1e-6) */
} mi355_hiera_hparams;

typedef struct mi355_hiera_block {
    mi355_tensor qkv_w, proj_w, fc1_w, fc2_w;
    mi355_tensor dim_proj_w; /* data NULL for blocks that keep their width */
    const float* norm1_w;
    const float* norm1_b;
    const float* qkv_b;
    const float* proj_b;
    const float* norm2_w;
    const float* norm2_b;
    const float* fc1_b;
    const float* fc2_b;
    const float* dim_proj_b;
} mi355_hiera_block;

/* Per-block metadata as the reference derives it: width in/out, heads,
 * window size (0 = global) and Q pooling. */
typedef struct mi355_hiera_block_info {
    int32_t dim_in, dim_out, num_heads, window_size, q_stride, stage;
} mi355_hiera_block_info;
int mi355_hiera_n_blocks(const mi355_hiera_hparams* hp);
mi355_status mi355_hiera_block_info_get(const mi355_hiera_hparams* hp, int block_index, mi355_hiera_block_info* out);
/* Device bytes the encoder keeps for its activations (allocated on first use). */
size_t mi355_hiera_workspace_size(const mi355_hiera_hparams* hp);
/* One block: x [S*S][dim_in] -> x_out [S'*S'][dim_out], S' = S/2 with Q pooling.
 * x_out must not overlap x. */
mi355_status mi355_hiera_block_forward(mi355_context* ctx, const mi355_hiera_hparams* hp, int block_index,
                                       const mi355_hiera_block* blk, const float* x, int spatial, float* x_out);
/* x = conv2d(image, patch_w, stride 4, pad 3) + patch_b + pos_embed, the patch
 * embedding mi355_hiera_encode starts from (sam3.cpp:4473-4494: ggml_conv_2d =
 * im2col + F32 mul_mat, + bias, + pos_embed): image device F32 [3][img][img],
 * patch_w [7, 7, 3, E] F32 or F16, patch_b [E], pos_embed and x [S0*S0][E]
 * token-major (S0 = img/4). */
mi355_status mi355_hiera_prefix(mi355_context* ctx, const mi355_hiera_hparams* hp, const float* image,
                                const mi355_tensor* patch_w, const float* patch_b, const float* pos_embed, float* x);
/* The whole backbone: image device F32 [3][img][img]; patch_w [7, 7, 3, E]
 * F32 or F16, patch_b [E], pos_embed [S0*S0][E] (S0 = img/4).  stage_out[s]
 * (device [S_s*S_s][C_s], or NULL) receive the output of each stage's last
 * block, which writes it there directly; the next stage reads it from there, so
 * the maps must not overlap one another. */
mi355_status mi355_hiera_encode(mi355_context* ctx, const mi355_hiera_hparams* hp, const float* image,
                                const mi355_tensor* patch_w, const float* patch_b, const float* pos_embed,
                                const mi355_hiera_block* blocks, int n_blocks, float* const stage_out[4]);

/* sam2_compute_pos_embed (sam3.cpp:4076-4157) on the device: the pos_embed
 * that mi355_hiera_encode adds, out [H*W][E] token-major (ggml [E, W, H]) =
 * bicubic(bkg -> H x W; Keys a = -0.75, half-pixel centres, border-clamped
 * taps, as torch's bicubic with align_corners=False) + the window table tiled
 * modulo ws.  bkg [E][bkg_h][bkg_w] and win [E][ws][ws] are device F32 in the
 * raw byte order of "hiera.pos_embed" ([bkg_w, bkg_h, E, 1]) and
 * "hiera.pos_embed_window" ([ws, ws, E, 1]).  For SAM2.1 Hiera at 1024:
 * bkg 7x7, ws 8, H = W = 256. */
mi355_status mi355_hiera_pos_embed(mi355_context* ctx, const float* bkg, int E, int bkg_h, int bkg_w, const float* win,
                                   int ws, int H, int W, float* out);

/* ---- SAM3 SimpleFPN neck ----------------------------------------------------
 * sam3_build_neck_graph (sam3.cpp:3867-3925) on this backend.  Activations
 * are device F32 token-major [H*W][C] (ggml [C, W, H]): the ViT output the
 * neck reads (vit_out [E, W, H]) and the four maps it writes (the reference's
 * out[i] after its final cont(permute(.., 1, 2, 0, 3))) are exactly the
 * reference's layouts.  Kernels are the registered ggml tensors
 * (sam3.cpp:2566-2600): conv-transpose [2, 2, Cout, Cin], conv [1, 1, Cin,
 * Cout] and [3, 3, Cin, Cout], F32 or F16 (F32 under quantized ftypes: their
 * ne0 of 1, 2 or 3 is not a block multiple), contiguous; biases F32.
 * Numerics per op as ggml-cpu: conv-transpose with the kernel cast to F16 and
 * the input converted to F16; conv_2d with the activations in the kernel's
 * type; f32 accumulation; f32 bias adds; GELU-erf after scale 0's first
 * conv-transpose. */
typedef struct mi355_neck_scale {
    const mi355_tensor* deconv1_w; /* scales 0 and 1: [2, 2, C1, E] */
    const float* deconv1_b;
    const mi355_tensor* deconv2_w; /* scale 0: [2, 2, D, C1] */
    const float* deconv2_b;
    const mi355_tensor* conv1x1_w; /* [1, 1, Cin, D] */
    const float* conv1x1_b;
    const mi355_tensor* conv3x3_w; /* [3, 3, D, D] */
    const float* conv3x3_b;
} mi355_neck_scale;
/* Device bytes the neck keeps in the context for a G x G grid of E channels. */
size_t mi355_neck_workspace_size(int E, int G, const mi355_neck_scale scales[4]);
/* out[0] [(4G)^2][D], out[1] [(2G)^2][D], out[2] [G^2][D], out[3] [(G/2)^2][D]
 * from x [G^2][E]; G even.  Scale 0: conv-transpose + GELU, conv-transpose,
 * 1x1, 3x3; scale 1: conv-transpose, 1x1, 3x3; scale 2: 1x1, 3x3; scale 3:
 * 2x2 max-pool, 1x1, 3x3; every conv adds its bias. */
mi355_status mi355_sam3_neck(mi355_context* ctx, const float* x, int E, int G, const mi355_neck_scale scales[4],
                             float* const out[4]);
/* The neck's node groups on token-major activations, for other graph builders:
 * ggml_conv_transpose_2d_p0(w [2, 2, Cout, Cin], x, 2) + bias (+ ggml_gelu_erf
 * when gelu): x [H*W][Cin] -> y [(2H)*(2W)][Cout]; */
mi355_status mi355_neck_deconv(mi355_context* ctx, const mi355_tensor* w, const float* b, const float* x, int H, int W,
                               int gelu, float* y);
/* ggml_conv_2d_sk_p0 (w [1, 1, Cin, Cout]) or ggml_conv_2d_s1_ph (w [3, 3, Cin,
 * Cout]) + bias: x [H*W][Cin] -> y [H*W][Cout]; */
mi355_status mi355_neck_conv(mi355_context* ctx, const mi355_tensor* w, const float* b, const float* x, int H, int W,
                             float* y);
/* ggml_pool_2d(MAX, 2, 2, 2, 2, 0, 0): x [H*W][C] -> y [(H/2)*(W/2)][C]. */
mi355_status mi355_neck_maxpool(mi355_context* ctx, const float* x, int H, int W, int C, float* y);

/* ---- Model files (sam3.cpp's .ggml format) ----------------------------------
 * sam3_load_model / sam3_load_tensors (sam3.cpp:3095-3348): a header (magic
 * "sam3" 0x73616D33 version 3, or "sam2" 0x73616D32 version 1; ftype; tensor
 * count), the hyperparameters as int32 fields (sam3_load_hparams 1481-1524,
 * sam2_load_hparams 1568-1630; SAM2 files with the Hiera backbone only), then
 * per tensor: n_dims, name length, ggml type, ne[0..n_dims), name, zero
 * padding to a 32-byte file offset, and the raw ggml rows.  Opening indexes the
 * records; data is read when a tensor is loaded. */
typedef struct mi355_model_file mi355_model_file;
typedef struct mi355_model_tensor_info {
    const char* name;   /* valid while the file is open */
    int32_t type;       /* ggml type id: 0 F32, 1 F16, 2 Q4_0, 3 Q4_1, 8 Q8_0 */
    int32_t n_dims;
    int64_t ne[4];      /* ggml order, unused dims 1 */
    uint64_t offset;    /* file offset of the data (32-byte aligned) */
    uint64_t nbytes;    /* data bytes */
} mi355_model_tensor_info;
mi355_status mi355_model_file_open(const char* path, mi355_model_file** out);
void mi355_model_file_close(mi355_model_file* f);
/* Text of the last open/query error (the calls without a context). */
const char* mi355_model_file_last_error(void);
mi355_status mi355_model_file_header(const mi355_model_file* f, uint32_t* magic, int32_t* version, int32_t* ftype,
                                     int32_t* n_tensors);
/* The hyperparameter fields in file order; returns their count (or -1). */
int mi355_model_file_hparams(const mi355_model_file* f, const int32_t** values);
/* Index of the tensor called name, or -1. */
int mi355_model_file_find(const mi355_model_file* f, const char* name);
mi355_status mi355_model_file_tensor(const mi355_model_file* f, int index, mi355_model_tensor_info* out);
/* Device bytes of tensor index loaded as dst_type (0 when no conversion exists):
 * the file's own type, F32 (from F16 or by dequantizing Q8_0/Q4_0/Q4_1), or F16
 * (from F32) - the conversions sam3_load_tensors applies (sam3.cpp:3150-3185). */
size_t mi355_model_file_load_bytes(const mi355_model_file* f, int index, int32_t dst_type);
/* Tensor data -> device memory dst (dst_bytes >= mi355_model_file_load_bytes),
 * converted on the GPU when dst_type differs.  Synchronous. */
mi355_status mi355_model_file_load(mi355_context* ctx, const mi355_model_file* f, int index, int32_t dst_type,
                                   void* dst, size_t dst_bytes);

/* A SAM3 file's ViT backbone in device memory: the tensors sam3_register_tensors
 * declares for it (sam3.cpp:2530-2560: "vit.patch_embed.proj.weight",
 * "vit.pos_embed", "vit.ln_pre.*", "vit.blocks.N.*"), weights in the file's
 * weight type when their rows are whole blocks and F32 otherwise, as the
 * reference registers them; the hyperparameters of mi355_vit_encode derived as
 * sam3_load_hparams does.  Quantized linear weights (Q8_0 / Q4_0 / Q4_1) are
 * handed out prepared (mi355_weight_prepare).  The tables stay valid until
 * mi355_vit_weights_free. */
typedef struct mi355_vit_weights mi355_vit_weights;
mi355_status mi355_vit_weights_load(mi355_context* ctx, const mi355_model_file* f, mi355_vit_weights** out);
void mi355_vit_weights_free(mi355_vit_weights* w);
mi355_status mi355_vit_weights_get(const mi355_vit_weights* w, mi355_vit_hparams* hp, const mi355_vit_block** blocks,
                                   int* n_blocks, const mi355_tensor** patch_w, const float** pos_embed,
                                   const float** ln_pre_w, const float** ln_pre_b);

/* sam3_quantize_model (examples/quantize.cpp:20-331): copies the .ggml file
 * in_path to out_path with the header's ftype set to qtype (Q4_0, Q4_1 or
 * Q8_0) and every tensor that the reference quantizes rewritten by
 * mi355_quantize_weights: 2-D or higher, ne0 a multiple of 32, F32 or F16,
 * and not one of the embedding / table names the reference keeps (token_embed,
 * pos_embed, freqs_cis, ...).  Header, hyperparameters (SAM3; SAM2 including
 * the EdgeTAM extension), the other tensors and any bytes after the last
 * tensor are copied unchanged; records are re-padded to 32-byte offsets.
 * stats (may be NULL) receives the reference's summary counts.  Errors:
 * unknown magic / bad arguments INVALID_ARG, unsupported version or tensor type
 * UNSUPPORTED, I/O FAILED; unlike the reference a truncated input is an error,
 * not a silently shortened output. */
typedef struct mi355_quantize_stats {
    int32_t n_quantized, n_total;
    int64_t size_org;  /* F32-equivalent bytes of every tensor */
    int64_t size_new;  /* data bytes written */
} mi355_quantize_stats;
mi355_status mi355_model_quantize(mi355_context* ctx, const char* in_path, const char* out_path, int32_t qtype,
                                  mi355_quantize_stats* stats);

/* A SAM2 file's Hiera backbone in device memory: the tensors sam3_register_tensors
 * declares for it (sam3.cpp:1800-1840: "hiera.patch_embed.*", "hiera.pos_embed",
 * "hiera.pos_embed_window", "hiera.blocks.N.*" with ".proj.*" at stage
 * transitions), weights in the file's weight type when their rows are whole
 * blocks and F32 otherwise; the hyperparameters of sam2_load_hparams
 * (sam3.cpp:1568-1590); pos_embed [S0*S0][E] (S0 = img/4) computed by
 * mi355_hiera_pos_embed from the two tables; quantized linear weights
 * prepared (mi355_weight_prepare).  Everything mi355_hiera_encode takes besides
 * the image; valid until mi355_hiera_weights_free. */
typedef struct mi355_hiera_weights mi355_hiera_weights;
mi355_status mi355_hiera_weights_load(mi355_context* ctx, const mi355_model_file* f, mi355_hiera_weights** out);
void mi355_hiera_weights_free(mi355_hiera_weights* w);
mi355_status mi355_hiera_weights_get(const mi355_hiera_weights* w, mi355_hiera_hparams* hp,
                                     const mi355_hiera_block** blocks, int* n_blocks, const mi355_tensor** patch_w,
                                     const float** patch_b, const float** pos_embed);

/* Fusion in the encoder runners (no counterpart in the reference, whose graph
 * always materialises f32 activations; on by default).  When on, the passes
 * that feed a MUL_MAT with Q8_0/Q4_0/Q4_1 or F16 weights (LayerNorm, bias+GELU,
 * the attention output) write its activation operand (the same from_float
 * quantization ggml applies to those f32 rows), and the GEMMs run the
 * following node group in their epilogue (bias + residual with the window
 * unpartition; the ViT's qkv split + RoPE).  Off gives the unfused sequence
 * of node groups, for parity checks: both produce the same bits. */
mi355_status mi355_context_set_fusion(mi355_context* ctx, int enable);
/* The skinny MUL_MAT kernel (no counterpart in the reference; on by default):
 * on the fp16 route (MI355_MMQ_F16, and ggml-layout weights behind the
 * encoders' fused operands), quantized GEMMs with K <= 128 over at least 4096
 * activation rows (SAM2 Hiera's stage-1 projections, K = 96) run on a kernel
 * that keeps the whole weight matrix in LDS and streams the activation rows;
 * it computes every output with the tiled kernel's instruction sequence, so
 * both give the same bits.  On the int8 route (prepared weights, and Q8_0 /
 * Q4_0 under MI355_MMQ_AUTO) the same shapes (N % 4 == 0, no K split) run on
 * an int8 skinny kernel that keeps each wavefront's activation fragments in
 * registers and reads the small weight matrix from L2, again bit-identical to
 * the tiled int8 kernel.  Off routes both to the tiled kernels (for
 * comparisons). */
mi355_status mi355_context_set_skinny(mi355_context* ctx, int enable);

/* The kernel behind 2-D MUL_MATs with Q8_0 / Q4_0 / Q4_1 weights in the
 * ggml layout (no counterpart in the reference).  All give the same bits: the
 * exact int32 block sums combined as acc = fma(isum, d_a * d_w, acc) in block
 * order.
 * - MI355_MMQ_F16: fp16 MFMAs over the quants as exact halves, weights used in
 *   their ggml rows and decoded in registers;
 * - MI355_MMQ_INT8: src1 quantized to one-byte quants, weights repacked into
 *   int8 rows with separate scale arrays on each call, block sums on
 *   v_mfma_i32_32x32x32_i8;
 * - MI355_MMQ_AUTO (the default): MI355_MMQ_INT8 for Q8_0 and Q4_0 weights,
 *   MI355_MMQ_F16 for Q4_1 (the faster per call with the repack counted).
 * Prepared weights always take the int8 kernel; other MUL_MATs keep their
 * own kernels. */
typedef enum {
    MI355_MMQ_F16 = 0,
    MI355_MMQ_INT8 = 1,
    MI355_MMQ_AUTO = 2,
} mi355_mmq_kernel;
mi355_status mi355_context_set_mmq_kernel(mi355_context* ctx, int kernel);

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
