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

// Activation operand of the MFMA GEMM kernel, fp16 rows of K halves:
// q[i12*s2 + i13*s3 + m*s1 + k] (strides in halves).  On the quantized path
// these are the Q8 quants as exact fp16 integers, contiguous ([Z][M][K]),
// with the per-block scale d[(z*M + m)*dp + b] and, for Q8_1, the block sum
// term s[(z*M + m)*dp + b], both fp16 as ggml stores them; dp =
// mmq_scale_pitch(K) is the block count rounded up to even (padding slot
// zero), so a row's two scales of one K stage are one aligned dword.  On the
// F16 path q holds src1 converted to F16 (or src1 itself) and d, s are unused.
struct ActF16 {
    const void* q;
    int64_t s1, s2, s3;
    const void* d;
    const void* s;
    int64_t dp;
    int64_t M, K;
    const void* dh = nullptr;  // int8 operand (ACT_I8*): q int8 [M][s1], d = dl and dh [M][dp / 2] dwords
};
inline int64_t mmq_scale_pitch(int64_t K) { return ((K / 32) + 1) & ~(int64_t)1; }

// Output of a pass that feeds a MUL_MAT: F32 rows (y), F16 rows (q as fp16
// values: the operand of F16 weights), the quantized operand of the fp16-MFMA
// kernel (q fp16 quants [rows][K], d [rows][dp], and Q8_1 sums s for Q4_1
// weights), or that of the int8 kernel for prepared weights (q int8 quants
// [rows][K]; d as two dword arrays [rows][dp / 2]: d (dl) holds the scale of
// an even block in the low half, dh that of an odd block in the high half,
// zero for a missing odd block; s as before).
enum { ACT_F32 = 0, ACT_F16 = 1, ACT_Q8 = 2, ACT_Q8S = 3, ACT_I8 = 4, ACT_I8S = 5 };
struct ActOut {
    int mode;
    float* y;
    uint16_t* q;
    uint16_t* d;
    uint16_t* s;
    int64_t dp;
    uint32_t* dh = nullptr;
};
__host__ __device__ inline bool act_has_sums(int mode) { return mode == ACT_Q8S || mode == ACT_I8S; }

// ggml from_float into contiguous ggml rows: type 8 (Q8_0), 9 (Q8_1), 1 (F16).
hipError_t launch_quantize_ggml(const SrcView& src, int type, bool ref_variant, void* dst, hipStream_t st);
// from_float (x86 variant, Q8_0 or with_sum Q8_1 semantics) into the ActF16
// quantized layout: q [rows][K] fp16, d and s [rows][dp] fp16.
hipError_t launch_quantize_mmq(const SrcView& src, bool with_sum, int64_t dp, uint16_t* q, uint16_t* d, uint16_t* s,
                               hipStream_t st);
// F32/F16 strided rows -> contiguous F16 rows [rows][ne0] (round to nearest even).
hipError_t launch_convert_f16(const SrcView& src, uint16_t* dst, int64_t pitch, hipStream_t st);
// n contiguous elements of type src_type -> dst_type: F16 -> F32, F32 -> F16
// (RNE), Q8_0 / Q4_0 / Q4_1 -> F32 (ggml's to_float: d*q, d*(q-8), d*q + m).
hipError_t launch_convert_weights(const void* src, int src_type, void* dst, int dst_type, int64_t n, hipStream_t st);

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

// dst = W^T . A on MFMA for W in Q8_0 / Q4_0 / Q4_1 (A = quantized
// activations) or F16 (A = F16 activations); ne12/ne13 batch dims.  With
// dots != nullptr (block types only) the kernel writes the exact per-block
// int32 dots [z][m][n][b] instead of dst.
// K split (split-K) of a 2-D GEMM: ks partial sums of [M][N] f32 in part
// (ks * M * N * 4 bytes), added in split order by a reduction that also runs
// the epilogue.  ks = 1: no split.
struct MmqSplit {
    int ks;
    float* part;
    bool skinny = true;  // K <= 128 GEMMs at large M may take the skinny kernel
    int cus = 0;         // compute units (0: unknown); the int8 kernel sizes its tiles by it
};
// The split mmq_ksplit picks for a GEMM on a GPU with cus compute units.
int mmq_ksplit(int type, int64_t M, int64_t N, int64_t K, int64_t Z, int cus);
hipError_t launch_mmq(const MatW& w, const ActF16& a, const MatD& d, int64_t N, int64_t ne12, int64_t ne13,
                      int32_t* dots, void* align_buf, const MmqSplit& sp, hipStream_t st);
// Bytes of the 4-byte-pitch weight copy launch_mmq needs (0 when rows are aligned).
size_t mmq_align_bytes(const MatW& w, int64_t N, int64_t K);

// GEMM row -> row of another token order, or -1 (a padding token, dropped).
enum { ROWMAP_IDENTITY = 0, ROWMAP_WIN_UNPART = 1, ROWMAP_SAM2_UNPART = 2 };
struct RowMap {
    int kind;
    int W, H;   // image grid (tokens)
    int ws;     // window side
    int nwh;    // SAM2: windows along H of the padded grid
};

// Fused MUL_MAT epilogues (one 2-D GEMM, dst [M][N] never written; N % 4 == 0):
//   MMQ_EPI_RESIDUAL  out[map(m)][n] = res[map(m)][n] + (dst[m][n] + bias[n]),
//                     rows with map(m) = -1 dropped
//   MMQ_EPI_QKV       the ViT qkv split: u = dst + bias over N = 3E columns
//                     [q | k | v], RoPE on q and k (rope non-null), fp16 out to
//                     q/k/v [M/ntok][nh][ntok][hd] (the qkv_rope pass)
enum { MMQ_EPI_STORE = 0, MMQ_EPI_RESIDUAL = 1, MMQ_EPI_QKV = 2 };
struct LnArgs;
struct MmqEpi {
    int kind;
    const float* bias;  // [N]
    const float* res;   // [rows][N] (may be out)
    float* out;         // [rows][N]
    RowMap map;
    const float* rope;  // [ntok][hd/2][2] (cos, sin) or null
    _Float16 *q, *k, *v;
    int ntok, nh, hd;
    // int8 route, MMQ_EPI_RESIDUAL: the LayerNorm to run on `out` afterwards (the next
    // block's first), fused into the K-split reduction where the shape allows; else null
    const LnArgs* ln_next;
};
hipError_t launch_mmq_epi(const MatW& w, const ActF16& a, int64_t N, const MmqEpi& e, void* align_buf,
                          const MmqSplit& sp, hipStream_t st);
// The split-K reduction: dst rows (or the epilogue) from ks partial sums [ks][M][N] f32 in split order.
hipError_t launch_mmq_reduce(const float* part, int ks, int M, int N, char* dst, int64_t d_nb1, const MmqEpi* epi,
                             hipStream_t st);

// ---- int8-MFMA MUL_MAT (mmq8.hip)
// Activation operand with one-byte quants: q int8 [M][s1 bytes] (s1 a
// multiple of 16); the scales split by block parity into the operands of the
// kernel's scale MFMA; Q8_1 sums fp16 [M][2 nst] as ActF16's.
struct ActI8 {
    const void* q;        // int8 [M][s1]
    int64_t s1;
    const uint32_t* dl;   // [M][nst]: d of block 2s in the low half of dword s (high half zero)
    const uint32_t* dh;   // [M][nst]: d of block 2s + 1 in the high half (low half zero)
    const void* s;        // fp16 [M][2 nst] Q8_1 sums (Q4_1 weights)
    int64_t nst;          // mmq_scale_pitch(K) / 2
    int64_t M, K;
};
// Weights repacked for the int8 kernel: quants int8 [N][q_s1 bytes] (Q8_0 as
// stored, Q4_0 as nibble - 8, Q4_1 as the nibble 0..15), d (and Q4_1's m) fp16
// [N][dpw], dpw = mmq_scale_pitch(K) with a zero padding slot.
struct WRep {
    int type;
    int8_t* q;
    int64_t q_s1;
    _Float16* d;
    _Float16* m;
    int dpw;
    int64_t N, K;
};
// Bytes of the repacked form of N rows of K elements (0: not a repackable type).
size_t wrep_bytes(int type, int64_t N, int64_t K);
// The descriptor of a repacked form already at base (the layout launch_repack_weights writes:
// quants, then d, then m, each part 256-byte aligned).
WRep wrep_view(int type, int64_t N, int64_t K, void* base);
// Repacks the 2-D ggml weights w (rows at w.data + n * w.nb1) into dst (wrep_bytes) and describes it in *out.
hipError_t launch_repack_weights(const MatW& w, int64_t N, int64_t K, void* dst, WRep* out, hipStream_t st);
// Operands the int8 kernel takes (alignment, pitches, 32-bit buffer offsets).
bool mmq8_supported(const WRep& w, const ActI8& a);
// The K split (1: none) the int8 kernel runs an M x N x K GEMM with on cus compute units,
// chosen with its tile height by a cost model fitted to kernel times.
int mmq8_ksplit(int64_t M, int64_t N, int64_t K, int cus);
// The int8 kernel's tile height (128 or 64 rows) for that GEMM at K split ks.
int mmq8_tile_rows(int64_t M, int64_t N, int64_t K, int ks, int cus);
// dst = W^T . A (2-D) on int8 MFMA, bit-identical to launch_mmq on the same
// operands; epilogues and split-K as launch_mmq / launch_mmq_epi.
// With dots != nullptr the kernel writes the exact int32 block sums [M][N][K/32] instead.
hipError_t launch_mmq8(const WRep& w, const ActI8& a, const MatD& d, const MmqEpi* epi, const MmqSplit& sp,
                       hipStream_t st, int32_t* dots = nullptr);
// from_float (x86 variant) into the int8 operand layout: q [rows][s1] int8,
// d -> dl [rows][dp / 2] followed by dh [rows][dp / 2] (uint32), s as ActF16's.
hipError_t launch_quantize_mmq_i8(const SrcView& src, bool with_sum, int64_t s1, int64_t dp, int8_t* q, uint16_t* d,
                                  uint16_t* s, hipStream_t st);


// Row softmax of scale*x (F32, strided rows) into dst (F32, strided rows).
hipError_t launch_soft_max(const SrcView& src, float scale, char* dst, const int64_t dnb[4], hipStream_t st);

// FLASH_ATTN_EXT operands (byte strides; rows of D contiguous elements).
struct FaArgs {
    const char* q;
    const char* k;
    const char* v;
    float* dst;  // [D, nh, nq, B] contiguous
    int64_t q_nb1, q_nb2, q_nb3;
    int64_t k_nb1, k_nb2, k_nb3;
    int64_t v_nb1, v_nb2, v_nb3;
    int nq, nkv, nh, rk2, rv2;  // rk2 = nh / n_head_k, rv2 = nh / n_head_v
    float c;                    // |scale| * log2(e), at least 1e-30
    int negq;                   // scale < 0: Q enters negated
    ActOut out;                 // mode ACT_F32: dst; else the next MUL_MAT's operand, rows
                                // b*nq + iq of K = nh*D (Q8 quants + scales or F16)
    int B;                      // batch count (set by launch_fattn)
    int kv_split, kv_chunk;     // keys split into kv_split ranges of kv_chunk (a multiple of 64);
    float* part;                // > 1: per range unnormalised O [D] and (max, sum) per query,
                                // combined by a second kernel; fattn_part_bytes() of workspace
};
// Key-range split for grids too small to fill the GPU (1 = none), and its workspace.
int fattn_kv_split(int nq, int nkv, int nh, int B, int cus);
size_t fattn_part_bytes(int D, int nq, int nh, int B, int kv_split);
hipError_t launch_fattn(const FaArgs& a, int D, bool qf32, bool kvf32, int B, hipStream_t st);

// F32 x F32 MUL_MAT: D[z][m][n] = sum_k X[z][m][k] W[z'][n][k] (byte strides).
struct GemmF32Args {
    const float* W;
    int64_t w_nb1, w_nb2, w_nb3;
    const float* X;
    int64_t x_nb1, x_nb2, x_nb3;
    float* D;
    int64_t d_nb1, d_nb2, d_nb3;
    int M, N, K, ne12, r2, r3;
    const float* bias = nullptr;  // [N], added to every row (or none)
    // implicit 3x3 / stride 1 / pad 1 convolution: X is a token-major map [H*Wd][C], row m
    // of the GEMM is output pixel m, and K = 9*C runs (tap, channel) with W rows in that order
    int conv = 0, H = 0, Wd = 0, C = 0;
    // optional addend [M][N] (row pitch N floats, Z == 1), added after the bias: D = (acc + bias) + add
    const float* add = nullptr;
    // K split for grids too small to fill the device (Z == 1 only): when part is given, the
    // launch may split K into ranges whose fp32 partial sums go to part [split][M][N] (at most
    // part_bytes) and are then added in split order, with the bias, by a reduce pass
    float* part = nullptr;
    size_t part_bytes = 0;
};
hipError_t launch_gemm_f32(const GemmF32Args& a, int Z, hipStream_t st);
// partial-sum bytes launch_gemm_f32 uses for an M x N x K tiled GEMM (0: no K split)
size_t gemm_f32_part_bytes(int64_t M, int64_t N, int64_t K);
// D[m][n] = bias[n] + part[0][m][n] + ... + part[S - 1][m][n], added in split order
// (float4 columns: N % 4 == 0; D row pitch d_nb1 bytes; bias may be null; f16out: D holds
// fp16, the sums rounded RNE)
hipError_t launch_split_reduce(const float* part, int S, int M, int N, const float* bias, float* D, int64_t d_nb1,
                               hipStream_t st, bool f16out = false);

// K split count of a GEMM of `tiles` 128 x 128 output tiles and nst K stages: grids of `full`
// tiles or more are not split; smaller ones take the S (at most 16, at least four stages per
// split, no split left empty) that minimises the busiest CU's stage count, ceil(tiles * S /
// 256) * ceil(nst / S), plus the reduce (a launch and S + 1 passes over M x N floats at
// 4 TB/s), in units of stage_us, one stage's time alone on a CU
inline int gemm_ksplit(int64_t tiles, int64_t full, int64_t M, int64_t N, int64_t nst, double stage_us) {
    if (tiles >= full || N % 4 != 0) return 1;
    double best = (double)((tiles + 255) / 256) * (double)nst;
    int bs = 1;
    for (int S = 2; S <= 16 && nst >= 4 * S; ++S) {
        const int64_t sps = (nst + S - 1) / S;
        if ((nst + sps - 1) / sps != S) continue;
        const double red = (3.0 + (double)(S + 1) * (double)M * (double)N * 4.0 / 4.0e6) / stage_us;
        const double c = (double)((tiles * S + 255) / 256) * (double)sps + red;
        if (c < best) {
            best = c;
            bs = S;
        }
    }
    return bs;
}

// ---- SAM3 ViT glue (rows of E contiguous floats)
struct LnArgs {
    const float* x;     // [rows][E], image token order
    const float* add;   // optional addend before the norm: same rows, or a tiled [add_grid^2][E] table
    int add_grid;       // > 0: add row = (y % add_grid) * add_grid + x % add_grid
    const float* w;     // optional affine (ggml_mul), [E]
    const float* b;     // optional affine (ggml_add), [E]
    ActOut out;         // [rows][E]; row win_row(r) when ws > 0, else r
    int64_t rows;
    int E;
    int grid;           // tokens per image side (rows = grid^2 when ws > 0 or add_grid > 0)
    int ws;             // window size of the output order (0: image order)
    float eps;
};
hipError_t launch_layer_norm(const LnArgs& a, hipStream_t st);
// x = x + (sum of ks partial sums [ks][rows][1024] in order + bias), then the LayerNorm a of
// that x (a.x == x, E = 1024, no addend): the K-split reduction and the next LayerNorm in one pass
hipError_t launch_reduce_residual_ln1024(const float* part, int ks, const float* bias, float* x, const LnArgs& a,
                                        hipStream_t st);

struct QkvArgs {
    const float* qkv;   // [M][3E] (rows in attention-batch order)
    const float* bias;  // [3E]
    const float* rope;  // [N][HD/2][2] (cos, sin) or null
    _Float16* q;        // [M/N][NH][N][HD] each
    _Float16* k;
    _Float16* v;
    int64_t M;
    int N, NH, HD;
};
hipError_t launch_qkv_rope(const QkvArgs& a, hipStream_t st);
hipError_t launch_proj_residual(float* x, const float* p, const float* b, int64_t rows, int E, int grid, int ws,
                                hipStream_t st);
hipError_t launch_bias_gelu(float* h, const float* b, int64_t rows, int n, hipStream_t st);
hipError_t launch_bias_gelu_act(const float* h, const float* b, int64_t rows, int n, const ActOut& o, hipStream_t st);
// h + b -> activation (act 0: gelu_erf, 1: ggml_gelu table form) -> an int8 operand
// (o.mode ACT_I8 / ACT_I8S; n % 32 == 0, rows * n / 16 < 2^30).
hipError_t launch_bias_act_i8(int act, const float* h, const float* b, int64_t rows, int n, const ActOut& o,
                              hipStream_t st);
hipError_t launch_bias_residual(float* x, const float* f, const float* b, int64_t rows, int n, hipStream_t st);
hipError_t launch_im2col(const float* img, float* cols, int C, int Himg, int Wimg, int P, int grid, hipStream_t st);

// ---- SAM2 Hiera glue
struct HieraLnArgs {
    const float* x;    // [H*W][C] image order
    const float* w;    // [C]
    const float* b;    // [C]
    ActOut out;        // [rows_out][C]: window order (ws > 0, padding rows zero) or image order
    ActOut out_img;    // optional image-order copy (ws > 0 only; out_img.y and .q null when unused)
    int64_t rows_out;  // nW * ws * ws, or H * W
    int C, W, H, ws, nwh;
    float eps;
};
hipError_t launch_hiera_ln(const HieraLnArgs& a, hipStream_t st);
struct HieraQkvArgs {
    const float* qkv;   // [B*Nkv][3C] window-order rows
    const float* bias;  // [3C]
    _Float16* q;        // [B][NH][Nq][HD]
    _Float16* k;        // [B][NH][Nkv][HD]
    _Float16* v;
    int B, Nkv, Nq, NH, HD;
    int qpool;          // Q is the 2x2 max over each window's ws x ws grid
    int ws;
};
hipError_t launch_hiera_qkv(const HieraQkvArgs& a, hipStream_t st);
// Q of a pooled block: the 2x2 window max of the unpooled fp16 q [B][NH][Nkv][HD] into
// q [B][NH][Nq][HD] (Nkv = ws * ws, Nq = Nkv / 4).
hipError_t launch_hiera_qpool(const _Float16* qf, _Float16* q, int64_t B, int NH, int Nkv, int Nq, int ws, int HD,
                              hipStream_t st);
hipError_t launch_hiera_bias_maxpool(const float* p, const float* b, float* out, int C, int W, int H, bool pool,
                                     hipStream_t st);
hipError_t launch_hiera_proj_residual(float* x, const float* shortcut, const float* p, const float* b, int C, int W,
                                      int H, int ws, int nwh, hipStream_t st);
hipError_t launch_bias_gelu_tanh(float* h, const float* b, int64_t rows, int n, hipStream_t st);
hipError_t launch_bias_gelu_tanh_act(const float* h, const float* b, int64_t rows, int n, const ActOut& o,
                                     hipStream_t st);
// conv2d columns cols[m][k] at row pitch kp >= C*KH*KW, zero past K (see im2col_pad_kernel)
hipError_t launch_im2col_pad(const float* img, float* cols, int C, int Hin, int Win, int KH, int KW, int stride, int pad,
                             int OH, int OW, int kp, bool round16, hipStream_t st);
// rows x K F32 (or F16, widened) -> rows x kp F32, zero past K
hipError_t launch_pad_rows_f32(const void* src, bool f16, int64_t rows, int K, int kp, float* dst, hipStream_t st);
// SimpleFPN neck passes (neck.hip); activations token-major [H*W][C]
hipError_t launch_deconv_pack(const void* w, int wtype, int Cin, int Cout, uint16_t* out, hipStream_t st);
hipError_t launch_deconv_scatter(const float* D, const float* b, int H, int W, int Cout, bool gelu, float* y,
                                 hipStream_t st);
hipError_t launch_im2col3x3(const float* x, int H, int W, int C, bool f16, void* cols, hipStream_t st);
hipError_t launch_conv3x3_pack(const float* w, int Cin, int Cout, float* out, hipStream_t st);
hipError_t launch_conv3x3_pack_f16(const uint16_t* w, int Cin, int Cout, uint16_t* out, hipStream_t st);
// taps: 9 (3x3, kernel packed by launch_conv3x3_pack_f16), 1 (1x1, the kernel as
// stored) or 4 (2x2 / stride-2 conv-transpose, kernel packed by launch_deconv_pack,
// N = 4 * Cout, y the 2x map, GELU-erf after the bias if gelu). Taps 1 and 9 may split K
// into ranges whose partial sums go to part [split][M][N] (at most part_bytes; none without
// part) and are added, with the bias, by launch_split_reduce.
// x16 / y16: the map in / out is fp16 (the f32 values rounded RNE, which the kernel's own rounding
// of an F32 map gives: the same products), for maps only these kernels read.
hipError_t launch_conv_f16(int taps, const void* x, bool x16, const uint16_t* w, const float* bias, int H, int W, int C,
                           int N, bool gelu, void* y, bool y16, hipStream_t st, float* part = nullptr,
                           size_t part_bytes = 0);
// partial-sum bytes launch_conv_f16 uses for taps 1 or 9 over M pixels, C input and N output
// channels (0: no K split)
size_t conv_f16_part_bytes(int taps, int64_t M, int64_t C, int64_t N);
hipError_t launch_bias_rows(float* y, const float* b, int64_t rows, int C, hipStream_t st);
hipError_t launch_maxpool2(const float* x, int H, int W, int C, float* y, hipStream_t st);
hipError_t launch_hiera_pos_embed(const float* bkg, int E, int bh, int bw, const float* win, int ws, int H, int W,
                                  float* out, hipStream_t st);

}  // namespace mi355
