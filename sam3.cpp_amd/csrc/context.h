// Host-side internals shared by the C-ABI translation units: the context
// object behind mi355_context* and the validation / error / timing helpers.
#pragma once

#include <hip/hip_runtime.h>

#include <functional>
#include <map>
#include <string>
#include <vector>

#include "kernels.h"
#include "sam3_mi355.h"

struct mi355_context {
    int device = 0;
    int cus = 0;               // compute units of the device (split-K sizing)
    hipStream_t stream = nullptr;
    void* ws = nullptr;        // per-call scratch of mul_mat (activation operand, scales)
    size_t ws_size = 0;
    void* enc = nullptr;       // activation buffers of the image-encoder runner
    size_t enc_size = 0;
    void* neck = nullptr;      // maps and scratch of the SimpleFPN neck
    size_t neck_size = 0;
    // device address of the no-allocation entry point's static scratch on this
    // context's device (null if it could not be resolved: scratch_error says why)
    void* scratch = nullptr;
    std::string scratch_error;
    hipEvent_t scratch_done = nullptr;  // recorded after this context's last no-allocation call
    std::string last_error;
    // encoder runners: producer passes write the next MUL_MAT's operand
    bool fuse = true;
    // quantized 2-D MUL_MATs with K <= 128 over at least 4096 rows take a skinny kernel: the
    // fp16 route's (ggml-layout Q4_1 under MI355_MMQ_AUTO, any quantized type under
    // MI355_MMQ_F16) or the int8 route's (prepared weights, Q8_0 / Q4_0 under AUTO; N % 4 == 0,
    // no K split); F16 weights stay on the tiled kernel
    bool skinny = true;
    // kernel of 2-D MUL_MATs with block-quantized weights (MI355_MMQ_*)
    int mmq_kernel = MI355_MMQ_AUTO;
    // kernel timing
    bool prof = false;
    struct Pending { const char* name; hipEvent_t a, b; };
    std::vector<Pending> pending;
    std::vector<std::string> names;
    std::map<std::string, std::pair<int, double>> totals;
};

namespace mi355 {

mi355_status fail(mi355_context* ctx, mi355_status st, const char* fmt, ...);
mi355_status hip_check(mi355_context* ctx, hipError_t e, const char* what);
int64_t type_size(int t);
int blck(int t);
int64_t row_size(int t, int64_t ne0);
// ne, nb non-negative and the ggml layout
bool dims_ok(const mi355_tensor* t);
// a prepared weight (mi355_weight_prepare's output): 2-D Q8_0 / Q4_0 / Q4_1, K % 32 == 0, 256-byte aligned
bool prepared_ok(const mi355_tensor* t);
SrcView view_of(const mi355_tensor* t);
size_t align_up(size_t x);
// Grows a device buffer owned by the context to at least bytes (waits for the
// stream first: earlier kernels may still read the old buffer).
mi355_status ensure_buffer(mi355_context* ctx, void** buf, size_t* size, size_t bytes);

// The activation layout a producer pass should write for weights of type t:
// Q8 quants for Q8_0/Q4_0, Q8 with Q8_1 sums for Q4_1, F16 for F16, F32 otherwise.
int act_mode_for(int weight_type);
// The same for a weight tensor: a prepared weight (MI355_LAYOUT_INT8) takes the
// int8 operand (ACT_I8, or ACT_I8S for Q4_1).
int act_mode_for_weight(const mi355_tensor* w);
// MUL_MAT of weights s0 with an activation operand already in the layout
// act_mode_for(s0->type) describes (a: quants or F16 rows, scales), as a
// fused producer pass writes it; dst F32 [N][M] rows.  Same validation and
// kernels as mi355_mul_mat minus the activation quantize.  With epi the
// epilogue replaces the dst store (dst only gives the shape).
mi355_status mul_mat_act(mi355_context* ctx, const mi355_tensor* s0, const ActF16& a, const mi355_tensor* dst,
                         const MmqEpi* epi = nullptr);
// The host-side checks of mi355_flash_attn_ext (no launch).
mi355_status check_flash_attn(mi355_context* ctx, const mi355_tensor* q, const mi355_tensor* k, const mi355_tensor* v,
                              const mi355_tensor* mask, float max_bias, float logit_softcap, const mi355_tensor* dst);
// FLASH_ATTN_EXT with the checks of mi355_flash_attn_ext; with op the output
// goes to the next MUL_MAT's operand (rows b*n_q + iq, K = n_head*D) instead
// of dst (which still gives the shape).
mi355_status flash_attn_act(mi355_context* ctx, const mi355_tensor* q, const mi355_tensor* k, const mi355_tensor* v,
                            const mi355_tensor* mask, float scale, float max_bias, float logit_softcap,
                            const mi355_tensor* dst, const ActOut* op);
// mul_mat_act with a fused epilogue (residual or qkv split); dst [M][N] never
// exists.
mi355_status mul_mat_epi(mi355_context* ctx, const mi355_tensor* s0, const ActF16& a, const MmqEpi& e);

// Resolves the device address of the static scratch array of
// mi355_mul_mat_noalloc on ctx's device (current) into ctx->scratch; the
// lookup runs once per device.
mi355_status noalloc_scratch_init(mi355_context* ctx);
// Runs work (launches on ctx's stream that use the static scratch) ordered after the device's
// previous no-allocation call from another context, and records ctx's scratch event after it;
// not under stream capture.  The launches are asynchronous: the host lock is held only while
// they are issued.
mi355_status noalloc_run(mi355_context* ctx, const std::function<mi355_status()>& work);
// The context's scratch event, before the context is freed (its stream synchronized).
void noalloc_release(mi355_context* ctx);

// Brackets one launch with events when timing is enabled.
struct Timed {
    mi355_context* c;
    const char* name;
    hipEvent_t a = nullptr;
    Timed(mi355_context* ctx, const char* n) : c(ctx), name(n) {
        if (c && c->prof && hipEventCreate(&a) == hipSuccess) (void)hipEventRecord(a, c->stream);
    }
    hipError_t done(hipError_t e) {
        if (!a) return e;
        hipEvent_t b = nullptr;
        if (hipEventCreate(&b) == hipSuccess) {
            (void)hipEventRecord(b, c->stream);
            c->pending.push_back({name, a, b});
        } else {
            (void)hipEventDestroy(a);
        }
        a = nullptr;
        return e;
    }
};

}  // namespace mi355
