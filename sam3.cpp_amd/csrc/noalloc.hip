// The fixed device scratch of mi355_mul_mat_noalloc: the quantized (or F16)
// activation operand, the split-K partial sums and the 4-byte-pitch weight
// copy of one MUL_MAT live here instead of in the context's workspace, so the
// entry point never allocates.  Each device that loads the library holds its
// own copy of the array until the process ends; its address on a device comes
// from hipGetSymbolAddress (the array's name in host code is only a stand-in).
//
// Calls from different streams (several contexts or a context's stream
// changing hands) are ordered on the array: each context owns one event,
// created with the context; a call makes its stream wait for the event the
// device's previous call recorded (when another context recorded it), runs,
// and records its own.  Under stream capture neither happens (the captured
// work runs when the graph is launched, which the caller orders).
#include <functional>
#include <mutex>

#include "context.h"

namespace {

static __device__ __align__(256) uint8_t scratch[MI355_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch[kMaxDevices] = {};
hipEvent_t g_last[kMaxDevices] = {};  // event recorded after the device's latest call (owned by its context)

}  // namespace

namespace mi355 {

mi355_status noalloc_scratch_init(mi355_context* ctx) {
    if (ctx->device < 0 || ctx->device >= kMaxDevices)
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "noalloc scratch: device %d beyond %d", ctx->device, kMaxDevices);
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_scratch[ctx->device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            (void)hipGetLastError();
            return fail(ctx, MI355_STATUS_FAILED, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        }
        g_scratch[ctx->device] = p;
    }
    if (!ctx->scratch_done) {
        const hipError_t e = hipEventCreateWithFlags(&ctx->scratch_done, hipEventDisableTiming);
        if (e != hipSuccess) {
            ctx->scratch_done = nullptr;
            (void)hipGetLastError();
            return fail(ctx, MI355_STATUS_FAILED, "noalloc scratch event: %s", hipGetErrorString(e));
        }
    }
    ctx->scratch = g_scratch[ctx->device];
    return MI355_STATUS_SUCCESS;
}

mi355_status noalloc_run(mi355_context* ctx, const std::function<mi355_status()>& work) {
    std::lock_guard<std::mutex> lk(g_mu);
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(ctx->stream, &cap) != hipSuccess) {
        (void)hipGetLastError();
        cap = hipStreamCaptureStatusNone;
    }
    const bool order = cap == hipStreamCaptureStatusNone;
    hipEvent_t& last = g_last[ctx->device];
    if (order && last && last != ctx->scratch_done) {
        const hipError_t e = hipStreamWaitEvent(ctx->stream, last, 0);
        if (e != hipSuccess) return hip_check(ctx, e, "noalloc: wait for the previous user of the scratch");
    }
    const mi355_status st = work();
    if (order) {
        const hipError_t e = hipEventRecord(ctx->scratch_done, ctx->stream);
        if (e != hipSuccess) return hip_check(ctx, e, "noalloc: record the scratch event");
        last = ctx->scratch_done;
    }
    return st;
}

void noalloc_release(mi355_context* ctx) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (ctx->device >= 0 && ctx->device < kMaxDevices && g_last[ctx->device] == ctx->scratch_done)
        g_last[ctx->device] = nullptr;  // the caller synchronized the stream: nothing is left to wait for
    if (ctx->scratch_done) (void)hipEventDestroy(ctx->scratch_done);
    ctx->scratch_done = nullptr;
}

}  // namespace mi355
