// The fixed device scratch of mi355_mul_mat_noalloc: the quantized (or F16)
// activation operand, the split-K partial sums and the 4-byte-pitch weight
// copy of one MUL_MAT live here instead of in the context's workspace, so the
// entry point never allocates.  Each device that loads the library holds its
// own copy of the array until the process ends; its address on a device comes
// from hipGetSymbolAddress (the array's name in host code is only a stand-in).
#include <mutex>

#include "context.h"

namespace {

static __device__ __align__(256) uint8_t scratch[MI355_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch[kMaxDevices] = {};

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
    ctx->scratch = g_scratch[ctx->device];
    return MI355_STATUS_SUCCESS;
}

}  // namespace mi355
