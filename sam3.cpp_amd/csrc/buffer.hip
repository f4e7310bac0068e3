// Device buffers of the backend: the ggml-backend buffer calls sam3.cpp makes
// around a graph, on this backend.
//   ggml_backend_alloc_ctx_tensors (sam3.cpp:3320, the model's weights) and
//   ggml_gallocr_alloc_graph (sam3.cpp:6101-6115, a graph's intermediates)
//     -> mi355_buffer_alloc + mi355_buffer_place
//   ggml_backend_tensor_set / _get (sam3.cpp:3156-3179, 6117) and
//   ggml_backend_tensor_memset / ggml_backend_buffer_clear
//     -> mi355_tensor_set / _get / _memset, mi355_buffer_clear
// Copies are ordered on the context's stream and return once the host side is
// done, as the ggml calls do.  Memsets run as a byte-fill kernel, so a caller
// may also record them into a HIP graph.
#include <cstring>

#include "context.h"

struct mi355_buffer {
    int device = 0;
    void* base = nullptr;
    size_t size = 0;
};

namespace {

using namespace mi355;

constexpr size_t kBufAlign = 256;

__global__ __launch_bounds__(256) void fill_bytes_kernel(uint8_t* __restrict__ p, size_t n, uint32_t v4) {
    // 16-byte stores over the aligned middle, single bytes at the two ends
    const size_t head = (16 - (reinterpret_cast<uintptr_t>(p) & 15)) & 15;
    const size_t h = head < n ? head : n;
    const size_t nv = (n - h) / 16;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint4* mid = reinterpret_cast<uint4*>(p + h);
    for (size_t i = t; i < nv; i += stride) mid[i] = make_uint4(v4, v4, v4, v4);
    const uint8_t b = (uint8_t)(v4 & 0xff);
    if (t < h) p[t] = b;
    const size_t tail0 = h + nv * 16;
    if (t < n - tail0) p[tail0 + t] = b;
}

mi355_status fill(mi355_context* ctx, void* p, uint8_t value, size_t n) {
    if (n == 0) return MI355_STATUS_SUCCESS;
    const uint32_t v4 = 0x01010101u * value;
    const size_t nv = n / 16 + 1;
    const unsigned grid = (unsigned)std::min<size_t>((nv + 255) / 256, 4096);
    fill_bytes_kernel<<<grid, 256, 0, ctx->stream>>>(static_cast<uint8_t*>(p), n, v4);
    return hip_check(ctx, hipGetLastError(), "fill_bytes launch");
}

// ggml_nbytes of the layout: the span from data to one past the last element
// (blocks for quantized types), 0 for an empty tensor; false on overflow or an
// unknown type or layout.  A prepared weight spans its prepared form.
bool layout_bytes(const mi355_tensor* t, size_t* out) {
    *out = 0;
    if (t->layout == MI355_LAYOUT_INT8) {  // a prepared weight: the bytes of its prepared form
        if (!(t->type == T_Q8_0 || t->type == T_Q4_0 || t->type == T_Q4_1) || t->ne[0] < 0 || t->ne[1] < 0 ||
            t->ne[2] != 1 || t->ne[3] != 1 || t->ne[0] % 32 != 0)
            return false;
        *out = wrep_bytes(t->type, t->ne[1], t->ne[0]);
        return true;
    }
    const int64_t ts = type_size(t->type), bs = blck(t->type);
    if (!ts || !bs || !dims_ok(t)) return false;
    for (int i = 0; i < 4; ++i)
        if (t->ne[i] == 0) return true;
    unsigned __int128 n = bs == 1 ? (unsigned __int128)ts : (unsigned __int128)t->ne[0] * (uint64_t)t->nb[0] / (uint64_t)bs;
    for (int i = bs == 1 ? 0 : 1; i < 4; ++i) n += (unsigned __int128)(t->ne[i] - 1) * (uint64_t)t->nb[i];
    if (n > (unsigned __int128)SIZE_MAX) return false;
    *out = (size_t)n;
    return true;
}

mi355_status check_range(mi355_context* ctx, const mi355_tensor* t, const void* host, size_t offset, size_t size,
                         const char* what) {
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "%s: null context", what);
    if (!t || !t->data) return fail(ctx, MI355_STATUS_INVALID_ARG, "%s: null tensor or data", what);
    if (!host && size) return fail(ctx, MI355_STATUS_INVALID_ARG, "%s: null host pointer", what);
    size_t nb = 0;
    if (!layout_bytes(t, &nb)) return fail(ctx, MI355_STATUS_INVALID_ARG, "%s: bad tensor layout", what);
    if (offset > nb || size > nb - offset)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "%s: offset %zu + size %zu beyond the tensor's %zu bytes", what,
                    offset, size, nb);
    return MI355_STATUS_SUCCESS;
}

}  // namespace

extern "C" {

size_t mi355_buffer_alignment(void) { return kBufAlign; }

mi355_status mi355_buffer_alloc(mi355_context* ctx, size_t size, mi355_buffer** out) {
    if (!out) return fail(ctx, MI355_STATUS_INVALID_ARG, "buffer_alloc: out is null");
    *out = nullptr;
    if (!ctx) return fail(nullptr, MI355_STATUS_INVALID_ARG, "buffer_alloc: null context");
    (void)hipSetDevice(ctx->device);
    void* p = nullptr;
    // a zero-size buffer still gets a distinct base (ggml allocates at least one alignment unit)
    const hipError_t e = hipMalloc(&p, size ? size : kBufAlign);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(ctx, MI355_STATUS_ALLOC_FAILED, "buffer_alloc: hipMalloc(%zu): %s", size, hipGetErrorString(e));
    }
    mi355_buffer* b = new mi355_buffer();
    b->device = ctx->device;
    b->base = p;
    b->size = size;
    *out = b;
    return MI355_STATUS_SUCCESS;
}

void mi355_buffer_free(mi355_buffer* buf) {
    if (!buf) return;
    (void)hipSetDevice(buf->device);
    (void)hipFree(buf->base);  // waits for the device's work that may still use it
    delete buf;
}

void* mi355_buffer_base(const mi355_buffer* buf) { return buf ? buf->base : nullptr; }
size_t mi355_buffer_size(const mi355_buffer* buf) { return buf ? buf->size : 0; }

mi355_status mi355_buffer_place(const mi355_buffer* buf, size_t offset, mi355_tensor* t) {
    if (!buf || !t) return fail(nullptr, MI355_STATUS_INVALID_ARG, "buffer_place: null argument");
    if (offset % kBufAlign != 0)
        return fail(nullptr, MI355_STATUS_INVALID_ARG, "buffer_place: offset %zu not a multiple of %zu", offset, kBufAlign);
    size_t nb = 0;
    if (!layout_bytes(t, &nb)) return fail(nullptr, MI355_STATUS_INVALID_ARG, "buffer_place: bad tensor layout");
    if (offset > buf->size || nb > buf->size - offset)
        return fail(nullptr, MI355_STATUS_INVALID_ARG, "buffer_place: %zu bytes at %zu exceed the buffer's %zu", nb,
                    offset, buf->size);
    t->data = static_cast<char*>(buf->base) + offset;
    return MI355_STATUS_SUCCESS;
}

size_t mi355_tensor_nbytes(const mi355_tensor* t) {
    size_t n = 0;
    return t && layout_bytes(t, &n) ? n : 0;
}

mi355_status mi355_buffer_clear(mi355_context* ctx, mi355_buffer* buf, uint8_t value) {
    if (!ctx || !buf) return fail(ctx, MI355_STATUS_INVALID_ARG, "buffer_clear: null argument");
    if (buf->device != ctx->device) return fail(ctx, MI355_STATUS_INVALID_ARG, "buffer_clear: buffer on another device");
    (void)hipSetDevice(ctx->device);
    const mi355_status st = fill(ctx, buf->base, value, buf->size);
    if (st != MI355_STATUS_SUCCESS) return st;
    return hip_check(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

mi355_status mi355_tensor_set(mi355_context* ctx, const mi355_tensor* t, const void* data, size_t offset, size_t size) {
    mi355_status st = check_range(ctx, t, data, offset, size, "tensor_set");
    if (st != MI355_STATUS_SUCCESS || size == 0) return st;
    (void)hipSetDevice(ctx->device);
    st = hip_check(ctx, hipMemcpyAsync(static_cast<char*>(t->data) + offset, data, size, hipMemcpyHostToDevice, ctx->stream),
                   "tensor_set: hipMemcpyAsync");
    if (st != MI355_STATUS_SUCCESS) return st;
    return hip_check(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

mi355_status mi355_tensor_get(mi355_context* ctx, const mi355_tensor* t, void* data, size_t offset, size_t size) {
    mi355_status st = check_range(ctx, t, data, offset, size, "tensor_get");
    if (st != MI355_STATUS_SUCCESS || size == 0) return st;
    (void)hipSetDevice(ctx->device);
    st = hip_check(ctx, hipMemcpyAsync(data, static_cast<const char*>(t->data) + offset, size, hipMemcpyDeviceToHost, ctx->stream),
                   "tensor_get: hipMemcpyAsync");
    if (st != MI355_STATUS_SUCCESS) return st;
    return hip_check(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

mi355_status mi355_tensor_memset(mi355_context* ctx, const mi355_tensor* t, uint8_t value, size_t offset, size_t size) {
    const uint8_t probe = 0;
    mi355_status st = check_range(ctx, t, &probe, offset, size, "tensor_memset");
    if (st != MI355_STATUS_SUCCESS || size == 0) return st;
    (void)hipSetDevice(ctx->device);
    st = fill(ctx, static_cast<char*>(t->data) + offset, value, size);
    if (st != MI355_STATUS_SUCCESS) return st;
    return hip_check(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

}  // extern "C"
