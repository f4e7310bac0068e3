// A C++ caller of the backend that uses nothing but include/sam3_mi355.h:
// the way sam3.cpp's loader and graph runner would drive it (no torch, no
// Python).  It loads tests/golden/capi_fixture.bin, allocates device buffers
// through the buffer API (ggml_backend_alloc_ctx_tensors /
// ggml_gallocr_alloc_graph, sam3.cpp:3320, 6101-6115), uploads the operands
// with mi355_tensor_set (ggml_backend_tensor_set, sam3.cpp:3156-3179), asks
// the supports queries, runs one Q8_0 MUL_MAT and one FLASH_ATTN_EXT, reads
// the results back with mi355_tensor_get and checks them against the
// oracle's results stored in the fixture:
//   mul_mat:        |got - ggml| <= 1e-5 * sum_b |d_w d_a| sum_j |q_w q_a|
//   flash_attn_ext: |got - exact| <= 2e-3 * (attention of |V|)
// It also clears a tensor with mi355_tensor_memset and reads it back.
// Exit status: 0 pass, 1 a result out of bounds, 2 no usable device,
// 3 an API error, 4 a bad fixture.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "sam3_mi355.h"

namespace {

struct Rec {
    uint32_t type;
    std::vector<uint8_t> bytes;
};

bool load_fixture(const char* path, std::map<std::string, Rec>* out) {
    FILE* f = std::fopen(path, "rb");
    if (!f) return false;
    char magic[8];
    uint32_t n = 0;
    bool ok = std::fread(magic, 1, 8, f) == 8 && std::memcmp(magic, "MI355FX1", 8) == 0 && std::fread(&n, 4, 1, f) == 1;
    for (uint32_t i = 0; ok && i < n; ++i) {
        char name[33] = {};
        uint32_t et = 0, zero = 0;
        uint64_t nb = 0;
        ok = std::fread(name, 1, 32, f) == 32 && std::fread(&et, 4, 1, f) == 1 && std::fread(&zero, 4, 1, f) == 1 &&
             std::fread(&nb, 8, 1, f) == 1 && nb < (64u << 20);
        if (!ok) break;
        Rec r;
        r.type = et;
        r.bytes.resize(nb);
        ok = std::fread(r.bytes.data(), 1, nb, f) == nb;
        const size_t pad = (8 - nb % 8) % 8;
        char skip[8];
        ok = ok && std::fread(skip, 1, pad, f) == pad;
        (*out)[name] = std::move(r);
    }
    std::fclose(f);
    return ok;
}

template <typename T>
std::vector<T> as(const Rec& r) {
    std::vector<T> v(r.bytes.size() / sizeof(T));
    std::memcpy(v.data(), r.bytes.data(), v.size() * sizeof(T));
    return v;
}

mi355_tensor tensor(int type, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3, int64_t type_size, int64_t row) {
    mi355_tensor t;
    std::memset(&t, 0, sizeof(t));
    t.type = type;
    t.ne[0] = ne0;
    t.ne[1] = ne1;
    t.ne[2] = ne2;
    t.ne[3] = ne3;
    t.nb[0] = type_size;
    t.nb[1] = row;
    t.nb[2] = row * ne1;
    t.nb[3] = row * ne1 * ne2;
    return t;
}

size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

mi355_context* g_ctx = nullptr;

#define CHECK(call)                                                                                          \
    do {                                                                                                     \
        const mi355_status st_ = (call);                                                                     \
        if (st_ != MI355_STATUS_SUCCESS) {                                                                   \
            std::fprintf(stderr, "%s: %s (%s)\n", #call, mi355_status_to_string(st_), mi355_last_error(g_ctx)); \
            return 3;                                                                                        \
        }                                                                                                    \
    } while (0)

}  // namespace

int main(int argc, char** argv) {
    if (argc < 2) {
        std::fprintf(stderr, "usage: %s capi_fixture.bin\n", argv[0]);
        return 4;
    }
    std::map<std::string, Rec> fx;
    const char* names[] = {"dims", "mm.w_q8_0", "mm.x", "mm.dst", "mm.absterm", "fa.q", "fa.k", "fa.v", "fa.out", "fa.wabs"};
    if (!load_fixture(argv[1], &fx)) {
        std::fprintf(stderr, "cannot read fixture %s\n", argv[1]);
        return 4;
    }
    for (const char* n : names)
        if (!fx.count(n)) {
            std::fprintf(stderr, "fixture lacks %s\n", n);
            return 4;
        }
    const std::vector<int32_t> dims = as<int32_t>(fx["dims"]);
    const int64_t M = dims[0], N = dims[1], K = dims[2], D = dims[3], n = dims[4], nh = dims[5];

    // backend init (sam3.cpp:3278-3292): device 0, its default stream
    const mi355_status cst = mi355_context_create(0, nullptr, &g_ctx);
    if (cst != MI355_STATUS_SUCCESS) {
        std::fprintf(stderr, "mi355_context_create: %s (%s)\n", mi355_status_to_string(cst), mi355_last_error(nullptr));
        return 2;
    }

    // tensors in ggml layouts
    const int64_t rowq = (K / 32) * 34;
    mi355_tensor w = tensor(MI355_TYPE_Q8_0, K, N, 1, 1, 34, rowq);
    mi355_tensor x = tensor(MI355_TYPE_F32, K, M, 1, 1, 4, 4 * K);
    mi355_tensor dst = tensor(MI355_TYPE_F32, N, M, 1, 1, 4, 4 * N);
    mi355_tensor q = tensor(MI355_TYPE_F16, D, n, nh, 1, 2, 2 * D);  // [D, n, nh, 1] over [1][nh][n][D]
    mi355_tensor k = q, v = q;
    mi355_tensor o = tensor(MI355_TYPE_F32, D, nh, n, 1, 4, 4 * D);  // [D, nh, n, 1]
    if (mi355_tensor_nbytes(&w) != fx["mm.w_q8_0"].bytes.size() || mi355_tensor_nbytes(&x) != fx["mm.x"].bytes.size() ||
        mi355_tensor_nbytes(&q) != fx["fa.q"].bytes.size() || mi355_tensor_nbytes(&o) != fx["fa.out"].bytes.size()) {
        std::fprintf(stderr, "fixture sizes do not match its dims\n");
        return 4;
    }

    // one weight buffer (the model's), one buffer for the graph's tensors
    const size_t al = mi355_buffer_alignment();
    mi355_buffer* wbuf = nullptr;
    mi355_buffer* gbuf = nullptr;
    CHECK(mi355_buffer_alloc(g_ctx, round_up(mi355_tensor_nbytes(&w), al), &wbuf));
    CHECK(mi355_buffer_place(wbuf, 0, &w));
    mi355_tensor* graph_tensors[] = {&x, &dst, &q, &k, &v, &o};
    size_t off[6], total = 0;
    for (int i = 0; i < 6; ++i) {
        off[i] = total;
        total += round_up(mi355_tensor_nbytes(graph_tensors[i]), al);
    }
    CHECK(mi355_buffer_alloc(g_ctx, total, &gbuf));
    CHECK(mi355_buffer_clear(g_ctx, gbuf, 0));
    for (int i = 0; i < 6; ++i) CHECK(mi355_buffer_place(gbuf, off[i], graph_tensors[i]));

    CHECK(mi355_tensor_set(g_ctx, &w, fx["mm.w_q8_0"].bytes.data(), 0, fx["mm.w_q8_0"].bytes.size()));
    CHECK(mi355_tensor_set(g_ctx, &x, fx["mm.x"].bytes.data(), 0, fx["mm.x"].bytes.size()));
    CHECK(mi355_tensor_set(g_ctx, &q, fx["fa.q"].bytes.data(), 0, fx["fa.q"].bytes.size()));
    CHECK(mi355_tensor_set(g_ctx, &k, fx["fa.k"].bytes.data(), 0, fx["fa.k"].bytes.size()));
    CHECK(mi355_tensor_set(g_ctx, &v, fx["fa.v"].bytes.data(), 0, fx["fa.v"].bytes.size()));

    // every node is checked before the graph runs on this backend
    if (!mi355_supports_mul_mat(&w, &x, &dst) || !mi355_supports_flash_attn_ext(&q, &k, &v, nullptr, 0.0f, 0.0f, &o)) {
        std::fprintf(stderr, "supports query rejected a node\n");
        return 3;
    }
    CHECK(mi355_mul_mat(g_ctx, &w, &x, &dst));
    CHECK(mi355_flash_attn_ext(g_ctx, &q, &k, &v, nullptr, 0.125f, 0.0f, 0.0f, &o));
    CHECK(mi355_synchronize(g_ctx));

    std::vector<float> got_mm(M * N), got_fa(n * nh * D);
    CHECK(mi355_tensor_get(g_ctx, &dst, got_mm.data(), 0, got_mm.size() * 4));
    CHECK(mi355_tensor_get(g_ctx, &o, got_fa.data(), 0, got_fa.size() * 4));
    const std::vector<float> ref_mm = as<float>(fx["mm.dst"]), at = as<float>(fx["mm.absterm"]);
    const std::vector<float> ref_fa = as<float>(fx["fa.out"]), wabs = as<float>(fx["fa.wabs"]);
    double e_mm = 0.0, e_fa = 0.0;
    for (size_t i = 0; i < got_mm.size(); ++i) {
        const double e = std::fabs((double)got_mm[i] - ref_mm[i]) / std::fmax((double)at[i], 1e-30);
        e_mm = std::isnan(e) ? INFINITY : std::fmax(e_mm, e);
    }
    for (size_t i = 0; i < got_fa.size(); ++i) {
        const double e = std::fabs((double)got_fa[i] - ref_fa[i]) / std::fmax((double)wabs[i], 1e-30);
        e_fa = std::isnan(e) ? INFINITY : std::fmax(e_fa, e);
    }

    // ggml_backend_tensor_memset of part of dst, read back
    CHECK(mi355_tensor_memset(g_ctx, &dst, 0xAB, 12, 1000));
    std::vector<uint8_t> raw(mi355_tensor_nbytes(&dst));
    CHECK(mi355_tensor_get(g_ctx, &dst, raw.data(), 0, raw.size()));
    bool mem_ok = true;
    for (size_t i = 0; i < raw.size(); ++i) {
        const uint8_t want = (i >= 12 && i < 1012) ? 0xAB : reinterpret_cast<const uint8_t*>(got_mm.data())[i];
        mem_ok = mem_ok && raw[i] == want;
    }
    // a range past the tensor is refused
    const bool refused = mi355_tensor_set(g_ctx, &x, fx["mm.x"].bytes.data(), 8, fx["mm.x"].bytes.size()) ==
                         MI355_STATUS_INVALID_ARG;

    mi355_buffer_free(gbuf);
    mi355_buffer_free(wbuf);
    mi355_context_free(g_ctx);
    std::printf("capi_check: mul_mat Q8_0 %lldx%lldx%lld max err/absterm %.3e (bar 1e-5); flash_attn_ext "
                "D=%lld n=%lld heads=%lld max err/W %.3e (bar 2e-3); memset %s; out-of-range set %s\n",
                (long long)M, (long long)N, (long long)K, e_mm, (long long)D, (long long)n, (long long)nh, e_fa,
                mem_ok ? "ok" : "WRONG", refused ? "refused" : "NOT REFUSED");
    const bool pass = e_mm <= 1e-5 && e_fa <= 2e-3 && mem_ok && refused;
    std::printf("%s\n", pass ? "capi_check ok" : "capi_check FAILED");
    return pass ? 0 : 1;
}
