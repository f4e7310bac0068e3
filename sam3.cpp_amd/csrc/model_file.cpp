// sam3.cpp's `.ggml` model files on the MI355X backend: the header and
// hyperparameters (sam3_load_model, sam3.cpp:3204-3262; sam3_load_hparams
// 1481-1524; sam2_load_hparams 1568-1630), the tensor records
// (sam3_load_tensors, sam3.cpp:3095-3198: n_dims, name_len, dtype, ggml ne,
// name, padding to a 32-byte file offset, raw bytes), and their upload to
// device memory with the reference's type conversions (same type: copy;
// F16<->F32; quantized -> F32 dequantize), the last two on the GPU.
//
// The index is built once by walking the records; data is read on demand with
// pread into a pinned staging buffer and copied to the device on the
// context's stream.  On top of it, mi355_vit_weights_load uploads a SAM3 ViT
// backbone (sam3_register_tensors' "vit.*" names, sam3.cpp:2530-2560) into
// the block table the encoder entry points take.
#include <fcntl.h>
#include <unistd.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "context.h"

using namespace mi355;

namespace {

constexpr uint32_t kMagicSam3 = 0x73616D33;  // "sam3"
constexpr uint32_t kMagicSam2 = 0x73616D32;  // "sam2"
constexpr int kVersionSam3 = 3, kVersionSam2 = 1;
constexpr int kSam2Hparams = 57;  // int32 fields of sam2_load_hparams (SAM2 / SAM2.1 Hiera)

struct TensorRec {
    std::string name;
    int32_t type = 0, n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint64_t offset = 0, nbytes = 0;
};

}  // namespace

struct mi355_model_file {
    int fd = -1;
    uint32_t magic = 0;
    int32_t version = 0, ftype = 0, n_tensors = 0;
    std::vector<int32_t> hparams;
    std::vector<TensorRec> tensors;
    std::unordered_map<std::string, int> by_name;
    uint64_t size = 0;
};

namespace {

std::string g_file_error;

mi355_status file_fail(mi355_status st, const char* fmt, const std::string& a = "") {
    char buf[512];
    snprintf(buf, sizeof(buf), fmt, a.c_str());
    g_file_error = buf;
    return st;
}

bool read_at(int fd, uint64_t off, void* dst, size_t n) {
    char* p = static_cast<char*>(dst);
    while (n > 0) {
        const ssize_t r = pread(fd, p, n, (off_t)off);
        if (r <= 0) return false;
        p += r;
        off += (uint64_t)r;
        n -= (size_t)r;
    }
    return true;
}

int64_t block_bytes(int type) { return type == T_Q8_0 ? 34 : type == T_Q4_0 ? 18 : type == T_Q4_1 ? 20 : 0; }

// bytes of a tensor record's data as sam3_load_tensors computes them
// (false for an unknown type, a row not made of whole blocks, or an element
// count whose f32 size does not fit in int64: the dequantized copy must fit too)
bool data_bytes(int type, const int64_t ne[4], uint64_t* out) {
    int64_t n = 1, n4 = 0;
    for (int i = 0; i < 4; ++i)
        if (ne[i] <= 0 || __builtin_mul_overflow(n, ne[i], &n)) return false;
    if (__builtin_mul_overflow(n, (int64_t)4, &n4)) return false;
    if (type == T_F32) *out = (uint64_t)n * 4;
    else if (type == T_F16) *out = (uint64_t)n * 2;
    else if (block_bytes(type)) {
        if (ne[0] % 32 != 0) return false;
        *out = (uint64_t)(n / 32) * (uint64_t)block_bytes(type);
    } else
        return false;
    return true;
}

// the header's hyperparameters: SAM3 (sam3_load_hparams field order, the
// global-block list holding min(n, 4) entries) or SAM2 (a fixed list)
bool read_hparams(mi355_model_file* f, uint64_t* pos) {
    auto rd = [&](int32_t* v) {
        if (!read_at(f->fd, *pos, v, 4)) return false;
        *pos += 4;
        f->hparams.push_back(*v);
        return true;
    };
    int32_t v = 0;
    if (f->magic == kMagicSam3) {
        for (int i = 0; i < 8; ++i)  // img_size .. n_global_attn
            if (!rd(&v)) return false;
        const int n_global = std::min(std::max(f->hparams[7], 0), 4);
        for (int i = 0; i < n_global + 27; ++i)  // global indices, text_width .. visual_only
            if (!rd(&v)) return false;
        return true;
    }
    for (int i = 0; i < kSam2Hparams; ++i)
        if (!rd(&v)) return false;
    return true;
}

}  // namespace

extern "C" {

const char* mi355_model_file_last_error(void) { return g_file_error.c_str(); }

mi355_status mi355_model_file_open(const char* path, mi355_model_file** out) {
    if (!path || !out) return file_fail(MI355_STATUS_INVALID_ARG, "model_file_open: null argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return file_fail(MI355_STATUS_FAILED, "model_file_open: cannot open '%s'", path);
    auto* f = new mi355_model_file();
    f->fd = fd;
    f->size = (uint64_t)lseek(fd, 0, SEEK_END);
    auto bad = [&](mi355_status st, const char* msg, const std::string& a = "") {
        mi355_model_file_close(f);
        return file_fail(st, msg, a);
    };
    int32_t hdr[4];
    if (!read_at(fd, 0, hdr, sizeof(hdr))) return bad(MI355_STATUS_FAILED, "model_file_open: short header");
    f->magic = (uint32_t)hdr[0];
    f->version = hdr[1];
    f->ftype = hdr[2];
    f->n_tensors = hdr[3];
    if (f->magic == kMagicSam3) {
        if (f->version != kVersionSam3) return bad(MI355_STATUS_UNSUPPORTED, "model_file_open: unsupported SAM3 version");
    } else if (f->magic == kMagicSam2) {
        if (f->version != kVersionSam2) return bad(MI355_STATUS_UNSUPPORTED, "model_file_open: unsupported SAM2 version");
    } else {
        return bad(MI355_STATUS_INVALID_ARG, "model_file_open: unknown magic");
    }
    if (!(f->ftype == 0 || f->ftype == 1 || f->ftype == 2 || f->ftype == 3 || f->ftype == 8))
        return bad(MI355_STATUS_UNSUPPORTED, "model_file_open: unsupported ftype");
    if (f->n_tensors < 0) return bad(MI355_STATUS_INVALID_ARG, "model_file_open: negative tensor count");
    uint64_t pos = sizeof(hdr);
    if (!read_hparams(f, &pos)) return bad(MI355_STATUS_FAILED, "model_file_open: short hyperparameters");
    if (f->magic == kMagicSam2 && f->hparams[1] != 1)
        return bad(MI355_STATUS_UNSUPPORTED, "model_file_open: only the Hiera backbone (backbone_type 1) is supported");
    f->tensors.reserve((size_t)f->n_tensors);
    for (int t = 0; t < f->n_tensors; ++t) {
        int32_t h3[3];
        if (!read_at(fd, pos, h3, sizeof(h3))) return bad(MI355_STATUS_FAILED, "model_file_open: short tensor record");
        pos += sizeof(h3);
        TensorRec r;
        r.n_dims = h3[0];
        r.type = h3[2];
        if (r.n_dims < 1 || r.n_dims > 4 || h3[1] <= 0 || h3[1] > 4096)
            return bad(MI355_STATUS_INVALID_ARG, "model_file_open: bad tensor record");
        int32_t shape[4];
        if (!read_at(fd, pos, shape, 4 * (size_t)r.n_dims)) return bad(MI355_STATUS_FAILED, "model_file_open: short shape");
        pos += 4 * (uint64_t)r.n_dims;
        for (int i = 0; i < r.n_dims; ++i) {
            if (shape[i] <= 0) return bad(MI355_STATUS_INVALID_ARG, "model_file_open: non-positive dimension");
            r.ne[i] = shape[i];
        }
        r.name.resize((size_t)h3[1]);
        if (!read_at(fd, pos, &r.name[0], r.name.size())) return bad(MI355_STATUS_FAILED, "model_file_open: short name");
        pos += r.name.size();
        pos += (32 - pos % 32) % 32;  // data starts at a 32-byte file offset
        if (!data_bytes(r.type, r.ne, &r.nbytes))
            return bad(MI355_STATUS_UNSUPPORTED, "model_file_open: tensor '%s' has an unsupported type or shape", r.name);
        r.offset = pos;
        if (pos > f->size || r.nbytes > f->size - pos)
            return bad(MI355_STATUS_FAILED, "model_file_open: tensor '%s' runs past the end", r.name);
        pos += r.nbytes;
        if (!f->by_name.emplace(r.name, t).second)
            return bad(MI355_STATUS_INVALID_ARG, "model_file_open: duplicate tensor '%s'", r.name);
        f->tensors.push_back(std::move(r));
    }
    *out = f;
    return MI355_STATUS_SUCCESS;
}

void mi355_model_file_close(mi355_model_file* f) {
    if (!f) return;
    if (f->fd >= 0) close(f->fd);
    delete f;
}

mi355_status mi355_model_file_header(const mi355_model_file* f, uint32_t* magic, int32_t* version, int32_t* ftype,
                                     int32_t* n_tensors) {
    if (!f) return file_fail(MI355_STATUS_INVALID_ARG, "model_file_header: null file");
    if (magic) *magic = f->magic;
    if (version) *version = f->version;
    if (ftype) *ftype = f->ftype;
    if (n_tensors) *n_tensors = f->n_tensors;
    return MI355_STATUS_SUCCESS;
}

int mi355_model_file_hparams(const mi355_model_file* f, const int32_t** values) {
    if (!f) return -1;
    if (values) *values = f->hparams.data();
    return (int)f->hparams.size();
}

int mi355_model_file_find(const mi355_model_file* f, const char* name) {
    if (!f || !name) return -1;
    const auto it = f->by_name.find(name);
    return it == f->by_name.end() ? -1 : it->second;
}

mi355_status mi355_model_file_tensor(const mi355_model_file* f, int index, mi355_model_tensor_info* out) {
    if (!f || !out) return file_fail(MI355_STATUS_INVALID_ARG, "model_file_tensor: null argument");
    if (index < 0 || index >= (int)f->tensors.size())
        return file_fail(MI355_STATUS_INVALID_ARG, "model_file_tensor: index out of range");
    const TensorRec& r = f->tensors[(size_t)index];
    out->name = r.name.c_str();
    out->type = r.type;
    out->n_dims = r.n_dims;
    for (int i = 0; i < 4; ++i) out->ne[i] = r.ne[i];
    out->offset = r.offset;
    out->nbytes = r.nbytes;
    return MI355_STATUS_SUCCESS;
}

size_t mi355_model_file_load_bytes(const mi355_model_file* f, int index, int32_t dst_type) {
    if (!f || index < 0 || index >= (int)f->tensors.size()) return 0;
    const TensorRec& r = f->tensors[(size_t)index];
    if (dst_type == r.type) return (size_t)r.nbytes;
    int64_t n = r.ne[0] * r.ne[1] * r.ne[2] * r.ne[3];
    if (dst_type == T_F32) return (size_t)n * 4;
    if (dst_type == T_F16 && r.type == T_F32) return (size_t)n * 2;
    return 0;
}

mi355_status mi355_model_file_load(mi355_context* ctx, const mi355_model_file* f, int index, int32_t dst_type,
                                   void* dst, size_t dst_bytes) {
    if (!ctx || !f || !dst) return fail(ctx, MI355_STATUS_INVALID_ARG, "model_file_load: null argument");
    if (index < 0 || index >= (int)f->tensors.size())
        return fail(ctx, MI355_STATUS_INVALID_ARG, "model_file_load: index %d out of range", index);
    const TensorRec& r = f->tensors[(size_t)index];
    const size_t need = mi355_model_file_load_bytes(f, index, dst_type);
    if (need == 0)
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "model_file_load: '%s': no conversion from type %d to %d", r.name.c_str(),
                    r.type, dst_type);
    if (dst_bytes < need)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "model_file_load: '%s' needs %zu bytes", r.name.c_str(), need);
    (void)hipSetDevice(ctx->device);
    // raw bytes -> pinned staging -> device (dst itself, or the workspace before a conversion)
    const bool same = dst_type == r.type;
    if (!same) {
        mi355_status st = ensure_buffer(ctx, &ctx->ws, &ctx->ws_size, (size_t)r.nbytes);
        if (st != MI355_STATUS_SUCCESS) return st;
    }
    char* dev = same ? static_cast<char*>(dst) : static_cast<char*>(ctx->ws);
    constexpr size_t kChunk = 16u << 20;
    void* host = nullptr;
    if (hipHostMalloc(&host, std::min<size_t>(kChunk, (size_t)r.nbytes), hipHostMallocDefault) != hipSuccess)
        return fail(ctx, MI355_STATUS_ALLOC_FAILED, "model_file_load: pinned staging allocation failed");
    mi355_status st = MI355_STATUS_SUCCESS;
    for (uint64_t done = 0; done < r.nbytes && st == MI355_STATUS_SUCCESS;) {
        const size_t n = (size_t)std::min<uint64_t>(kChunk, r.nbytes - done);
        if (!read_at(f->fd, r.offset + done, host, n)) {
            st = fail(ctx, MI355_STATUS_FAILED, "model_file_load: read of '%s' failed", r.name.c_str());
            break;
        }
        st = hip_check(ctx, hipMemcpyAsync(dev + done, host, n, hipMemcpyHostToDevice, ctx->stream), "upload");
        if (st == MI355_STATUS_SUCCESS)
            st = hip_check(ctx, hipStreamSynchronize(ctx->stream), "upload");  // the staging buffer is reused
        done += n;
    }
    (void)hipHostFree(host);
    if (st != MI355_STATUS_SUCCESS || same) return st;
    const int64_t n = r.ne[0] * r.ne[1] * r.ne[2] * r.ne[3];
    Timed t(ctx, "convert_weights");
    return hip_check(ctx, t.done(launch_convert_weights(dev, r.type, dst, dst_type, n, ctx->stream)),
                     "convert_weights launch");
}

// ---- backbones from a file, tensors typed as sam3_register_tensors types them

namespace {

// Uploads named tensors of a file into fresh device buffers (kept in allocs):
// shapes must match the registered ones, the type is the registered type.
struct Uploader {
    mi355_context* ctx;
    const mi355_model_file* f;
    std::vector<void*>* allocs;
    const char* what;
    std::vector<void*> raw;  // ggml-layout weights whose prepared forms replace them
    mi355_status load(const std::string& name, int type, std::initializer_list<int64_t> ne, void** dptr,
                      mi355_tensor* t) {
        const int idx = mi355_model_file_find(f, name.c_str());
        if (idx < 0) return fail(ctx, MI355_STATUS_INVALID_ARG, "%s: tensor '%s' missing", what, name.c_str());
        const TensorRec& r = f->tensors[(size_t)idx];
        int64_t want[4] = {1, 1, 1, 1};
        int i = 0;
        for (int64_t v : ne) want[i++] = v;
        for (int k = 0; k < 4; ++k)
            if (r.ne[k] != want[k])
                return fail(ctx, MI355_STATUS_INVALID_ARG, "%s: '%s' has an unexpected shape", what, name.c_str());
        const size_t bytes = mi355_model_file_load_bytes(f, idx, type);
        void* d = nullptr;
        if (bytes == 0 || hipMalloc(&d, bytes) != hipSuccess)
            return fail(ctx, MI355_STATUS_ALLOC_FAILED, "%s: cannot place '%s'", what, name.c_str());
        allocs->push_back(d);
        const mi355_status st = mi355_model_file_load(ctx, f, idx, type, d, bytes);
        if (st != MI355_STATUS_SUCCESS) return st;
        *dptr = d;
        if (t) {
            *t = mi355_tensor{};
            t->type = type;
            for (int k = 0; k < 4; ++k) t->ne[k] = want[k];
            t->nb[0] = type_size(type);
            t->nb[1] = (int64_t)row_size(type, want[0]);
            t->nb[2] = t->nb[1] * want[1];
            t->nb[3] = t->nb[2] * want[2];
            t->data = d;
        }
        return MI355_STATUS_SUCCESS;
    }
    // A 2-D Q8_0 / Q4_0 / Q4_1 weight is replaced by its prepared form
    // (mi355_weight_prepare: the int8 kernel's layout); other tensors stay as loaded.
    mi355_status prepare(mi355_tensor* t) {
        const size_t n = mi355_weight_prepared_nbytes(t);
        if (n == 0) return MI355_STATUS_SUCCESS;
        void* d = nullptr;
        if (hipMalloc(&d, n) != hipSuccess) {
            (void)hipGetLastError();
            return fail(ctx, MI355_STATUS_ALLOC_FAILED, "%s: cannot place a prepared weight (%zu bytes)", what, n);
        }
        allocs->push_back(d);
        mi355_tensor pt;
        const mi355_status st = mi355_weight_prepare(ctx, t, d, n, &pt);
        if (st != MI355_STATUS_SUCCESS) return st;
        raw.push_back(t->data);
        *t = pt;
        return MI355_STATUS_SUCCESS;
    }
    // Waits for the repacks, then frees the ggml-layout copies they read.
    mi355_status finish() {
        const mi355_status st = mi355_synchronize(ctx);
        if (st != MI355_STATUS_SUCCESS) return st;
        for (void* p : raw) {
            for (auto it = allocs->begin(); it != allocs->end(); ++it)
                if (*it == p) {
                    allocs->erase(it);
                    break;
                }
            (void)hipFree(p);
        }
        raw.clear();
        return MI355_STATUS_SUCCESS;
    }
};

// the weight type of a file's ftype (sam3_load_model's map, sam3.cpp:3246-3255)
int weight_type(int32_t ftype) {
    return ftype == 0 ? T_F32 : ftype == 1 ? T_F16 : ftype == 2 ? T_Q4_0 : ftype == 3 ? T_Q4_1 : T_Q8_0;
}

}  // namespace

// ---- SAM3 ViT backbone (sam3_register_tensors, sam3.cpp:2530-2560)

struct mi355_vit_weights {
    mi355_vit_hparams hp{};
    std::vector<mi355_vit_block> blocks;
    mi355_tensor patch_w{};
    float *pos = nullptr, *ln_w = nullptr, *ln_b = nullptr;
    std::vector<void*> allocs;
};

void mi355_vit_weights_free(mi355_vit_weights* w) {
    if (!w) return;
    for (void* p : w->allocs) (void)hipFree(p);
    delete w;
}

mi355_status mi355_vit_weights_load(mi355_context* ctx, const mi355_model_file* f, mi355_vit_weights** out) {
    if (!ctx || !f || !out) return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_weights_load: null argument");
    *out = nullptr;
    if (f->magic != kMagicSam3) return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_weights_load: not a SAM3 file");
    const int32_t* h = f->hparams.data();
    // sam3_load_hparams: img_size, patch_size, embed, depth, heads, mlp ratio x1000, window, n_global, idx...
    const int img = h[0], P = h[1], E = h[2], depth = h[3], NH = h[4], ws = h[6];
    const int n_global = std::min(std::max(h[7], 0), 4);
    if (img <= 0 || P <= 0 || E <= 0 || depth <= 0 || NH <= 0 || img % P != 0 || (img / P) % 3 != 0)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "vit_weights_load: bad hyperparameters");
    auto* w = new mi355_vit_weights();
    w->hp.embed_dim = E;
    w->hp.num_heads = NH;
    w->hp.mlp_dim = (int32_t)(E * (h[5] / 1000.0f));  // as sam3_load_hparams derives vit_mlp_dim
    w->hp.window_size = ws;
    w->hp.grid = img / P;
    w->hp.patch_size = P;
    w->hp.pos_grid = img / P / 3;  // pos_embed at pretrained resolution, tiled 3x
    w->hp.eps = 1e-5f;
    const int wtype = weight_type(f->ftype);
    const int wblk = blck(wtype);
    auto bad = [&](mi355_status st) {
        mi355_vit_weights_free(w);
        return st;
    };
    // weights (T2/T4) in the file's weight type when ne0 is a whole number of blocks, else F32
    Uploader up{ctx, f, &w->allocs, "vit_weights_load"};
    auto load = [&](const std::string& name, int type, std::initializer_list<int64_t> ne, void** dptr,
                    mi355_tensor* t) { return up.load(name, type, ne, dptr, t); };
    auto wt = [&](int64_t ne0) { return ne0 % wblk == 0 ? wtype : (int)T_F32; };
    const int MLP = w->hp.mlp_dim, pg = w->hp.pos_grid, G = w->hp.grid;
    void* p = nullptr;
    mi355_status st;
    if ((st = load("vit.patch_embed.proj.weight", wt(P), {P, P, 3, E}, &p, &w->patch_w)) != MI355_STATUS_SUCCESS) return bad(st);
    if ((st = load("vit.pos_embed", T_F32, {E, pg, pg, 1}, &p, nullptr)) != MI355_STATUS_SUCCESS) return bad(st);
    w->pos = static_cast<float*>(p);
    if ((st = load("vit.ln_pre.weight", T_F32, {E}, &p, nullptr)) != MI355_STATUS_SUCCESS) return bad(st);
    w->ln_w = static_cast<float*>(p);
    if ((st = load("vit.ln_pre.bias", T_F32, {E}, &p, nullptr)) != MI355_STATUS_SUCCESS) return bad(st);
    w->ln_b = static_cast<float*>(p);
    w->blocks.resize((size_t)depth);
    for (int i = 0; i < depth; ++i) {
        mi355_vit_block& b = w->blocks[(size_t)i];
        const std::string pre = "vit.blocks." + std::to_string(i);
        bool global = false;
        for (int g = 0; g < n_global; ++g) global |= h[8 + g] == i;
        const int64_t rope_n = global ? (int64_t)G * G : (int64_t)ws * ws;
        struct V { const char* sfx; int64_t n; const float** dst; } vecs[] = {
            {".norm1.weight", E, &b.norm1_w}, {".norm1.bias", E, &b.norm1_b}, {".attn.qkv.bias", 3LL * E, &b.qkv_b},
            {".attn.proj.bias", E, &b.proj_b}, {".norm2.weight", E, &b.norm2_w}, {".norm2.bias", E, &b.norm2_b},
            {".mlp.lin1.bias", MLP, &b.fc1_b}, {".mlp.lin2.bias", E, &b.fc2_b}};
        for (const V& v : vecs) {
            if ((st = load(pre + v.sfx, T_F32, {v.n}, &p, nullptr)) != MI355_STATUS_SUCCESS) return bad(st);
            *v.dst = static_cast<const float*>(p);
        }
        if ((st = load(pre + ".attn.qkv.weight", wt(E), {E, 3LL * E}, &p, &b.qkv_w)) != MI355_STATUS_SUCCESS) return bad(st);
        if ((st = load(pre + ".attn.proj.weight", wt(E), {E, E}, &p, &b.proj_w)) != MI355_STATUS_SUCCESS) return bad(st);
        if ((st = load(pre + ".mlp.lin1.weight", wt(E), {E, MLP}, &p, &b.fc1_w)) != MI355_STATUS_SUCCESS) return bad(st);
        if ((st = load(pre + ".mlp.lin2.weight", wt(MLP), {MLP, E}, &p, &b.fc2_w)) != MI355_STATUS_SUCCESS) return bad(st);
        if ((st = load(pre + ".attn.freqs_cis", T_F32, {2, E / NH / 2, rope_n}, &p, nullptr)) != MI355_STATUS_SUCCESS)
            return bad(st);
        b.freqs_cis = static_cast<const float*>(p);
        b.is_global = global ? 1 : 0;
        for (mi355_tensor* t : {&b.qkv_w, &b.proj_w, &b.fc1_w, &b.fc2_w})
            if ((st = up.prepare(t)) != MI355_STATUS_SUCCESS) return bad(st);
    }
    if ((st = up.finish()) != MI355_STATUS_SUCCESS) return bad(st);
    *out = w;
    return MI355_STATUS_SUCCESS;
}

// ---- SAM2 Hiera backbone (sam3_register_tensors' "hiera.*" names, sam3.cpp:1800-1840;
// hyperparameters of sam2_load_hparams, sam3.cpp:1568-1590)

struct mi355_hiera_weights {
    mi355_hiera_hparams hp{};
    std::vector<mi355_hiera_block> blocks;
    mi355_tensor patch_w{};
    float *patch_b = nullptr, *pos = nullptr;
    std::vector<void*> allocs;
};

void mi355_hiera_weights_free(mi355_hiera_weights* w) {
    if (!w) return;
    for (void* p : w->allocs) (void)hipFree(p);
    delete w;
}

mi355_status mi355_hiera_weights_load(mi355_context* ctx, const mi355_model_file* f, mi355_hiera_weights** out) {
    if (!ctx || !f || !out) return fail(ctx, MI355_STATUS_INVALID_ARG, "hiera_weights_load: null argument");
    *out = nullptr;
    if (f->magic != kMagicSam2 || f->hparams.size() < 25)
        return fail(ctx, MI355_STATUS_INVALID_ARG, "hiera_weights_load: not a SAM2 file");
    // img_size, backbone_type, embed, heads, num_stages, stages[4], global_n, global_idx[8],
    // q_pool, window_spec[4], pos_embed_bkg_h, pos_embed_bkg_w
    const int32_t* h = f->hparams.data();
    auto* w = new mi355_hiera_weights();
    auto bad = [&](mi355_status st) {
        mi355_hiera_weights_free(w);
        return st;
    };
    mi355_hiera_hparams& hp = w->hp;
    hp.img_size = h[0];
    hp.embed_dim = h[2];
    hp.num_heads = h[3];
    for (int i = 0; i < 4; ++i) hp.stages[i] = h[5 + i];
    hp.n_global = h[9];
    for (int i = 0; i < 8; ++i) hp.global_idx[i] = h[10 + i];
    hp.q_pool = h[18];
    for (int i = 0; i < 4; ++i) hp.window_spec[i] = h[19 + i];
    hp.eps = 1e-6f;
    const int bkg_h = h[23], bkg_w = h[24], E = hp.embed_dim;
    const int n = mi355_hiera_n_blocks(&hp);
    if (h[4] != 4 || n <= 0 || hp.n_global < 0 || hp.n_global > 8 || bkg_h <= 0 || bkg_w <= 0 || hp.img_size % 4 != 0)
        return bad(fail(ctx, MI355_STATUS_INVALID_ARG, "hiera_weights_load: bad hyperparameters"));
    const int wtype = weight_type(f->ftype), wblk = blck(wtype);
    auto wt = [&](int64_t ne0) { return ne0 % wblk == 0 ? wtype : (int)T_F32; };
    Uploader up{ctx, f, &w->allocs, "hiera_weights_load"};
    void* p = nullptr;
    mi355_status st;
    if ((st = up.load("hiera.patch_embed.weight", wt(7), {7, 7, 3, E}, &p, &w->patch_w)) != MI355_STATUS_SUCCESS)
        return bad(st);
    if ((st = up.load("hiera.patch_embed.bias", T_F32, {E}, &p, nullptr)) != MI355_STATUS_SUCCESS) return bad(st);
    w->patch_b = static_cast<float*>(p);
    // the positional table of the encoder's grid, built on the device from the two tables
    // (sam2_compute_pos_embed, sam3.cpp:4118-4157)
    const int ws0 = hp.window_spec[0], S0 = hp.img_size / 4;
    void *bkg = nullptr, *win = nullptr;
    if ((st = up.load("hiera.pos_embed", T_F32, {bkg_w, bkg_h, E, 1}, &bkg, nullptr)) != MI355_STATUS_SUCCESS)
        return bad(st);
    if ((st = up.load("hiera.pos_embed_window", T_F32, {ws0, ws0, E, 1}, &win, nullptr)) != MI355_STATUS_SUCCESS)
        return bad(st);
    if (hipMalloc(&p, (size_t)S0 * S0 * E * 4) != hipSuccess)
        return bad(fail(ctx, MI355_STATUS_ALLOC_FAILED, "hiera_weights_load: pos_embed allocation failed"));
    w->allocs.push_back(p);
    w->pos = static_cast<float*>(p);
    if ((st = mi355_hiera_pos_embed(ctx, static_cast<const float*>(bkg), E, bkg_h, bkg_w, static_cast<const float*>(win),
                                    ws0, S0, S0, w->pos)) != MI355_STATUS_SUCCESS)
        return bad(st);
    w->blocks.resize((size_t)n);
    for (int i = 0; i < n; ++i) {
        mi355_hiera_block_info info;
        if ((st = mi355_hiera_block_info_get(&hp, i, &info)) != MI355_STATUS_SUCCESS) return bad(st);
        const int din = info.dim_in, dout = info.dim_out;
        mi355_hiera_block& b = w->blocks[(size_t)i];
        b = mi355_hiera_block{};
        const std::string pre = "hiera.blocks." + std::to_string(i);
        struct V { const char* sfx; int64_t n; const float** dst; } vecs[] = {
            {".norm1.weight", din, &b.norm1_w}, {".norm1.bias", din, &b.norm1_b}, {".attn.qkv.bias", 3LL * dout, &b.qkv_b},
            {".attn.proj.bias", dout, &b.proj_b}, {".norm2.weight", dout, &b.norm2_w}, {".norm2.bias", dout, &b.norm2_b},
            {".mlp.fc1.bias", 4LL * dout, &b.fc1_b}, {".mlp.fc2.bias", dout, &b.fc2_b}};
        for (const V& v : vecs) {
            if ((st = up.load(pre + v.sfx, T_F32, {v.n}, &p, nullptr)) != MI355_STATUS_SUCCESS) return bad(st);
            *v.dst = static_cast<const float*>(p);
        }
        if ((st = up.load(pre + ".attn.qkv.weight", wt(din), {din, 3LL * dout}, &p, &b.qkv_w)) != MI355_STATUS_SUCCESS ||
            (st = up.load(pre + ".attn.proj.weight", wt(dout), {dout, dout}, &p, &b.proj_w)) != MI355_STATUS_SUCCESS ||
            (st = up.load(pre + ".mlp.fc1.weight", wt(dout), {dout, 4LL * dout}, &p, &b.fc1_w)) != MI355_STATUS_SUCCESS ||
            (st = up.load(pre + ".mlp.fc2.weight", wt(4LL * dout), {4LL * dout, dout}, &p, &b.fc2_w)) != MI355_STATUS_SUCCESS)
            return bad(st);
        if (din != dout) {  // dimension projection at a stage transition
            if ((st = up.load(pre + ".proj.weight", wt(din), {din, dout}, &p, &b.dim_proj_w)) != MI355_STATUS_SUCCESS)
                return bad(st);
            if ((st = up.load(pre + ".proj.bias", T_F32, {dout}, &p, nullptr)) != MI355_STATUS_SUCCESS) return bad(st);
            b.dim_proj_b = static_cast<const float*>(p);
        }
        for (mi355_tensor* t : {&b.qkv_w, &b.proj_w, &b.fc1_w, &b.fc2_w, &b.dim_proj_w})
            if (t->data && (st = up.prepare(t)) != MI355_STATUS_SUCCESS) return bad(st);
    }
    if ((st = up.finish()) != MI355_STATUS_SUCCESS) return bad(st);
    *out = w;
    return MI355_STATUS_SUCCESS;
}

mi355_status mi355_hiera_weights_get(const mi355_hiera_weights* w, mi355_hiera_hparams* hp,
                                     const mi355_hiera_block** blocks, int* n_blocks, const mi355_tensor** patch_w,
                                     const float** patch_b, const float** pos_embed) {
    if (!w) return fail(nullptr, MI355_STATUS_INVALID_ARG, "hiera_weights_get: null weights");
    if (hp) *hp = w->hp;
    if (blocks) *blocks = w->blocks.data();
    if (n_blocks) *n_blocks = (int)w->blocks.size();
    if (patch_w) *patch_w = &w->patch_w;
    if (patch_b) *patch_b = w->patch_b;
    if (pos_embed) *pos_embed = w->pos;
    return MI355_STATUS_SUCCESS;
}

}  // extern "C"

// ---- sam3_quantize_model (examples/quantize.cpp:20-331) with the GPU quantizer

namespace {

// Tensors the reference keeps unquantized by name: the embeddings, lookup
// tables, positional encodings and special tokens that sam3_register_tensors
// registers as F32 (quantize.cpp:195-216).
const char* const kKeepByName[] = {
    "token_embed", "pos_embed", "query_embed", "label_embed", "cls_embed", "point_embeddings", "not_a_point_embed",
    "no_mask_embed", "no_mem_embed", "no_obj_embed", "presence_token.weight", "iou_token", "mask_tokens",
    "obj_score_token", "pe_gaussian", "freqs_cis", "gamma", "tpos_enc", "no_obj_ptr", "no_mem_pos_enc",
    "trk_mask_ds", "latents"};

bool keep_by_name(const std::string& name) {
    for (const char* k : kKeepByName)
        if (name.find(k) != std::string::npos) return true;
    return false;
}

struct OutFile {
    int fd = -1;
    uint64_t pos = 0;
    bool write(const void* p, size_t n) {
        const char* c = static_cast<const char*>(p);
        while (n > 0) {
            const ssize_t w = ::write(fd, c, n);
            if (w <= 0) return false;
            c += w;
            n -= (size_t)w;
            pos += (uint64_t)w;
        }
        return true;
    }
};

// pinned host staging, freed on scope exit
struct Pinned {
    void* p = nullptr;
    ~Pinned() {
        if (p) (void)hipHostFree(p);
    }
};

}  // namespace

extern "C" {

mi355_status mi355_model_quantize(mi355_context* ctx, const char* in_path, const char* out_path, int32_t qtype,
                                  mi355_quantize_stats* stats) {
    if (!ctx || !in_path || !out_path) return fail(ctx, MI355_STATUS_INVALID_ARG, "model_quantize: null argument");
    if (!(qtype == T_Q4_0 || qtype == T_Q4_1 || qtype == T_Q8_0))
        return fail(ctx, MI355_STATUS_UNSUPPORTED, "model_quantize: type %d is not q4_0, q4_1 or q8_0", qtype);
    (void)hipSetDevice(ctx->device);
    const int in = open(in_path, O_RDONLY);
    if (in < 0) return fail(ctx, MI355_STATUS_FAILED, "model_quantize: cannot open '%s' for reading", in_path);
    OutFile out;
    out.fd = open(out_path, O_WRONLY | O_CREAT | O_TRUNC, 0644);
    if (out.fd < 0) {
        close(in);
        return fail(ctx, MI355_STATUS_FAILED, "model_quantize: cannot open '%s' for writing", out_path);
    }
    const uint64_t in_size = (uint64_t)lseek(in, 0, SEEK_END);
    uint64_t pos = 0;
    mi355_quantize_stats acc{};
    Pinned hin, hout;
    size_t hin_cap = 0, hout_cap = 0;
    auto finish = [&](mi355_status st) {
        close(in);
        close(out.fd);
        if (st != MI355_STATUS_SUCCESS) unlink(out_path);  // no half-written model
        else if (stats) *stats = acc;
        return st;
    };
    auto rd = [&](void* dst, size_t n) {
        if (!read_at(in, pos, dst, n)) return false;
        pos += n;
        return true;
    };
    auto pinned = [&](Pinned& b, size_t& cap, size_t n) {
        if (cap >= n) return true;
        if (b.p) (void)hipHostFree(b.p);
        b.p = nullptr;
        cap = 0;
        if (hipHostMalloc(&b.p, n, hipHostMallocDefault) != hipSuccess) return false;
        cap = n;
        return true;
    };
    // copy n bytes from the input's current position through the staging buffer
    auto copy_through = [&](uint64_t n) -> mi355_status {
        constexpr size_t kChunk = 16u << 20;
        if (n > 0 && !pinned(hin, hin_cap, (size_t)std::min<uint64_t>(n, kChunk)))
            return fail(ctx, MI355_STATUS_ALLOC_FAILED, "model_quantize: staging allocation failed");
        while (n > 0) {
            const size_t c = (size_t)std::min<uint64_t>(n, hin_cap);
            if (!rd(hin.p, c)) return fail(ctx, MI355_STATUS_FAILED, "model_quantize: '%s' is truncated", in_path);
            if (!out.write(hin.p, c)) return fail(ctx, MI355_STATUS_FAILED, "model_quantize: write to '%s' failed", out_path);
            n -= c;
        }
        return MI355_STATUS_SUCCESS;
    };

    // header: magic, version, ftype (replaced by qtype), tensor count
    int32_t hdr[4];
    if (!rd(hdr, sizeof(hdr))) return finish(fail(ctx, MI355_STATUS_FAILED, "model_quantize: short header"));
    const uint32_t magic = (uint32_t)hdr[0];
    if (magic == kMagicSam3) {
        if (hdr[1] != kVersionSam3)
            return finish(fail(ctx, MI355_STATUS_UNSUPPORTED, "model_quantize: unsupported SAM3 version %d", hdr[1]));
    } else if (magic == kMagicSam2) {
        if (hdr[1] != kVersionSam2)
            return finish(fail(ctx, MI355_STATUS_UNSUPPORTED, "model_quantize: unsupported SAM2 version %d", hdr[1]));
    } else {
        return finish(fail(ctx, MI355_STATUS_INVALID_ARG, "model_quantize: unknown magic 0x%08x", magic));
    }
    const int32_t n_tensors = hdr[3];
    if (n_tensors < 0) return finish(fail(ctx, MI355_STATUS_INVALID_ARG, "model_quantize: negative tensor count"));
    hdr[2] = qtype;
    if (!out.write(hdr, sizeof(hdr))) return finish(fail(ctx, MI355_STATUS_FAILED, "model_quantize: write failed"));

    // hyperparameters, copied through: SAM3 8 + min(n_global, 4) + 27 fields;
    // SAM2 57, plus 19 for the EdgeTAM (RepViT, backbone_type 2) extension
    {
        int32_t h[8];
        const size_t first = magic == kMagicSam3 ? 8 : 2;
        if (!rd(h, first * 4)) return finish(fail(ctx, MI355_STATUS_FAILED, "model_quantize: short hyperparameters"));
        if (!out.write(h, first * 4)) return finish(fail(ctx, MI355_STATUS_FAILED, "model_quantize: write failed"));
        const uint64_t rest = magic == kMagicSam3 ? (uint64_t)std::min(std::max(h[7], 0), 4) + 27
                                                  : 55 + (h[1] == 2 ? 19 : 0);
        const mi355_status st = copy_through(rest * 4);
        if (st != MI355_STATUS_SUCCESS) return finish(st);
    }

    for (int t = 0; t < n_tensors; ++t) {
        int32_t h3[3];
        if (!rd(h3, sizeof(h3))) return finish(fail(ctx, MI355_STATUS_FAILED, "model_quantize: '%s' is truncated", in_path));
        const int32_t n_dims = h3[0], name_len = h3[1], dtype = h3[2];
        if (n_dims < 1 || n_dims > 4 || name_len <= 0 || name_len > 4096)
            return finish(fail(ctx, MI355_STATUS_INVALID_ARG, "model_quantize: bad tensor record %d", t));
        int32_t ne[4] = {1, 1, 1, 1};
        std::string name((size_t)name_len, '\0');
        if (!rd(ne, 4 * (size_t)n_dims) || !rd(&name[0], name.size()))
            return finish(fail(ctx, MI355_STATUS_FAILED, "model_quantize: '%s' is truncated", in_path));
        pos += (32 - pos % 32) % 32;
        int64_t ne64[4];
        for (int i = 0; i < 4; ++i) {
            if (ne[i] <= 0)
                return finish(fail(ctx, MI355_STATUS_INVALID_ARG, "model_quantize: '%s' has a non-positive dimension",
                                   name.c_str()));
            ne64[i] = ne[i];
        }
        uint64_t in_bytes = 0;
        if (!data_bytes(dtype, ne64, &in_bytes))
            return finish(fail(ctx, MI355_STATUS_UNSUPPORTED, "model_quantize: '%s' has type %d or too many elements",
                               name.c_str(), dtype));
        if (pos > in_size || in_bytes > in_size - pos)
            return finish(fail(ctx, MI355_STATUS_FAILED, "model_quantize: '%s' is truncated", in_path));
        const int64_t n_el = ne64[0] * ne64[1] * ne64[2] * ne64[3];  // data_bytes checked 4 * n_el fits
        const bool quantize = n_dims >= 2 && ne[0] % 32 == 0 && (dtype == T_F32 || dtype == T_F16) && !keep_by_name(name);
        const int32_t dtype_out = quantize ? qtype : dtype;
        // record header with the output type, padded to a 32-byte offset of the output
        std::string rec;
        const int32_t h3o[3] = {n_dims, name_len, dtype_out};
        rec.append(reinterpret_cast<const char*>(h3o), sizeof(h3o));
        rec.append(reinterpret_cast<const char*>(ne), 4 * (size_t)n_dims);
        rec.append(name);
        rec.append((32 - (out.pos + rec.size()) % 32) % 32, '\0');
        if (!out.write(rec.data(), rec.size())) return finish(fail(ctx, MI355_STATUS_FAILED, "model_quantize: write failed"));
        uint64_t out_bytes = in_bytes;
        if (!quantize) {
            const mi355_status st = copy_through(in_bytes);
            if (st != MI355_STATUS_SUCCESS) return finish(st);
        } else {
            // whole rows per chunk: file -> pinned -> device -> quantize -> pinned -> file
            const int64_t rows = n_el / ne[0];
            const size_t in_row = (size_t)ne[0] * (dtype == T_F32 ? 4 : 2);
            const size_t out_row = row_size(qtype, ne[0]);
            const int64_t chunk_rows = std::max<int64_t>(1, (int64_t)((32u << 20) / in_row));
            const int64_t cr = std::min(rows, chunk_rows);
            const size_t in_dev = (size_t)cr * in_row, dev_off = (in_dev + 255) & ~(size_t)255;
            mi355_status st = ensure_buffer(ctx, &ctx->ws, &ctx->ws_size, dev_off + (size_t)cr * out_row);
            if (st != MI355_STATUS_SUCCESS) return finish(st);
            if (!pinned(hin, hin_cap, in_dev) || !pinned(hout, hout_cap, (size_t)cr * out_row))
                return finish(fail(ctx, MI355_STATUS_ALLOC_FAILED, "model_quantize: staging allocation failed"));
            char* dsrc = static_cast<char*>(ctx->ws);
            char* ddst = dsrc + dev_off;
            for (int64_t r0 = 0; r0 < rows; r0 += cr) {
                const int64_t nr = std::min(cr, rows - r0);
                if (!rd(hin.p, (size_t)nr * in_row))
                    return finish(fail(ctx, MI355_STATUS_FAILED, "model_quantize: '%s' is truncated", in_path));
                st = hip_check(ctx, hipMemcpyAsync(dsrc, hin.p, (size_t)nr * in_row, hipMemcpyHostToDevice, ctx->stream),
                               "upload");
                mi355_tensor src{};
                src.type = dtype;
                src.ne[0] = ne[0];
                src.ne[1] = nr;
                src.ne[2] = src.ne[3] = 1;
                src.nb[0] = dtype == T_F32 ? 4 : 2;
                src.nb[1] = (int64_t)in_row;
                src.nb[2] = src.nb[3] = (int64_t)in_row * nr;
                src.data = dsrc;
                if (st == MI355_STATUS_SUCCESS) st = mi355_quantize_weights(ctx, qtype, &src, ddst);
                if (st == MI355_STATUS_SUCCESS)
                    st = hip_check(ctx, hipMemcpyAsync(hout.p, ddst, (size_t)nr * out_row, hipMemcpyDeviceToHost,
                                                       ctx->stream),
                                   "download");
                if (st == MI355_STATUS_SUCCESS) st = hip_check(ctx, hipStreamSynchronize(ctx->stream), "quantize");
                if (st != MI355_STATUS_SUCCESS) return finish(st);
                if (!out.write(hout.p, (size_t)nr * out_row))
                    return finish(fail(ctx, MI355_STATUS_FAILED, "model_quantize: write to '%s' failed", out_path));
            }
            out_bytes = (uint64_t)rows * out_row;
            ++acc.n_quantized;
        }
        acc.size_new += (int64_t)out_bytes;
        acc.size_org += n_el * 4;
        ++acc.n_total;
    }
    // whatever follows the last tensor (the embedded tokenizer) is copied verbatim
    if (pos > in_size) return finish(fail(ctx, MI355_STATUS_FAILED, "model_quantize: '%s' is truncated", in_path));
    return finish(copy_through(in_size - pos));
}

mi355_status mi355_vit_weights_get(const mi355_vit_weights* w, mi355_vit_hparams* hp, const mi355_vit_block** blocks,
                                   int* n_blocks, const mi355_tensor** patch_w, const float** pos_embed,
                                   const float** ln_pre_w, const float** ln_pre_b) {
    if (!w) return fail(nullptr, MI355_STATUS_INVALID_ARG, "vit_weights_get: null weights");
    if (hp) *hp = w->hp;
    if (blocks) *blocks = w->blocks.data();
    if (n_blocks) *n_blocks = (int)w->blocks.size();
    if (patch_w) *patch_w = &w->patch_w;
    if (pos_embed) *pos_embed = w->pos;
    if (ln_pre_w) *ln_pre_w = w->ln_w;
    if (ln_pre_b) *ln_pre_b = w->ln_b;
    return MI355_STATUS_SUCCESS;
}

}  // extern "C"
