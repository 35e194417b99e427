// kore_gguf.cpp - the C ABI of include/kore_gguf.h: kore's GGUF parse
// (load_model, kore.cpp:188-285) over a read-only mapping, and the copies of
// its tensors into HBM.
#include "kore_gguf.h"

#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

struct kore_gguf {
    const uint8_t *map = nullptr;
    size_t size = 0;
    kore_gguf_hparams hp{};
    std::vector<std::string> names;                 // first appearances, file order
    std::vector<kore_gguf_tensor> tensors;          // same order; name points into names
    std::unordered_map<std::string, size_t> index;
    std::string error;
};

namespace {

thread_local std::string g_error;

int fail(kore_gguf *g, int code, const std::string &msg) {
    (g ? g->error : g_error) = msg;
    return code;
}

// GGUF metadata value types (gguf_type; kore.cpp:59-62).
enum : uint32_t { kU8, kI8, kU16, kI16, kU32, kI32, kF32, kBool, kStr, kArr, kU64, kI64, kF64 };

uint64_t scalar_bytes(uint32_t t) {
    switch (t) {
        case kU8: case kI8: case kBool: return 1;
        case kU16: case kI16: return 2;
        case kU32: case kI32: case kF32: return 4;
        case kU64: case kI64: case kF64: return 8;
        default: return 0;
    }
}

// Values per block and bytes per block of the ggml types kore knows
// (kore.cpp:141-158); false for any other.
bool block_shape(uint32_t type, uint64_t *per, uint64_t *bytes) {
    static const struct { uint32_t t; uint64_t per, bytes; } kTable[] = {
        {0, 1, 4}, {1, 1, 2}, {2, 32, 18}, {3, 32, 20}, {6, 32, 22}, {7, 32, 24}, {8, 32, 34}, {10, 256, 84},
        {11, 256, 110}, {12, 256, 144}, {13, 256, 176}, {14, 256, 210}, {15, 256, 292}, {30, 1, 2}};
    for (const auto &e : kTable)
        if (e.t == type) {
            *per = e.per;
            *bytes = e.bytes;
            return true;
        }
    return false;
}

// Bounds-checked reads over the mapping; the first failure sticks (kore's
// Reader, kore.cpp:46-100) and names where it happened.
struct Cursor {
    const uint8_t *base;
    size_t size, pos = 0;
    std::string why;

    bool ok() const { return why.empty(); }
    bool take(void *dst, size_t n) {
        if (!ok()) return false;
        if (n > size - pos) {
            why = "read past the end at offset " + std::to_string(pos);
            return false;
        }
        memcpy(dst, base + pos, n);
        pos += n;
        return true;
    }
    uint32_t u32() { uint32_t v = 0; take(&v, 4); return v; }
    uint64_t u64() { uint64_t v = 0; take(&v, 8); return v; }
    float f32() { float v = 0; take(&v, 4); return v; }
    void skip(uint64_t n) {
        if (!ok()) return;
        if (n > size - pos) { why = "skip past the end at offset " + std::to_string(pos); return; }
        pos += (size_t)n;
    }
    // length-prefixed string (not NUL-terminated in the file)
    std::string str() {
        const uint64_t n = u64();
        if (!ok()) return {};
        if (n > size - pos) { why = "a string of " + std::to_string(n) + " bytes leaves the file"; return {}; }
        std::string s((const char *)base + pos, (size_t)n);
        pos += (size_t)n;
        return s;
    }
    void skip_value(uint32_t t) {
        if (t == kStr) { (void)str(); return; }
        if (t == kArr) {
            const uint32_t et = u32();
            const uint64_t n = u64();
            if (!ok()) return;
            if (et == kStr) {
                for (uint64_t i = 0; i < n && ok(); ++i) (void)str();
            } else if (scalar_bytes(et) && n <= (size - pos) / scalar_bytes(et)) {
                skip(n * scalar_bytes(et));
            } else {
                why = "an array of element type " + std::to_string(et) + " and length " + std::to_string(n);
            }
            return;
        }
        if (scalar_bytes(t)) { skip(scalar_bytes(t)); return; }
        why = "unknown metadata type " + std::to_string(t);
    }
};

int parse(kore_gguf *g) {
    Cursor c{g->map, g->size, 0, {}};
    char magic[4] = {0, 0, 0, 0};
    c.take(magic, 4);
    if (!c.ok() || memcmp(magic, "GGUF", 4) != 0) return fail(g, KORE_GGUF_E_FORMAT, "not a GGUF file");
    kore_gguf_hparams &hp = g->hp;
    hp.version = c.u32();                        // versions other than 2 and 3 are read all the same (kore warns)
    const uint64_t n_tensors = c.u64(), n_kv = c.u64();
    hp.alignment = 32;
    hp.file_size = g->size;

    // metadata: the keys kore uses, with kore's type requirements; the rest skipped
    for (uint64_t i = 0; i < n_kv && c.ok(); ++i) {
        const std::string key = c.str();
        const uint32_t t = c.u32();
        if (!c.ok()) break;
        struct U32Key { const char *key; uint32_t *dst; };
        const U32Key u32keys[] = {{"qwen2.block_count", &hp.n_layer}, {"qwen2.embedding_length", &hp.n_embd},
                                  {"qwen2.feed_forward_length", &hp.n_ff}, {"qwen2.attention.head_count", &hp.n_head},
                                  {"qwen2.attention.head_count_kv", &hp.n_head_kv},
                                  {"qwen2.context_length", &hp.n_ctx}};
        bool used = false;
        if (key == "general.alignment" && t == kU32) {
            const uint32_t a = c.u32();
            if (a) hp.alignment = a;
            used = true;
        }
        for (const U32Key &k : u32keys)
            if (!used && key == k.key && t == kU32) { *k.dst = c.u32(); used = true; }
        if (!used && key == "qwen2.rope.freq_base" && t == kF32) { hp.rope_base = c.f32(); used = true; }
        if (!used && key == "qwen2.attention.layer_norm_rms_epsilon" && t == kF32) { hp.rms_eps = c.f32(); used = true; }
        if (!used && key == "tokenizer.ggml.tokens" && t == kArr && c.size - c.pos >= 12) {
            uint64_t n = 0;                          // the element count follows the element type
            memcpy(&n, c.base + c.pos + 4, 8);
            hp.n_vocab = (uint32_t)n;
            c.skip_value(t);
            used = true;
        }
        if (!used) c.skip_value(t);
    }

    // tensor table: name, n_dims, dims, type, offset from the data start
    struct Entry { std::string name; kore_gguf_tensor t; uint64_t offset; };
    std::vector<Entry> entries;
    for (uint64_t i = 0; i < n_tensors && c.ok(); ++i) {
        Entry e{};
        e.name = c.str();
        e.t.n_dims = c.u32();
        if (!c.ok()) break;
        if (e.t.n_dims == 0 || e.t.n_dims > 4)
            return fail(g, KORE_GGUF_E_FORMAT, "tensor with " + std::to_string(e.t.n_dims) + " dimensions");
        for (int d = 0; d < 4; ++d) e.t.dims[d] = 1;
        uint64_t nelem = 1;
        for (uint32_t d = 0; d < e.t.n_dims; ++d) nelem *= (e.t.dims[d] = c.u64());
        e.t.type = c.u32();
        e.offset = c.u64();
        if (!c.ok()) break;
        uint64_t per = 0, bytes = 0;
        if (block_shape(e.t.type, &per, &bytes) && nelem % per == 0) e.t.nbytes = nelem / per * bytes;
        entries.push_back(std::move(e));
    }
    if (!c.ok()) return fail(g, KORE_GGUF_E_FORMAT, c.why);

    hp.data_start = (c.pos + hp.alignment - 1) / hp.alignment * hp.alignment;
    if (hp.data_start > g->size) return fail(g, KORE_GGUF_E_FORMAT, "file truncated before the tensor data");
    const uint64_t avail = g->size - hp.data_start;
    for (Entry &e : entries) {
        if (e.t.nbytes) {
            if (e.offset > avail || e.t.nbytes > avail - e.offset)
                return fail(g, KORE_GGUF_E_FORMAT, "tensor " + e.name + " leaves the file");
            e.t.data = g->map + hp.data_start + e.offset;
        }
        if (g->index.count(e.name)) continue;      // the first of a repeated name is kept
        g->index.emplace(e.name, g->tensors.size());
        g->names.push_back(e.name);
        g->tensors.push_back(e.t);
    }
    for (size_t i = 0; i < g->tensors.size(); ++i) g->tensors[i].name = g->names[i].c_str();
    return KORE_GGUF_OK;
}

}  // namespace

extern "C" {

KORE_GGUF_API int kore_gguf_open(const char *path, kore_gguf_t *out) {
    if (!out || !path) return fail(nullptr, KORE_GGUF_E_IO, "path or out is NULL");
    *out = nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(nullptr, KORE_GGUF_E_IO, std::string("open ") + path + ": " + strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return fail(nullptr, KORE_GGUF_E_IO, std::string("fstat: ") + strerror(errno));
    }
    const size_t size = (size_t)st.st_size;
    void *map = size ? mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0) : nullptr;
    close(fd);
    if (size && map == MAP_FAILED) return fail(nullptr, KORE_GGUF_E_IO, std::string("mmap: ") + strerror(errno));
    kore_gguf *g = new (std::nothrow) kore_gguf;
    if (!g) {
        if (map) munmap(map, size);
        return fail(nullptr, KORE_GGUF_E_IO, "out of host memory");
    }
    g->map = (const uint8_t *)map;
    g->size = size;
    const int rc = parse(g);
    if (rc != KORE_GGUF_OK) {
        g_error = g->error;
        kore_gguf_close(g);
        return rc;
    }
    *out = g;
    return KORE_GGUF_OK;
}

KORE_GGUF_API void kore_gguf_close(kore_gguf_t g) {
    if (!g) return;
    if (g->map) munmap((void *)g->map, g->size);
    delete g;
}

KORE_GGUF_API int kore_gguf_get_hparams(kore_gguf_t g, kore_gguf_hparams *hp) {
    if (!g || !hp) return fail(g, KORE_GGUF_E_IO, "handle or hp is NULL");
    *hp = g->hp;
    return KORE_GGUF_OK;
}

KORE_GGUF_API int64_t kore_gguf_tensor_count(kore_gguf_t g) { return g ? (int64_t)g->tensors.size() : -1; }

KORE_GGUF_API int kore_gguf_tensor_at(kore_gguf_t g, int64_t i, kore_gguf_tensor *t) {
    if (!g || !t) return fail(g, KORE_GGUF_E_IO, "handle or t is NULL");
    if (i < 0 || i >= (int64_t)g->tensors.size()) return fail(g, KORE_GGUF_E_NOT_FOUND, "tensor index out of range");
    *t = g->tensors[(size_t)i];
    return KORE_GGUF_OK;
}

KORE_GGUF_API int kore_gguf_find(kore_gguf_t g, const char *name, kore_gguf_tensor *t) {
    if (!g || !name || !t) return fail(g, KORE_GGUF_E_IO, "handle, name or t is NULL");
    const auto it = g->index.find(name);
    if (it == g->index.end()) return fail(g, KORE_GGUF_E_NOT_FOUND, std::string("no tensor ") + name);
    *t = g->tensors[it->second];
    return KORE_GGUF_OK;
}

KORE_GGUF_API int kore_gguf_to_qmv(kore_gguf_t g, const char *name, kore_qmv_tensor_t *out) {
    kore_gguf_tensor t{};
    if (int rc = kore_gguf_find(g, name, &t)) return rc;
    if (!out) return fail(g, KORE_GGUF_E_IO, "out is NULL");
    if ((t.type != KORE_QMV_Q4_K && t.type != KORE_QMV_Q6_K) || !t.data)
        return fail(g, KORE_GGUF_E_TYPE, std::string(name) + " is not Q4_K or Q6_K");
    const int64_t rows = (int64_t)(t.dims[1] * t.dims[2] * t.dims[3]), cols = (int64_t)t.dims[0];
    if (kore_qmv_tensor_create(out, (int)t.type, rows, cols, t.data, 0) != KORE_QMV_OK)
        return fail(g, KORE_GGUF_E_DEVICE, std::string(name) + ": " + kore_qmv_last_error(nullptr));
    return KORE_GGUF_OK;
}

KORE_GGUF_API int kore_gguf_to_device_f32(kore_gguf_t g, const char *name, float **dev) {
    kore_gguf_tensor t{};
    if (int rc = kore_gguf_find(g, name, &t)) return rc;
    if (!dev) return fail(g, KORE_GGUF_E_IO, "dev is NULL");
    *dev = nullptr;
    if (t.type != 0 || !t.data) return fail(g, KORE_GGUF_E_TYPE, std::string(name) + " is not F32");
    float *p = nullptr;
    hipError_t e = hipMalloc((void **)&p, t.nbytes);
    if (e == hipSuccess) e = hipMemcpy(p, t.data, t.nbytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        if (p) (void)hipFree(p);
        return fail(g, KORE_GGUF_E_DEVICE, std::string(name) + ": " + hipGetErrorString(e));
    }
    *dev = p;
    return KORE_GGUF_OK;
}

KORE_GGUF_API void kore_gguf_free_device(void *dev) {
    if (dev) (void)hipFree(dev);
}

KORE_GGUF_API const char *kore_gguf_last_error(kore_gguf_t g) { return g ? g->error.c_str() : g_error.c_str(); }

}  // extern "C"
