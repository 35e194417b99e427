// kore_model.cpp - the C ABI of include/kore_model.h: kore's engine_init over a
// GGUF file with the tensors in HBM, and forward() for one token on the GPU.
#include "kore_model.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <new>
#include <string>
#include <vector>

#include "kore_layer.h"

struct kore_model {
    kore_gguf_hparams hp{};
    int ctx = 0, n_vocab = 0, head_dim = 0, kv_dim = 0;
    size_t weight_bytes = 0;
    int avx2 = 1;                                 // kore's e.avx2: the matvecs' summation order
    std::vector<kore_layer_weights> layers;
    std::vector<kore_qmv_tensor_t> mats;          // every matrix, for destruction
    std::vector<float *> arrays;                  // every device F32 array
    kore_qmv_tensor_t head = nullptr;
    const float *out_norm = nullptr;
    void *embd = nullptr;                         // token_embd in the file's layout
    int embd_type = 0;
    kore_attn_t attn = nullptr;
    kore_layer_t layer = nullptr;
    float *x = nullptr, *logits = nullptr;
    int bsz = 0;                                  // kore's e.bsz = min(64, ctx) (kore.cpp:1354)
    float *bx = nullptr;                          // forward_batch()'s rows, [bsz][n_embd]
    hipStream_t stream = nullptr;
    std::string error;
};

namespace {

thread_local std::string g_error;

int fail(kore_model *m, int code, const std::string &msg) {
    (m ? m->error : g_error) = msg;
    return code;
}

void release(kore_model *m) {
    for (kore_qmv_tensor_t t : m->mats) kore_qmv_tensor_destroy(t);
    for (float *p : m->arrays) (void)hipFree(p);
    for (void *p : {(void *)m->embd, (void *)m->x, (void *)m->logits, (void *)m->bx})
        if (p) (void)hipFree(p);
    if (m->layer) kore_layer_destroy(m->layer);
    if (m->attn) kore_attn_destroy(m->attn);
    if (m->stream) (void)hipStreamDestroy(m->stream);
    delete m;
}

// kore's e.avx2 = KORE_HAVE_AVX2 && cpu_has_avx2() (kore.cpp:512-519, 1293):
// an x86-64 host whose CPU reports AVX2 and FMA (host code: the device pass of
// this file does not know the CPU builtins)
int host_avx2() {
#if defined(__x86_64__) && !defined(__HIP_DEVICE_COMPILE__)
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") ? 1 : 0;
#else
    return 0;
#endif
}

// engine_init (kore.cpp:1274-1365) with the tensors copied to the device
int build(kore_model *m, kore_gguf_t g, int ctx_max) {
    kore_gguf_get_hparams(g, &m->hp);
    const kore_gguf_hparams &h = m->hp;
    if (h.n_layer == 0 || h.n_head == 0 || h.n_head_kv == 0 || h.n_embd % h.n_head != 0 || h.n_head % h.n_head_kv != 0 ||
        h.rope_base <= 0)
        return fail(m, KORE_MODEL_E_LOAD, "qwen2.* hyper-parameters missing or invalid");
    if (h.n_embd % 256 != 0 || h.n_ff % 256 != 0) return fail(m, KORE_MODEL_E_LOAD, "n_embd and n_ff must be multiples of 256");
    m->head_dim = (int)(h.n_embd / h.n_head);
    if (m->head_dim % 2 != 0) return fail(m, KORE_MODEL_E_LOAD, "odd head_dim");
    m->kv_dim = (int)h.n_head_kv * m->head_dim;
    if (ctx_max <= 0) return fail(m, KORE_MODEL_E_LOAD, "ctx_max must be positive");
    m->ctx = h.n_ctx ? (int)std::min<uint32_t>(h.n_ctx, (uint32_t)ctx_max) : ctx_max;

    // The shape of every tensor the forward pass reads, checked before any of
    // them reaches the device: a parseable file with a short norm or bias, or
    // a head of the wrong width, would otherwise send the kernels past the
    // ends of their buffers (kore would read past its host arrays there).
    {
        const uint64_t E = h.n_embd, FF = h.n_ff, KVD = (uint64_t)m->kv_dim;
        std::string bad;
        auto shape = [&](const std::string &n, uint64_t cols, uint64_t rows) {   // 2-D matrix [rows][cols]
            kore_gguf_tensor t{};
            if (!bad.empty() || kore_gguf_find(g, n.c_str(), &t) != KORE_GGUF_OK) return;   // missing: reported below
            if (t.n_dims > 2 || t.dims[0] != cols || (rows && t.dims[1] != rows) || t.dims[1] == 0)
                bad = n + " has the wrong shape";
        };
        auto vec = [&](const std::string &n, uint64_t len) {                      // F32 array of len floats
            kore_gguf_tensor t{};
            if (!bad.empty() || kore_gguf_find(g, n.c_str(), &t) != KORE_GGUF_OK) return;
            if (t.type == 0 && (t.n_dims != 1 || t.dims[0] != len || t.nbytes != 4 * len))
                bad = n + " does not hold " + std::to_string(len) + " floats";
        };
        shape("token_embd.weight", E, 0);
        shape("output.weight", E, 0);
        vec("output_norm.weight", E);
        for (uint32_t l = 0; l < h.n_layer && bad.empty(); ++l) {
            const std::string p = "blk." + std::to_string(l) + ".";
            shape(p + "attn_q.weight", E, E);
            shape(p + "attn_k.weight", E, KVD);
            shape(p + "attn_v.weight", E, KVD);
            shape(p + "attn_output.weight", E, E);
            shape(p + "ffn_gate.weight", E, FF);
            shape(p + "ffn_up.weight", E, FF);
            shape(p + "ffn_down.weight", FF, E);
            vec(p + "attn_q.bias", E);
            vec(p + "attn_k.bias", KVD);
            vec(p + "attn_v.bias", KVD);
            vec(p + "attn_norm.weight", E);
            vec(p + "ffn_norm.weight", E);
        }
        if (!bad.empty()) return fail(m, KORE_MODEL_E_LOAD, bad);
    }

    std::string missing;
    auto mat = [&](const std::string &n) -> kore_qmv_tensor_t {      // matvec weights: Q4_K or Q6_K
        kore_gguf_tensor t{};
        if (kore_gguf_find(g, n.c_str(), &t) != KORE_GGUF_OK || !t.data) { missing = "missing tensor " + n; return nullptr; }
        if (t.type != KORE_QMV_Q4_K && t.type != KORE_QMV_Q6_K) { missing = n + " is not Q4_K/Q6_K"; return nullptr; }
        kore_qmv_tensor_t q = nullptr;
        if (kore_gguf_to_qmv(g, n.c_str(), &q) != KORE_GGUF_OK) { missing = kore_gguf_last_error(g); return nullptr; }
        m->mats.push_back(q);
        m->weight_bytes += t.nbytes;
        return q;
    };
    auto arr = [&](const std::string &n) -> const float * {         // norms and biases: F32
        kore_gguf_tensor t{};
        if (kore_gguf_find(g, n.c_str(), &t) != KORE_GGUF_OK || !t.data) { missing = "missing tensor " + n; return nullptr; }
        if (t.type != 0) { missing = n + " is not F32"; return nullptr; }
        float *p = nullptr;
        if (kore_gguf_to_device_f32(g, n.c_str(), &p) != KORE_GGUF_OK) { missing = kore_gguf_last_error(g); return nullptr; }
        m->arrays.push_back(p);
        m->weight_bytes += t.nbytes;
        return p;
    };
    kore_gguf_tensor te{}, to{};
    if (kore_gguf_find(g, "token_embd.weight", &te) != KORE_GGUF_OK || !te.data)
        return fail(m, KORE_MODEL_E_LOAD, "missing tensor token_embd.weight");
    m->head = mat("output.weight");
    m->out_norm = missing.empty() ? arr("output_norm.weight") : nullptr;
    for (uint32_t l = 0; l < h.n_layer && missing.empty(); ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        kore_layer_weights w{};
        w.wq = mat(p + "attn_q.weight");
        w.bq = arr(p + "attn_q.bias");
        w.wk = mat(p + "attn_k.weight");
        w.bk = arr(p + "attn_k.bias");
        w.wv = mat(p + "attn_v.weight");
        w.bv = arr(p + "attn_v.bias");
        w.wo = mat(p + "attn_output.weight");
        w.attn_norm = arr(p + "attn_norm.weight");
        w.ffn_norm = arr(p + "ffn_norm.weight");
        w.w_gate = mat(p + "ffn_gate.weight");
        w.w_up = mat(p + "ffn_up.weight");
        w.w_down = mat(p + "ffn_down.weight");
        m->layers.push_back(w);
    }
    if (!missing.empty()) return fail(m, KORE_MODEL_E_LOAD, missing);
    kore_gguf_find(g, "output.weight", &to);
    m->n_vocab = (int)to.dims[1];
    if ((int)te.dims[1] != m->n_vocab) return fail(m, KORE_MODEL_E_LOAD, "token_embd and output differ in vocabulary");
    if (te.dims[0] != h.n_embd) return fail(m, KORE_MODEL_E_LOAD, "token_embd rows are not n_embd long");
    if (te.type != 0 && te.type != 1 && te.type != 30 && te.type != KORE_QMV_Q4_K && te.type != KORE_QMV_Q6_K)
        return fail(m, KORE_MODEL_E_LOAD, "token_embd type not supported by get_row");

    hipError_t e = hipStreamCreate(&m->stream);
    if (e == hipSuccess) e = hipMalloc(&m->embd, te.nbytes);
    if (e == hipSuccess) e = hipMemcpy(m->embd, te.data, te.nbytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMalloc((void **)&m->x, h.n_embd * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void **)&m->logits, (size_t)m->n_vocab * sizeof(float));
    m->bsz = std::min(64, m->ctx);
    if (e == hipSuccess) e = hipMalloc((void **)&m->bx, (size_t)m->bsz * h.n_embd * sizeof(float));
    if (e != hipSuccess) return fail(m, KORE_MODEL_E_DEVICE, std::string("device buffers: ") + hipGetErrorString(e));
    m->embd_type = (int)te.type;
    m->weight_bytes += te.nbytes;
    if (kore_attn_create(&m->attn, (int)h.n_layer, m->ctx, (int)h.n_head, (int)h.n_head_kv, m->head_dim, h.rope_base,
                         0) != KORE_ATTN_OK)
        return fail(m, KORE_MODEL_E_DEVICE, std::string("KV cache: ") + kore_attn_last_error(nullptr));
    if (kore_layer_create(&m->layer, (int)h.n_embd, (int)h.n_ff, (int)h.n_head, (int)h.n_head_kv, h.rms_eps) !=
        KORE_LAYER_OK)
        return fail(m, KORE_MODEL_E_DEVICE, std::string("layer scratch: ") + kore_layer_last_error(nullptr));
    return KORE_MODEL_OK;
}

}  // namespace

extern "C" {

KORE_MODEL_API int kore_model_load(const char *gguf_path, int ctx_max, kore_model_t *out) {
    return kore_model_load_ex(gguf_path, ctx_max, -1, out);
}

KORE_MODEL_API int kore_model_load_ex(const char *gguf_path, int ctx_max, int avx2, kore_model_t *out) {
    if (!out) return fail(nullptr, KORE_MODEL_E_LOAD, "out is NULL");
    *out = nullptr;
    if (avx2 < -1 || avx2 > 1) return fail(nullptr, KORE_MODEL_E_LOAD, "avx2 must be -1, 0 or 1");
    kore_gguf_t g = nullptr;
    if (kore_gguf_open(gguf_path, &g) != KORE_GGUF_OK)
        return fail(nullptr, KORE_MODEL_E_LOAD, kore_gguf_last_error(nullptr));
    kore_model *m = new (std::nothrow) kore_model;
    if (!m) {
        kore_gguf_close(g);
        return fail(nullptr, KORE_MODEL_E_LOAD, "out of host memory");
    }
    m->avx2 = avx2 < 0 ? host_avx2() : avx2;
    const int rc = build(m, g, ctx_max);
    kore_gguf_close(g);                               // everything needed is on the device now
    if (rc != KORE_MODEL_OK) {
        g_error = m->error;
        release(m);
        return rc;
    }
    *out = m;
    return KORE_MODEL_OK;
}

KORE_MODEL_API void kore_model_destroy(kore_model_t m) {
    if (m) release(m);
}

KORE_MODEL_API int kore_model_get_info(kore_model_t m, kore_model_info *info) {
    if (!m || !info) return fail(m, KORE_MODEL_E_LOAD, "model or info is NULL");
    info->hp = m->hp;
    info->ctx = m->ctx;
    info->n_vocab = m->n_vocab;
    info->head_dim = m->head_dim;
    info->kv_dim = m->kv_dim;
    info->weight_bytes = m->weight_bytes;
    info->avx2 = m->avx2;
    return KORE_MODEL_OK;
}

KORE_MODEL_API int kore_model_decode_dev(kore_model_t m, int token, int pos, int want_logits, void *stream) {
    if (!m) return fail(nullptr, KORE_MODEL_E_RANGE, "model is NULL");
    if (token < 0 || token >= m->n_vocab || pos < 0 || pos >= m->ctx)          // kore.cpp:1400
        return fail(m, KORE_MODEL_E_RANGE, "token or position out of range");
    void *s = stream ? stream : (void *)m->stream;
    const int E = (int)m->hp.n_embd;
    if (kore_qmv_get_row_dev(m->embd_type, m->embd, token, E, m->x, s) != KORE_QMV_OK)
        return fail(m, KORE_MODEL_E_DEVICE, std::string("embedding: ") + kore_qmv_last_error(nullptr));
    for (int l = 0; l < (int)m->layers.size(); ++l)
        if (kore_layer_decode_dev(m->layer, &m->layers[(size_t)l], m->attn, l, pos, m->x, m->avx2, s) != KORE_LAYER_OK)
            return fail(m, KORE_MODEL_E_DEVICE, std::string("layer: ") + kore_layer_last_error(m->layer));
    if (want_logits) {                                 // kore.cpp:1474-1478
        kore_qmv_mv_opts o{};
        o.norm_w = m->out_norm;
        o.norm_eps = m->hp.rms_eps;
        if (kore_qmv_mv_group_ex_dev(1, &m->head, m->x, &o, &m->logits, m->avx2, s) != KORE_QMV_OK)
            return fail(m, KORE_MODEL_E_DEVICE, std::string("logits: ") + kore_qmv_last_error(m->head));
    }
    return KORE_MODEL_OK;
}

KORE_MODEL_API int kore_model_prefill_dev(kore_model_t m, const int *tokens, int n_tok, int pos0, int want_logits,
                                          void *stream) {
    if (!m) return fail(nullptr, KORE_MODEL_E_RANGE, "model is NULL");
    if (!tokens || n_tok <= 0 || n_tok > m->bsz || pos0 < 0 || pos0 + n_tok > m->ctx)   // kore.cpp:1490
        return fail(m, KORE_MODEL_E_RANGE, "n_tok must be 1..min(64, ctx) and pos0 + n_tok <= ctx");
    for (int z = 0; z < n_tok; ++z)                                                       // kore.cpp:1497
        if (tokens[z] < 0 || tokens[z] >= m->n_vocab) return fail(m, KORE_MODEL_E_RANGE, "token out of range");
    void *s = stream ? stream : (void *)m->stream;
    const int E = (int)m->hp.n_embd;
    for (int z = 0; z < n_tok; ++z)                                                       // kore.cpp:1496-1501
        if (kore_qmv_get_row_dev(m->embd_type, m->embd, tokens[z], E, m->bx + (size_t)z * E, s) != KORE_QMV_OK)
            return fail(m, KORE_MODEL_E_DEVICE, std::string("embedding: ") + kore_qmv_last_error(nullptr));
    for (int l = 0; l < (int)m->layers.size(); ++l)
        if (kore_layer_prefill_dev(m->layer, &m->layers[(size_t)l], m->attn, l, pos0, n_tok, m->bx, s) !=
            KORE_LAYER_OK)
            return fail(m, KORE_MODEL_E_DEVICE, std::string("layer: ") + kore_layer_last_error(m->layer));
    if (want_logits) {                                 // the last row only (kore.cpp:1592-1596)
        kore_qmv_mv_opts o{};
        o.norm_w = m->out_norm;
        o.norm_eps = m->hp.rms_eps;
        const float *last = m->bx + (size_t)(n_tok - 1) * E;
        if (kore_qmv_mv_group_ex_dev(1, &m->head, last, &o, &m->logits, m->avx2, s) != KORE_QMV_OK)
            return fail(m, KORE_MODEL_E_DEVICE, std::string("logits: ") + kore_qmv_last_error(m->head));
    }
    return KORE_MODEL_OK;
}

KORE_MODEL_API const float *kore_model_rows_dev(kore_model_t m) { return m ? m->bx : nullptr; }

KORE_MODEL_API int kore_model_sync(kore_model_t m) {
    if (!m) return fail(nullptr, KORE_MODEL_E_RANGE, "model is NULL");
    const hipError_t e = hipStreamSynchronize(m->stream);
    return e == hipSuccess ? KORE_MODEL_OK : fail(m, KORE_MODEL_E_DEVICE, hipGetErrorString(e));
}

KORE_MODEL_API const float *kore_model_logits_dev(kore_model_t m) { return m ? m->logits : nullptr; }

KORE_MODEL_API int kore_model_decode(kore_model_t m, int token, int pos, float *logits) {
    if (int rc = kore_model_decode_dev(m, token, pos, logits != nullptr, nullptr)) return rc;
    hipError_t e = hipSuccess;
    if (logits)
        e = hipMemcpyAsync(logits, m->logits, (size_t)m->n_vocab * sizeof(float), hipMemcpyDeviceToHost, m->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
    return e == hipSuccess ? KORE_MODEL_OK : fail(m, KORE_MODEL_E_DEVICE, hipGetErrorString(e));
}

KORE_MODEL_API kore_attn_t kore_model_attn(kore_model_t m) { return m ? m->attn : nullptr; }

KORE_MODEL_API const char *kore_model_last_error(kore_model_t m) { return m ? m->error.c_str() : g_error.c_str(); }

}  // extern "C"
