// kore_layer_api.cpp - the C ABI of include/kore_layer.h: one layer of kore's
// forward() chained from libkore_qmv's fused matvec launches and libkore_attn's
// decode, all on one stream.
#include "kore_layer.h"

#include <hip/hip_runtime.h>

#include <new>
#include <string>

struct kore_layer {
    int E = 0, FF = 0, n_head = 0, n_head_kv = 0, head_dim = 0, kvd = 0;
    float eps = 0.f;
    int device = 0;
    hipStream_t stream = nullptr;
    float *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr, *gate = nullptr, *up = nullptr;
    // forward_batch() rows (kore's e.bxb, bq, bk, bv, batt, bgate, bup), kMaxBatch each
    float *bxb = nullptr, *bq = nullptr, *bk = nullptr, *bv = nullptr, *batt = nullptr, *bgate = nullptr,
          *bup = nullptr;
    // the normalised rows' fp16 split for the batched matmuls (nullptr when
    // the split is not available: then the matmuls split bxb themselves)
    void *bx16 = nullptr;
    std::string error;
};

namespace {

thread_local std::string g_error;
constexpr int kMaxBatch = 64;   // kore's KORE_BMAX (kore.cpp:690)

int fail(kore_layer *L, int code, const std::string &msg) {
    (L ? L->error : g_error) = msg;
    return code;
}

void release(kore_layer *L) {
    for (float *p : {L->q, L->k, L->v, L->att, L->gate, L->up, L->bxb, L->bq, L->bk, L->bv, L->batt, L->bgate,
                     L->bup})
        if (p) (void)hipFree(p);
    if (L->bx16) (void)hipFree(L->bx16);
    if (L->stream) (void)hipStreamDestroy(L->stream);
    delete L;
}

bool shape_is(kore_qmv_tensor_t t, int64_t rows, int64_t cols) {
    kore_qmv_info info{};
    return t && kore_qmv_get_info(t, &info) == KORE_QMV_OK && info.rows == rows && info.cols == cols;
}

}  // namespace

extern "C" {

KORE_LAYER_API int kore_layer_create(kore_layer_t *out, int n_embd, int n_ff, int n_head, int n_head_kv,
                                     float rms_eps) {
    if (!out) return fail(nullptr, KORE_LAYER_E_INVALID, "out is NULL");
    *out = nullptr;
    if (n_embd <= 0 || n_ff <= 0 || n_head <= 0 || n_head_kv <= 0 || n_head % n_head_kv || n_embd % n_head ||
        n_embd % 256 || n_ff % 256)
        return fail(nullptr, KORE_LAYER_E_INVALID,
                    "n_embd, n_ff multiples of 256; n_head dividing n_embd; n_head_kv dividing n_head");
    kore_layer *L = new (std::nothrow) kore_layer;
    if (!L) return fail(nullptr, KORE_LAYER_E_HIP, "out of host memory");
    L->E = n_embd;
    L->FF = n_ff;
    L->n_head = n_head;
    L->n_head_kv = n_head_kv;
    L->head_dim = n_embd / n_head;
    L->kvd = n_head_kv * L->head_dim;
    L->eps = rms_eps;
    hipError_t e = hipGetDevice(&L->device);
    // a blocking stream: ordered with the null stream, so a caller's plain
    // hipMemcpy of x before a call is seen by it
    if (e == hipSuccess) e = hipStreamCreate(&L->stream);
    const size_t E = (size_t)L->E, kvd = (size_t)L->kvd, FF = (size_t)L->FF, B = kMaxBatch;
    const size_t sizes[13] = {E, kvd, kvd, E, FF, FF, B * E, B * E, B * kvd, B * kvd, B * E, B * FF, B * FF};
    float **bufs[13] = {&L->q,   &L->k,  &L->v,  &L->att,  &L->gate,  &L->up, &L->bxb,
                        &L->bq,  &L->bk, &L->bv, &L->batt, &L->bgate, &L->bup};
    for (int i = 0; i < 13 && e == hipSuccess; ++i) e = hipMalloc((void **)bufs[i], sizes[i] * sizeof(float));
    if (const size_t sb = kore_qmv_split_bytes(L->E); sb && e == hipSuccess) e = hipMalloc(&L->bx16, sb);
    if (e != hipSuccess) {
        g_error = std::string("kore_layer_create: ") + hipGetErrorString(e);
        release(L);
        return KORE_LAYER_E_HIP;
    }
    *out = L;
    return KORE_LAYER_OK;
}

KORE_LAYER_API void kore_layer_destroy(kore_layer_t L) {
    if (L) release(L);
}

namespace {

// The checks both layer steps make on their arguments.
int check_call(kore_layer *L, const kore_layer_weights *w, kore_attn_t attn, const float *x) {
    if (!w || !attn || !x || ((uintptr_t)x & 15)) return fail(L, KORE_LAYER_E_INVALID, "w, attn or x missing or x unaligned");
    if (!w->attn_norm || !w->ffn_norm) return fail(L, KORE_LAYER_E_INVALID, "attn_norm and ffn_norm are required");
    const int64_t E = L->E, FF = L->FF, kvd = L->kvd;
    if (!shape_is(w->wq, E, E) || !shape_is(w->wk, kvd, E) || !shape_is(w->wv, kvd, E) || !shape_is(w->wo, E, E) ||
        !shape_is(w->w_gate, FF, E) || !shape_is(w->w_up, FF, E) || !shape_is(w->w_down, E, FF))
        return fail(L, KORE_LAYER_E_INVALID, "a weight tensor's shape does not match the layer geometry");
    kore_attn_info ai{};
    if (kore_attn_get_info(attn, &ai) != KORE_ATTN_OK || ai.n_head != L->n_head || ai.n_head_kv != L->n_head_kv ||
        ai.head_dim != L->head_dim)
        return fail(L, KORE_LAYER_E_INVALID, "the attention handle's geometry differs from the layer's");
    return KORE_LAYER_OK;
}

}  // namespace

KORE_LAYER_API int kore_layer_decode_dev(kore_layer_t L, const kore_layer_weights *w, kore_attn_t attn, int layer,
                                         int pos, float *x, int avx2, void *stream) {
    if (!L) return fail(nullptr, KORE_LAYER_E_INVALID, "layer handle is NULL");
    if (int rc = check_call(L, w, attn, x)) return rc;
    void *s = stream ? stream : (void *)L->stream;
    auto qmv_err = [&](kore_qmv_tensor_t t, const char *what) {
        return fail(L, KORE_LAYER_E_STEP, std::string(what) + ": " + kore_qmv_last_error(t));
    };

    // 1. rmsnorm + quant + wq/wk/wv + biases (kore.cpp:1417-1423)
    kore_qmv_mv_opts o1{};
    o1.norm_w = w->attn_norm;
    o1.norm_eps = L->eps;
    o1.bias[0] = w->bq;
    o1.bias[1] = w->bk;
    o1.bias[2] = w->bv;
    kore_qmv_tensor_t qkv[3] = {w->wq, w->wk, w->wv};
    float *qkv_out[3] = {L->q, L->k, L->v};
    if (kore_qmv_mv_group_ex_dev(3, qkv, x, &o1, qkv_out, avx2, s) != KORE_QMV_OK) return qmv_err(w->wq, "q/k/v");
    // 2. RoPE + append + attention (kore.cpp:1424-1455)
    if (kore_attn_decode_dev(attn, layer, pos, L->n_head, L->n_head_kv, L->head_dim, L->q, L->k, L->v, L->att, s) !=
        KORE_ATTN_OK)
        return fail(L, KORE_LAYER_E_STEP, std::string("attention: ") + kore_attn_last_error(attn));
    // 3. quant + Wo, x += o (kore.cpp:1456-1458)
    kore_qmv_mv_opts o3{};
    o3.accumulate = 1;
    if (kore_qmv_mv_group_ex_dev(1, &w->wo, L->att, &o3, &x, avx2, s) != KORE_QMV_OK) return qmv_err(w->wo, "wo");
    // 4. rmsnorm + quant + gate/up (kore.cpp:1461-1464)
    kore_qmv_mv_opts o4{};
    o4.norm_w = w->ffn_norm;
    o4.norm_eps = L->eps;
    kore_qmv_tensor_t gu[2] = {w->w_gate, w->w_up};
    float *gu_out[2] = {L->gate, L->up};
    if (kore_qmv_mv_group_ex_dev(2, gu, x, &o4, gu_out, avx2, s) != KORE_QMV_OK) return qmv_err(w->w_gate, "gate/up");
    // 5. SwiGLU + quant + down, x += o (kore.cpp:1465-1471)
    kore_qmv_mv_opts o5{};
    o5.up = L->up;
    o5.accumulate = 1;
    if (kore_qmv_mv_group_ex_dev(1, &w->w_down, L->gate, &o5, &x, avx2, s) != KORE_QMV_OK) return qmv_err(w->w_down, "down");
    return KORE_LAYER_OK;
}

KORE_LAYER_API int kore_layer_prefill_dev(kore_layer_t L, const kore_layer_weights *w, kore_attn_t attn, int layer,
                                          int pos0, int n_tok, float *x, void *stream) {
    if (!L) return fail(nullptr, KORE_LAYER_E_INVALID, "layer handle is NULL");
    if (int rc = check_call(L, w, attn, x)) return rc;
    if (n_tok < 1 || n_tok > kMaxBatch) return fail(L, KORE_LAYER_E_INVALID, "n_tok must be 1..64 (kore's KORE_BMAX)");
    void *s = stream ? stream : (void *)L->stream;
    const int64_t E = L->E, FF = L->FF;
    auto qmv_err = [&](kore_qmv_tensor_t t, const char *what) {
        return fail(L, KORE_LAYER_E_STEP, std::string(what) + ": " + kore_qmv_last_error(t));
    };
    // rmsnorm of every row, then a batched matmul on the normalised rows: with
    // the split available the rmsnorm writes it and the matmul skips its own
    // split pre-pass (the same results, bit for bit)
    auto norm_matmul = [&](const float *norm_w, int nm, const kore_qmv_tensor_t *mats, const kore_qmv_mv_opts *o,
                           float *const *outs, const char *what) -> int {
        if (L->bx16) {
            if (kore_qmv_rmsnorm_rows_split_dev(x, norm_w, E, n_tok, L->eps, L->bxb, L->bx16, s) != KORE_QMV_OK)
                return qmv_err(nullptr, what);
            if (kore_qmv_matmul_batch_group_split_dev(nm, mats, L->bx16, n_tok, o, outs, s) != KORE_QMV_OK)
                return qmv_err(mats[0], what);
            return KORE_LAYER_OK;
        }
        if (kore_qmv_rmsnorm_rows_dev(x, norm_w, E, n_tok, L->eps, L->bxb, s) != KORE_QMV_OK)
            return qmv_err(nullptr, what);
        if (kore_qmv_matmul_batch_group_ex_dev(nm, mats, L->bxb, n_tok, o, outs, s) != KORE_QMV_OK)
            return qmv_err(mats[0], what);
        return KORE_LAYER_OK;
    };
    // 1. rmsnorm of every row, then q/k/v + biases (kore.cpp:1521-1532)
    kore_qmv_mv_opts o1{};
    o1.bias[0] = w->bq;
    o1.bias[1] = w->bk;
    o1.bias[2] = w->bv;
    kore_qmv_tensor_t qkv[3] = {w->wq, w->wk, w->wv};
    float *qkv_out[3] = {L->bq, L->bk, L->bv};
    if (int rc = norm_matmul(w->attn_norm, 3, qkv, &o1, qkv_out, "attn_norm, q/k/v")) return rc;
    // 2. RoPE + append + causal attention of the rows (kore.cpp:1533-1563)
    if (kore_attn_prefill_dev(attn, layer, pos0, n_tok, L->n_head, L->n_head_kv, L->head_dim, L->bq, L->bk, L->bv,
                              L->batt, s) != KORE_ATTN_OK)
        return fail(L, KORE_LAYER_E_STEP, std::string("attention: ") + kore_attn_last_error(attn));
    // 3. Wo, x += o (kore.cpp:1566-1570)
    kore_qmv_mv_opts acc{};
    acc.accumulate = 1;
    if (kore_qmv_matmul_batch_group_ex_dev(1, &w->wo, L->batt, n_tok, &acc, &x, s) != KORE_QMV_OK)
        return qmv_err(w->wo, "wo");
    // 4. rmsnorm, gate/up, SwiGLU (kore.cpp:1572-1583)
    kore_qmv_tensor_t gu[2] = {w->w_gate, w->w_up};
    float *gu_out[2] = {L->bgate, L->bup};
    if (L->bx16) {   // the SwiGLU where gate/up's split tiles are summed (bup is scratch)
        if (kore_qmv_rmsnorm_rows_split_dev(x, w->ffn_norm, E, n_tok, L->eps, L->bxb, L->bx16, s) != KORE_QMV_OK)
            return qmv_err(nullptr, "ffn_norm");
        if (kore_qmv_matmul_batch_glu_split_dev(gu, L->bx16, n_tok, L->bgate, L->bup, s) != KORE_QMV_OK)
            return qmv_err(w->w_gate, "gate/up, swiglu");
    } else {
        if (int rc = norm_matmul(w->ffn_norm, 2, gu, nullptr, gu_out, "ffn_norm, gate/up")) return rc;
        if (kore_qmv_swiglu_dev(L->bgate, L->bup, (int64_t)n_tok * FF, s) != KORE_QMV_OK)
            return qmv_err(nullptr, "swiglu");
    }
    // 5. down, x += o (kore.cpp:1585-1589)
    if (kore_qmv_matmul_batch_group_ex_dev(1, &w->w_down, L->bgate, n_tok, &acc, &x, s) != KORE_QMV_OK)
        return qmv_err(w->w_down, "down");
    return KORE_LAYER_OK;
}

KORE_LAYER_API int kore_layer_sync(kore_layer_t L) {
    if (!L) return fail(nullptr, KORE_LAYER_E_INVALID, "layer handle is NULL");
    const hipError_t e = hipStreamSynchronize(L->stream);
    return e == hipSuccess ? KORE_LAYER_OK : fail(L, KORE_LAYER_E_HIP, hipGetErrorString(e));
}

KORE_LAYER_API const char *kore_layer_last_error(kore_layer_t L) { return L ? L->error.c_str() : g_error.c_str(); }

}  // extern "C"
