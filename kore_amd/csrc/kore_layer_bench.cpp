// kore_layer_bench.cpp - benchmark driver of libkore_layer.so (libkore_layer_bench.so).
//
// Not part of the kore drop-in boundary.  It plays kore's decode loop for whole
// tokens (forward(), kore.cpp:1397-1484): the token's embedding row into x,
// every layer through kore_layer_decode_dev, then the logits (rmsnorm with
// out_norm, quant, the output head: kore.cpp:1474-1478), all on one stream, so
// a timed region contains no Python between launches.
#include "kore_layer.h"

#include <hip/hip_runtime.h>

#include <chrono>

#define KLB_API extern "C" __attribute__((visibility("default")))

// Runs tokens pos0 .. pos0 + n_tok - 1 (token t's embedding row emb[t]),
// `reps` times over the same positions.  region_ms (optional) receives the GPU
// time of the whole region (HIP events on the driver's stream), wall_ms the
// host time.  Returns 0 or the first failing library code (negated for HIP).
KLB_API int klb_tokens(kore_layer_t L, const kore_layer_weights *w, int n_layer, kore_attn_t attn,
                       kore_qmv_tensor_t head, const float *out_norm, float eps, const float *emb, int E, int n_tok,
                       int pos0, float *x, float *logits, int avx2, int reps, float *region_ms, double *wall_ms) {
    hipStream_t s = nullptr;
    if (hipStreamCreate(&s) != hipSuccess) return -1;
    hipEvent_t ev[2] = {nullptr, nullptr};
    int rc = 0;
    if (hipEventCreate(&ev[0]) != hipSuccess || hipEventCreate(&ev[1]) != hipSuccess) rc = -1;
    kore_qmv_mv_opts ho{};
    ho.norm_w = out_norm;
    ho.norm_eps = eps;
    if (!rc && hipStreamSynchronize(s) != hipSuccess) rc = -1;
    const auto t0 = std::chrono::steady_clock::now();
    if (!rc) (void)hipEventRecord(ev[0], s);
    for (int r = 0; r < reps && !rc; ++r) {
        for (int t = 0; t < n_tok && !rc; ++t) {
            if (hipMemcpyAsync(x, emb + (size_t)t * E, (size_t)E * sizeof(float), hipMemcpyDeviceToDevice, s) !=
                hipSuccess) {
                rc = -1;
                break;
            }
            for (int l = 0; l < n_layer && !rc; ++l) rc = kore_layer_decode_dev(L, &w[l], attn, l, pos0 + t, x, avx2, s);
            if (!rc) rc = kore_qmv_mv_group_ex_dev(1, &head, x, &ho, &logits, avx2, s);
        }
    }
    if (!rc) (void)hipEventRecord(ev[1], s);
    if (hipStreamSynchronize(s) != hipSuccess && !rc) rc = -1;
    const auto t1 = std::chrono::steady_clock::now();
    if (wall_ms) *wall_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    if (!rc && region_ms && hipEventElapsedTime(region_ms, ev[0], ev[1]) != hipSuccess) rc = -1;
    for (hipEvent_t e : ev)
        if (e) (void)hipEventDestroy(e);
    (void)hipStreamDestroy(s);
    return rc;
}

// kore's prompt prefill (forward_batch(), kore.cpp:1486-1598, as kore's prompt
// loop calls it in 64-token chunks, kore.cpp:1727-1733): chunk c's embedding
// rows emb[c * nb ..] into x [nb][E], every layer through kore_layer_prefill_dev
// at positions c * nb .., and after the prompt's last chunk the logits of its
// last row (kore's want_logits = last); `chunks` chunks, `reps` times over the
// same positions.  Same timing outputs and return codes as klb_tokens.
KLB_API int klb_prefill(kore_layer_t L, const kore_layer_weights *w, int n_layer, kore_attn_t attn,
                        kore_qmv_tensor_t head, const float *out_norm, float eps, const float *emb, int E, int nb,
                        int chunks, float *x, float *logits, int reps, float *region_ms, double *wall_ms) {
    hipStream_t s = nullptr;
    if (hipStreamCreate(&s) != hipSuccess) return -1;
    hipEvent_t ev[2] = {nullptr, nullptr};
    int rc = 0;
    if (hipEventCreate(&ev[0]) != hipSuccess || hipEventCreate(&ev[1]) != hipSuccess) rc = -1;
    kore_qmv_mv_opts ho{};
    ho.norm_w = out_norm;
    ho.norm_eps = eps;
    if (!rc && hipStreamSynchronize(s) != hipSuccess) rc = -1;
    const auto t0 = std::chrono::steady_clock::now();
    if (!rc) (void)hipEventRecord(ev[0], s);
    for (int r = 0; r < reps && !rc; ++r) {
        for (int c = 0; c < chunks && !rc; ++c) {
            const size_t row0 = (size_t)c * nb;
            if (hipMemcpyAsync(x, emb + row0 * E, (size_t)nb * E * sizeof(float), hipMemcpyDeviceToDevice, s) !=
                hipSuccess) {
                rc = -1;
                break;
            }
            for (int l = 0; l < n_layer && !rc; ++l) rc = kore_layer_prefill_dev(L, &w[l], attn, l, c * nb, nb, x, s);
            float *last = x + (size_t)(nb - 1) * E;
            if (!rc && c == chunks - 1) rc = kore_qmv_mv_group_ex_dev(1, &head, last, &ho, &logits, 1, s);
        }
    }
    if (!rc) (void)hipEventRecord(ev[1], s);
    if (hipStreamSynchronize(s) != hipSuccess && !rc) rc = -1;
    const auto t1 = std::chrono::steady_clock::now();
    if (wall_ms) *wall_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    if (!rc && region_ms && hipEventElapsedTime(region_ms, ev[0], ev[1]) != hipSuccess) rc = -1;
    for (hipEvent_t e : ev)
        if (e) (void)hipEventDestroy(e);
    (void)hipStreamDestroy(s);
    return rc;
}
