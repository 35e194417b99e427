// kore_attn_bench.cpp - benchmark driver of libkore_attn.so (libkore_attn_bench.so).
//
// Not part of the kore drop-in boundary.  It plays the part of kore's C++
// layer loop - forward() calls the attention block once per layer per token
// (kore.cpp:1413-1455), forward_batch() once per layer per chunk
// (kore.cpp:1516-1563) - so that a timed region contains no Python between
// launches.  Every launch goes through the public device-pointer entry points
// kore_attn_decode_dev / kore_attn_prefill_dev on the handle's own stream.
//
// Timing: std::chrono::steady_clock around the whole region (kore times
// with steady_clock, kore.cpp:1886-1889), bracketed by a stream
// synchronisation on both sides; when `region_ms` is given, a pair of HIP
// events on the same stream brackets the whole region (GPU time of all its
// launches, gaps between them included); when `launch_ms` is given, a pair
// of HIP events brackets each launch and its elapsed time is returned per
// launch (the events themselves add to the region's time, so a pass that
// measures the region should not ask for them).
#include "kore_attn.h"

#include <hip/hip_runtime.h>

#include <chrono>
#include <vector>

#define KAB_API extern "C" __attribute__((visibility("default")))

namespace {

struct Events {
    std::vector<hipEvent_t> ev;
    explicit Events(size_t n) : ev(n, nullptr) {}
    ~Events() {
        for (hipEvent_t e : ev)
            if (e) (void)hipEventDestroy(e);
    }
    bool create() {
        for (hipEvent_t &e : ev)
            if (hipEventCreate(&e) != hipSuccess) return false;
        return true;
    }
};

// Runs `body(i)` for i < n launches on `stream`, timing the region and
// (when launch_ms is non-null) each launch.
template <class Body>
int timed_region(hipStream_t stream, int n, float *launch_ms, float *region_ms, double *wall_ms, Body body) {
    Events evs(launch_ms ? 2 * (size_t)n : 0), reg(region_ms ? 2 : 0);
    if ((launch_ms && !evs.create()) || (region_ms && !reg.create())) return KORE_ATTN_E_HIP;
    if (hipStreamSynchronize(stream) != hipSuccess) return KORE_ATTN_E_HIP;
    const auto t0 = std::chrono::steady_clock::now();
    if (region_ms && hipEventRecord(reg.ev[0], stream) != hipSuccess) return KORE_ATTN_E_HIP;
    for (int i = 0; i < n; ++i) {
        if (launch_ms && hipEventRecord(evs.ev[2 * i], stream) != hipSuccess) return KORE_ATTN_E_HIP;
        if (int rc = body(i)) return rc;
        if (launch_ms && hipEventRecord(evs.ev[2 * i + 1], stream) != hipSuccess) return KORE_ATTN_E_HIP;
    }
    if (region_ms && hipEventRecord(reg.ev[1], stream) != hipSuccess) return KORE_ATTN_E_HIP;
    if (hipStreamSynchronize(stream) != hipSuccess) return KORE_ATTN_E_HIP;
    const auto t1 = std::chrono::steady_clock::now();
    if (wall_ms) *wall_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    if (region_ms && hipEventElapsedTime(region_ms, reg.ev[0], reg.ev[1]) != hipSuccess) return KORE_ATTN_E_HIP;
    if (launch_ms)
        for (int i = 0; i < n; ++i)
            if (hipEventElapsedTime(&launch_ms[i], evs.ev[2 * i], evs.ev[2 * i + 1]) != hipSuccess)
                return KORE_ATTN_E_HIP;
    return KORE_ATTN_OK;
}

}  // namespace

// n_steps single-token decode steps at positions pos_first + s * pos_step
// (pos_step 1: one new token per step; 0: the same position again) over
// layers 0..n_layer-1 (layer inner, like forward()).  Device inputs are laid
// out [layer][in_steps][dim] (step s of layer l at (l*in_steps + s)*dim);
// outputs [out_steps][layer][n_head*head_dim] with step s written to row
// s % out_steps.  launch_ms (optional) receives n_steps*n_layer durations,
// region_ms (optional) the GPU time of the whole region.
KAB_API int kab_decode_run(kore_attn_t h, int n_layer, int pos_first, int pos_step, int n_steps,
                           const float *q, const float *k, const float *v, int in_steps, float *out,
                           int out_steps, float *launch_ms, float *region_ms, double *wall_ms) {
    kore_attn_info inf;
    if (int rc = kore_attn_get_info(h, &inf)) return rc;
    if (n_layer <= 0 || n_layer > inf.n_layer || n_steps <= 0 || out_steps <= 0 || pos_step < 0 ||
        in_steps < (pos_step ? n_steps : 1))
        return KORE_ATTN_E_INVALID;
    const size_t E = (size_t)inf.n_head * inf.head_dim, kvd = (size_t)inf.n_head_kv * inf.head_dim;
    hipStream_t stream = (hipStream_t)inf.stream;
    return timed_region(stream, n_steps * n_layer, launch_ms, region_ms, wall_ms, [&](int i) {
        const int s = i / n_layer, l = i % n_layer;
        const size_t row = (size_t)l * in_steps + (pos_step ? s : 0);
        return kore_attn_decode_dev(h, l, pos_first + s * pos_step, inf.n_head, inf.n_head_kv, inf.head_dim,
                                    q + row * E, k + row * kvd, v + row * kvd,
                                    out + ((size_t)(s % out_steps) * n_layer + l) * E, nullptr);
    });
}

// n_steps passes of a causal prefill of n_tok rows at pos0 over layers
// 0..n_layer-1 (one forward_batch() chunk per layer).  Inputs [layer][n_tok][dim],
// outputs [layer][n_tok][n_head*head_dim].
KAB_API int kab_prefill_run(kore_attn_t h, int n_layer, int pos0, int n_tok, int n_steps,
                            const float *q, const float *k, const float *v, float *out,
                            float *launch_ms, float *region_ms, double *wall_ms) {
    kore_attn_info inf;
    if (int rc = kore_attn_get_info(h, &inf)) return rc;
    if (n_layer <= 0 || n_layer > inf.n_layer || n_steps <= 0 || n_tok <= 0) return KORE_ATTN_E_INVALID;
    const size_t E = (size_t)inf.n_head * inf.head_dim, kvd = (size_t)inf.n_head_kv * inf.head_dim;
    hipStream_t stream = (hipStream_t)inf.stream;
    return timed_region(stream, n_steps * n_layer, launch_ms, region_ms, wall_ms, [&](int i) {
        const int l = i % n_layer;
        const size_t row = (size_t)l * n_tok;
        return kore_attn_prefill_dev(h, l, pos0, n_tok, inf.n_head, inf.n_head_kv, inf.head_dim,
                                     q + row * E, k + row * kvd, v + row * kvd, out + row * E,
                                     nullptr);
    });
}

// The host-pointer round trip kore's own call sites would make: n_steps decode
// steps at positions pos_first.. over layers 0..n_layer-1 through
// kore_attn_decode (H2D of q/k/v, the kernels, D2H of the output, returning
// when the output is in host memory, like kore's loop at kore.cpp:1432-1455).
// Host inputs [layer][in_steps][dim]; out [n_layer][n_head*head_dim] (the last
// step).  wall_ms: steady_clock over the whole loop, after one untimed call
// (layer 0, first step) that re-decodes that step with the same inputs.
KAB_API int kab_decode_host_run(kore_attn_t h, int n_layer, int pos_first, int n_steps, const float *q,
                                const float *k, const float *v, int in_steps, float *out, double *wall_ms) {
    kore_attn_info inf;
    if (int rc = kore_attn_get_info(h, &inf)) return rc;
    if (n_layer <= 0 || n_layer > inf.n_layer || n_steps <= 0 || in_steps < n_steps || !wall_ms)
        return KORE_ATTN_E_INVALID;
    const size_t E = (size_t)inf.n_head * inf.head_dim, kvd = (size_t)inf.n_head_kv * inf.head_dim;
    // one untimed call first: the handle sizes its host staging on its first host-pointer call
    if (int rc = kore_attn_decode(h, 0, pos_first, inf.n_head, inf.n_head_kv, inf.head_dim, q, k, v, out)) return rc;
    const auto t0 = std::chrono::steady_clock::now();
    for (int s = 0; s < n_steps; ++s)
        for (int l = 0; l < n_layer; ++l) {
            const size_t row = (size_t)l * in_steps + s;
            if (int rc = kore_attn_decode(h, l, pos_first + s, inf.n_head, inf.n_head_kv, inf.head_dim, q + row * E,
                                          k + row * kvd, v + row * kvd, out + (size_t)l * E))
                return rc;
        }
    *wall_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    return KORE_ATTN_OK;
}

// The same for a prefill chunk: n_tok rows at pos0 over layers 0..n_layer-1
// through kore_attn_prefill (kore.cpp:1503-1563).  Host inputs and outputs
// [layer][n_tok][dim].
KAB_API int kab_prefill_host_run(kore_attn_t h, int n_layer, int pos0, int n_tok, const float *q, const float *k,
                                 const float *v, float *out, double *wall_ms) {
    kore_attn_info inf;
    if (int rc = kore_attn_get_info(h, &inf)) return rc;
    if (n_layer <= 0 || n_layer > inf.n_layer || n_tok <= 0 || !wall_ms) return KORE_ATTN_E_INVALID;
    const size_t E = (size_t)inf.n_head * inf.head_dim, kvd = (size_t)inf.n_head_kv * inf.head_dim;
    // one untimed call first: the handle sizes its host staging on its first host-pointer call
    if (int rc = kore_attn_prefill(h, 0, pos0, n_tok, inf.n_head, inf.n_head_kv, inf.head_dim, q, k, v, out)) return rc;
    const auto t0 = std::chrono::steady_clock::now();
    for (int l = 0; l < n_layer; ++l) {
        const size_t row = (size_t)l * n_tok;
        if (int rc = kore_attn_prefill(h, l, pos0, n_tok, inf.n_head, inf.n_head_kv, inf.head_dim, q + row * E,
                                       k + row * kvd, v + row * kvd, out + row * E))
            return rc;
    }
    *wall_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    return KORE_ATTN_OK;
}
