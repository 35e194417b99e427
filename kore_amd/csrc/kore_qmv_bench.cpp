// kore_qmv_bench.cpp - benchmark driver of libkore_qmv.so (libkore_qmv_bench.so).
//
// Not part of the kore drop-in boundary.  It plays the part of kore's
// forward() for the matvec half of a token: a fixed list of quant() and mv()
// calls (kore.cpp:1418-1421, 1456-1457, 1462-1464, 1469-1470, 1476-1477)
// replayed through the public device-pointer entry points
// kore_qmv_quantize_dev / kore_qmv_matvec_dev / kore_qmv_mv_group_dev on one
// stream, so that a timed region contains no Python between launches; and of
// forward_batch()'s matmul_batch_float calls (kore.cpp:1524-1585) through
// kore_qmv_matmul_batch_dev.
//
// Timing as in kore_attn_bench.cpp: steady_clock around the whole region,
// bracketed by a stream synchronisation on both sides; optionally a HIP event
// pair around the region and one around every operation.
#include "kore_qmv.h"

#include <hip/hip_runtime.h>

#include <chrono>
#include <vector>

#define KQB_API extern "C" __attribute__((visibility("default")))

struct KqbOp {
    int kind;              // 0: quantize x[n] -> xq; 1: matvec tensors[t[0]] . xq -> out[0];
                           // 2: quant + mv of n_t tensors sharing x (kore_qmv_mv_group_dev)
                           // 3: batched matmul of tensors[t[0]] with x[n][cols] -> out[0]
                           // 4: batched matmul of n_t tensors sharing x, one launch
    int n_t;               // kind 2: number of tensors (1..4)
    int t[4];              // indices into tensors
    const float *x;        // kinds 0, 2
    long long n;           // kind 0: elements; kind 3: activations
    void *xq;              // kinds 0, 1
    float *out[4];         // kinds 1 to 4
};

// Runs the n_ops operations `reps` times in order.  op_ms (optional) receives
// reps * n_ops per-operation durations, region_ms (optional) the GPU time of
// the whole region, wall_ms the host time.
KQB_API int kqb_run(const KqbOp *ops, int n_ops, kore_qmv_tensor_t *tensors, int avx2, int reps, void *stream,
                    float *op_ms, float *region_ms, double *wall_ms) {
    hipStream_t s = (hipStream_t)stream;
    const size_t n_ev = op_ms ? 2 * (size_t)n_ops * reps : 0;
    std::vector<hipEvent_t> ev(n_ev, nullptr), reg(region_ms ? 2 : 0, nullptr);
    int rc = KORE_QMV_OK;
    auto cleanup = [&]() {
        for (hipEvent_t e : ev)
            if (e) (void)hipEventDestroy(e);
        for (hipEvent_t e : reg)
            if (e) (void)hipEventDestroy(e);
    };
    for (hipEvent_t &e : ev)
        if (hipEventCreate(&e) != hipSuccess) { cleanup(); return KORE_QMV_E_HIP; }
    for (hipEvent_t &e : reg)
        if (hipEventCreate(&e) != hipSuccess) { cleanup(); return KORE_QMV_E_HIP; }
    if (hipStreamSynchronize(s) != hipSuccess) { cleanup(); return KORE_QMV_E_HIP; }
    const auto t0 = std::chrono::steady_clock::now();
    if (region_ms) (void)hipEventRecord(reg[0], s);
    for (int r = 0; r < reps && rc == KORE_QMV_OK; ++r) {
        for (int i = 0; i < n_ops; ++i) {
            const KqbOp &o = ops[i];
            const size_t k = 2 * ((size_t)r * n_ops + i);
            if (op_ms) (void)hipEventRecord(ev[k], s);
            if (o.kind == 0) {
                rc = kore_qmv_quantize_dev(o.x, o.n, o.xq, s);
            } else if (o.kind == 1) {
                rc = kore_qmv_matvec_dev(tensors[o.t[0]], o.xq, o.out[0], avx2, s);
            } else if (o.kind == 3) {
                rc = kore_qmv_matmul_batch_dev(tensors[o.t[0]], o.x, (int)o.n, o.out[0], s);
            } else {
                kore_qmv_tensor_t g[4];
                for (int m = 0; m < o.n_t && m < 4; ++m) g[m] = tensors[o.t[m]];
                if (o.kind == 4) rc = kore_qmv_matmul_batch_group_dev(o.n_t, g, o.x, (int)o.n, o.out, s);
                else rc = kore_qmv_mv_group_dev(o.n_t, g, o.x, o.out, avx2, s);
            }
            if (rc != KORE_QMV_OK) break;
            if (op_ms) (void)hipEventRecord(ev[k + 1], s);
        }
    }
    if (region_ms) (void)hipEventRecord(reg[1], s);
    if (hipStreamSynchronize(s) != hipSuccess && rc == KORE_QMV_OK) rc = KORE_QMV_E_HIP;
    const auto t1 = std::chrono::steady_clock::now();
    if (wall_ms) *wall_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    if (rc == KORE_QMV_OK && region_ms && hipEventElapsedTime(region_ms, reg[0], reg[1]) != hipSuccess)
        rc = KORE_QMV_E_HIP;
    if (rc == KORE_QMV_OK && op_ms)
        for (size_t k = 0; k < n_ev / 2; ++k)
            if (hipEventElapsedTime(&op_ms[k], ev[2 * k], ev[2 * k + 1]) != hipSuccess) { rc = KORE_QMV_E_HIP; break; }
    cleanup();
    return rc;
}
