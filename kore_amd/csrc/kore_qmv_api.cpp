// kore_qmv_api.cpp - the C ABI of include/kore_qmv.h over the gfx950
// kernels of kore_qmv_kernels.hip.
#include "kore_qmv.h"
#include "kore_qmv_synth.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <string>

#include "kore_qmv_kernels.h"

using namespace kore_qmv_gpu;

struct kore_qmv_tensor {
    int type = 0;
    int device = 0;
    int64_t rows = 0, cols = 0;
    int nblk = 0;
    int rows_per_wave = 16;
    int num_cu = 0;
    uint8_t *w = nullptr;      // Q4_K blocks or Q6_K bodies
    uint16_t *wd = nullptr;    // Q6_K scales
    uint8_t *xq = nullptr;     // quantised activations (the matvec's layout) when quantised apart
    size_t weight_bytes = 0;
    std::string error;
};

namespace {

thread_local std::string g_error;

int fail(kore_qmv_tensor *t, int code, const std::string &msg) {
    (t ? t->error : g_error) = msg;
    return code;
}

int hip_fail(kore_qmv_tensor *t, hipError_t e, const char *what) {
    return fail(t, KORE_QMV_E_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

#define QMV_TRY(t, call)                                        \
    do {                                                        \
        hipError_t e_ = (call);                                 \
        if (e_ != hipSuccess) return hip_fail((t), e_, #call);  \
    } while (0)

// Per-device workspace of the batched matmul, allocated once, at the first
// tensor creation on the device, and kept until the process ends: the partial
// sums of split tiles, sized for the largest grid, and the fp16 split of the
// activations, sized for the widest tensor any call accepts (kMaxBlocks
// blocks, 8.7 MB).  Neither is ever freed or regrown, so a launch enqueued
// from any thread, or captured in a graph, never holds a stale pointer.
// Calls on one device share it: they must not overlap.
struct GemmScratch {
    std::mutex mu;
    float *partials = nullptr;
    uint8_t *x16 = nullptr;
};
GemmScratch g_gemm[64];

int row_tiles(int64_t rows) { return (int)((rows + gemm_rows_per_tile() - 1) / gemm_rows_per_tile()); }

hipError_t gemm_scratch_reserve(int dev, int num_cu) {
    GemmScratch &g = g_gemm[dev];
    std::lock_guard<std::mutex> lock(g.mu);
    hipError_t e = hipSuccess;
    if (!g.partials) {
        // 2 slots per worker: the fp32 path's 64-row slots at up to 4 workgroups
        // per CU, the same bytes as the fp16 path's 256-row slots at 1 per CU
        static_assert(4 * kGemmSlotFloats == kG16SlotFloats, "slot sizes");
        const size_t bytes = (size_t)2 * gemm_max_workers(num_cu) * kGemmSlotFloats * sizeof(float);
        if ((e = hipMalloc((void **)&g.partials, bytes)) != hipSuccess) return e;
    }
    if (!g.x16) {
        if ((e = hipMalloc((void **)&g.x16, (size_t)kMaxBlocks * kG16BlockBytes)) != hipSuccess) return e;
    }
    return hipSuccess;
}

// Per-device staging buffers and stream of the synchronous host-pointer calls.
struct HostPath {
    std::mutex mu;
    hipStream_t stream = nullptr;
    void *buf = nullptr;
    size_t cap = 0;
};
HostPath g_host[64];

hipError_t host_path(int dev, size_t need, HostPath **out) {
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    HostPath &h = g_host[dev];
    if (!h.stream) {
        hipError_t e = hipStreamCreateWithFlags(&h.stream, hipStreamNonBlocking);
        if (e != hipSuccess) return e;
    }
    if (h.cap < need) {
        if (h.buf) (void)hipFree(h.buf);
        h.buf = nullptr;
        h.cap = 0;
        hipError_t e = hipMalloc(&h.buf, need);
        if (e != hipSuccess) return e;
        h.cap = need;
    }
    *out = &h;
    return hipSuccess;
}

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// Rows per wave: as many as still give the device about three waves per CU
// (six for long rows, more than 16 blocks, whose waves each take several
// load round trips); with fewer rows each wave spreads a row's blocks over
// more lanes, and every step's chain advances then run on fewer lanes.
// Measured on the 7B shapes (us per launch, rows per wave 1 / 2 / 4 / 8):
// attn_output 8.2 / 7.0 / 6.4 / 7.2, q+k+v 14.7 / 11.1 / 10.4 / 12.3,
// ffn_down (Q4_K) 18.4 / 17.0 / 19.7 / 29.1.  A matrix tall enough for more
// than eight such rounds at 16 rows per wave (the 152064-row output head)
// takes 4: 79-83 us against 89 at 16 and 85 at 8 (gate+up, three rounds,
// stays at 16: 20.6 us against 21.4 at 4).
int pick_rows_per_wave(int64_t rows, int nblk, int num_cu) {
    if (const char *env = getenv("KORE_QMV_ROWS_PER_WAVE")) {
        const int r = atoi(env);
        if (r == 1 || r == 2 || r == 4 || r == 8 || r == 16) return r;
    }
    const int64_t want = (nblk > 16 ? 6LL : 3LL) * std::max(num_cu, 1);
    if (rows / 16 > 8 * want) return 4;
    for (int r = 16; r > 1; r /= 2)
        if (rows / r >= want) return r;
    return 1;
}

// Workgroups of one matvec launch: one per tile of 4 x rows-per-wave rows
// (0), or about k per CU, each walking a contiguous run of tiles.
int max_workgroups(int num_cu) {
    if (const char *env = getenv("KORE_QMV_WGS_PER_CU")) {
        const int k = atoi(env);
        if (k > 0 && k <= 64) return k * num_cu;
    }
    return 0;
}

// Quantise inside the matvec workgroups (one launch instead of two) when
// every workgroup's share of it is small: few blocks per row and not so many
// workgroups that re-reading the activations costs more than a launch.
bool fuse_quantisation(int nblk, int64_t workgroups) {
    if (const char *env = getenv("KORE_QMV_FUSE")) return atoi(env) != 0;
    return nblk <= 16 && workgroups * nblk <= 65536;
}

int check_dev_ptr(kore_qmv_tensor *t, const void *p, size_t align, const char *what) {
    if (!p) return fail(t, KORE_QMV_E_INVALID, std::string(what) + " is NULL");
    if ((uintptr_t)p % align) return fail(t, KORE_QMV_E_INVALID, std::string(what) + " is not aligned");
    return KORE_QMV_OK;
}

}  // namespace

extern "C" {

KORE_QMV_API int kore_qmv_tensor_create(kore_qmv_tensor_t *out, int type, int64_t rows, int64_t cols,
                                        const void *data, int data_on_device) {
    if (!out) return fail(nullptr, KORE_QMV_E_INVALID, "out is NULL");
    *out = nullptr;
    if (type != KORE_QMV_Q4_K && type != KORE_QMV_Q6_K)
        return fail(nullptr, KORE_QMV_E_UNSUPPORTED, "weight type is not Q4_K (12) or Q6_K (14)");
    if (rows <= 0 || cols <= 0 || cols % 256 != 0)
        return fail(nullptr, KORE_QMV_E_INVALID, "rows must be > 0 and cols a positive multiple of 256");
    if (cols / 256 > kMaxBlocks)
        return fail(nullptr, KORE_QMV_E_UNSUPPORTED, "cols above 32768");
    if (rows > (int64_t)INT32_MAX) return fail(nullptr, KORE_QMV_E_UNSUPPORTED, "more than 2^31-1 rows");
    if (!data) return fail(nullptr, KORE_QMV_E_INVALID, "data is NULL");
    if (data_on_device && ((uintptr_t)data & 1)) return fail(nullptr, KORE_QMV_E_INVALID, "data is not 2-byte aligned");

    kore_qmv_tensor *t = new (std::nothrow) kore_qmv_tensor;
    if (!t) return fail(nullptr, KORE_QMV_E_NOMEM, "host allocation failed");
    auto bail = [&](int code) {
        g_error = t->error;
        if (t->w) (void)hipFree(t->w);
        if (t->wd) (void)hipFree(t->wd);
        if (t->xq) (void)hipFree(t->xq);
        delete t;
        return code;
    };
    t->type = type;
    t->rows = rows;
    t->cols = cols;
    t->nblk = (int)(cols / 256);
    hipError_t e = hipGetDevice(&t->device);
    if (e != hipSuccess) return bail(hip_fail(t, e, "hipGetDevice"));
    int num_cu = 0;
    e = hipDeviceGetAttribute(&num_cu, hipDeviceAttributeMultiprocessorCount, t->device);
    if (e != hipSuccess) return bail(hip_fail(t, e, "hipDeviceGetAttribute"));
    t->num_cu = num_cu;
    t->rows_per_wave = pick_rows_per_wave(rows, t->nblk, num_cu);
    if ((e = hipMalloc(&t->xq, (size_t)t->nblk * 308)) != hipSuccess) return bail(hip_fail(t, e, "hipMalloc"));
    if (t->device < 0 || t->device >= 64) return bail(fail(t, KORE_QMV_E_UNSUPPORTED, "device ordinal above 63"));
    if ((e = gemm_scratch_reserve(t->device, num_cu)) != hipSuccess)
        return bail(hip_fail(t, e, "matmul workspace"));

    const int64_t nblocks = rows * t->nblk;
    const size_t bb = type == KORE_QMV_Q4_K ? kQ4Bytes : kQ6Bytes;
    t->weight_bytes = (size_t)nblocks * bb;
    if (type == KORE_QMV_Q4_K) {
        if ((e = hipMalloc(&t->w, t->weight_bytes)) != hipSuccess) return bail(hip_fail(t, e, "hipMalloc"));
        e = hipMemcpy(t->w, data, t->weight_bytes, data_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice);
        if (e != hipSuccess) return bail(hip_fail(t, e, "hipMemcpy"));
        *out = t;
        return KORE_QMV_OK;
    }
    if ((e = hipMalloc(&t->w, (size_t)nblocks * kQ6Body)) != hipSuccess) return bail(hip_fail(t, e, "hipMalloc"));
    if ((e = hipMalloc(&t->wd, (size_t)nblocks * 2)) != hipSuccess) return bail(hip_fail(t, e, "hipMalloc"));
    const uint8_t *raw = (const uint8_t *)data;
    uint8_t *staged = nullptr;
    if (!data_on_device) {
        if ((e = hipMalloc(&staged, t->weight_bytes)) != hipSuccess) return bail(hip_fail(t, e, "hipMalloc"));
        e = hipMemcpy(staged, data, t->weight_bytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            (void)hipFree(staged);
            return bail(hip_fail(t, e, "hipMemcpy"));
        }
        raw = staged;
    }
    e = launch_q6k_split(raw, nblocks, t->w, t->wd, nullptr);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (staged) (void)hipFree(staged);
    if (e != hipSuccess) return bail(hip_fail(t, e, "Q6_K upload"));
    *out = t;
    return KORE_QMV_OK;
}

KORE_QMV_API void kore_qmv_tensor_destroy(kore_qmv_tensor_t t) {
    if (!t) return;
    int cur = -1;
    (void)hipGetDevice(&cur);
    if (cur != t->device) (void)hipSetDevice(t->device);
    if (t->w) (void)hipFree(t->w);
    if (t->wd) (void)hipFree(t->wd);
    if (t->xq) (void)hipFree(t->xq);
    if (cur >= 0 && cur != t->device) (void)hipSetDevice(cur);
    delete t;
}

KORE_QMV_API int kore_qmv_quantize_dev(const float *x, int64_t n, void *xq, void *stream) {
    if (n <= 0 || n % 256 != 0) return fail(nullptr, KORE_QMV_E_INVALID, "n must be a positive multiple of 256");
    if (int rc = check_dev_ptr(nullptr, x, 16, "x")) return rc;
    if (int rc = check_dev_ptr(nullptr, xq, 16, "xq")) return rc;
    hipError_t e = launch_quantize_q8k(x, n, (uint8_t *)xq, false, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(nullptr, e, "quantize launch");
    return KORE_QMV_OK;
}

KORE_QMV_API int kore_qmv_quantize(const float *x, int64_t n, void *xq) {
    if (!x || !xq) return fail(nullptr, KORE_QMV_E_INVALID, "x or xq is NULL");
    if (n <= 0 || n % 256 != 0) return fail(nullptr, KORE_QMV_E_INVALID, "n must be a positive multiple of 256");
    int dev = 0;
    QMV_TRY(nullptr, hipGetDevice(&dev));
    const size_t xb = align256((size_t)n * 4), qb = (size_t)(n / 256) * kQ8Bytes;
    HostPath *h = nullptr;
    std::lock_guard<std::mutex> lock(g_host[dev & 63].mu);
    QMV_TRY(nullptr, host_path(dev, xb + qb, &h));
    uint8_t *dx = (uint8_t *)h->buf, *dq = dx + xb;
    QMV_TRY(nullptr, hipMemcpyAsync(dx, x, (size_t)n * 4, hipMemcpyHostToDevice, h->stream));
    QMV_TRY(nullptr, launch_quantize_q8k((const float *)dx, n, dq, false, h->stream));
    QMV_TRY(nullptr, hipMemcpyAsync(xq, dq, qb, hipMemcpyDeviceToHost, h->stream));
    QMV_TRY(nullptr, hipStreamSynchronize(h->stream));
    return KORE_QMV_OK;
}

static MatDesc desc_of(kore_qmv_tensor *t, float *out, const float *bias = nullptr, int accumulate = 0) {
    return MatDesc{t->w, t->wd, out, (int)t->rows, t->type, 0, 0, bias, accumulate};
}

// One grouped launch: xq given (fused = false) or x quantised in the kernel
// (after the pre-op of opts, if any); opts also carries the store epilogue.
static int launch_group(int n, kore_qmv_tensor *const *ts, const void *xq, const float *x, float *const *outs,
                        int avx2, hipStream_t s, bool xq_image = false, const kore_qmv_mv_opts *opts = nullptr) {
    GroupArgs a{};
    int64_t rows = 0;
    for (int k = 0; k < n; ++k) {
        a.m[k] = desc_of(ts[k], outs[k], opts ? opts->bias[k] : nullptr, opts ? opts->accumulate : 0);
        rows += ts[k]->rows;
    }
    a.n_mat = n;
    a.nblk = ts[0]->nblk;
    a.xq = (const uint8_t *)xq;
    a.x = x;
    a.xq_image = xq_image ? 1 : 0;
    if (opts && x) {
        a.norm_w = opts->norm_w;
        a.norm_eps = opts->norm_eps;
        a.up = opts->up;
    }
    const int r = n == 1 ? ts[0]->rows_per_wave : pick_rows_per_wave(rows, ts[0]->nblk, ts[0]->num_cu);
    hipError_t e = launch_matvec_group(avx2 != 0, a, r, max_workgroups(ts[0]->num_cu), ts[0]->num_cu, s);
    if (e != hipSuccess) return hip_fail(ts[0], e, "matvec launch");
    return KORE_QMV_OK;
}

KORE_QMV_API int kore_qmv_matvec_dev(kore_qmv_tensor_t t, const void *xq, float *out, int avx2, void *stream) {
    if (!t) return fail(nullptr, KORE_QMV_E_INVALID, "tensor is NULL");
    if (int rc = check_dev_ptr(t, xq, 16, "xq")) return rc;
    if (int rc = check_dev_ptr(t, out, 4, "out")) return rc;
    return launch_group(1, &t, xq, nullptr, &out, avx2, (hipStream_t)stream);
}

KORE_QMV_API int kore_qmv_mv_group_ex_dev(int n, const kore_qmv_tensor_t *ts, const float *x,
                                          const kore_qmv_mv_opts *opts, float *const *outs, int avx2, void *stream) {
    if (n < 1 || n > kMaxGroup || !ts || !outs)
        return fail(nullptr, KORE_QMV_E_INVALID, "n must be 1..4 with tensors and outputs");
    for (int k = 0; k < n; ++k) {
        if (!ts[k]) return fail(nullptr, KORE_QMV_E_INVALID, "tensor is NULL");
        if (ts[k]->cols != ts[0]->cols || ts[k]->device != ts[0]->device)
            return fail(ts[0], KORE_QMV_E_INVALID, "tensors of a group must share cols and device");
        if (int rc = check_dev_ptr(ts[0], outs[k], 4, "out")) return rc;
    }
    kore_qmv_tensor *t0 = ts[0];
    if (int rc = check_dev_ptr(t0, x, 16, "x")) return rc;
    PreOp pre{nullptr, 0.f, nullptr};
    if (opts) {
        if (opts->norm_w && opts->up) return fail(t0, KORE_QMV_E_INVALID, "rmsnorm and SwiGLU together");
        if (opts->norm_w && check_dev_ptr(t0, opts->norm_w, 16, "norm_w")) return KORE_QMV_E_INVALID;
        if (opts->up && check_dev_ptr(t0, opts->up, 16, "up")) return KORE_QMV_E_INVALID;
        pre = PreOp{opts->norm_w, opts->norm_eps, opts->up};
    }
    int64_t rows = 0;
    for (int k = 0; k < n; ++k) rows += ts[k]->rows;
    const int r = n == 1 ? t0->rows_per_wave : pick_rows_per_wave(rows, t0->nblk, t0->num_cu);
    int64_t wgs = 0;
    for (int k = 0; k < n; ++k) wgs += (ts[k]->rows + 4 * r - 1) / (4 * r);
    if (const int cap = max_workgroups(t0->num_cu)) wgs = std::min<int64_t>(wgs, cap);
    hipStream_t s = (hipStream_t)stream;
    if (fuse_quantisation(t0->nblk, wgs)) return launch_group(n, ts, nullptr, x, outs, avx2, s, false, opts);
    hipError_t e = launch_quantize_q8k(x, t0->cols, t0->xq, true, s, pre);
    if (e != hipSuccess) return hip_fail(t0, e, "quantize launch");
    return launch_group(n, ts, t0->xq, nullptr, outs, avx2, s, true, opts);
}

KORE_QMV_API int kore_qmv_mv_group_dev(int n, const kore_qmv_tensor_t *ts, const float *x, float *const *outs,
                                       int avx2, void *stream) {
    return kore_qmv_mv_group_ex_dev(n, ts, x, nullptr, outs, avx2, stream);
}

KORE_QMV_API int kore_qmv_mv_dev(kore_qmv_tensor_t t, const float *x, float *out, int avx2, void *stream) {
    return kore_qmv_mv_group_dev(1, &t, x, &out, avx2, stream);
}

static int matvec_host(kore_qmv_tensor_t t, const float *x, const void *xq, float *out, int avx2) {
    const size_t qb = (size_t)t->nblk * kQ8Bytes, ob = align256((size_t)t->rows * 4);
    const size_t xb = x ? align256((size_t)t->cols * 4) : 0;
    HostPath *h = nullptr;
    std::lock_guard<std::mutex> lock(g_host[t->device & 63].mu);
    QMV_TRY(t, host_path(t->device, ob + align256(qb) + xb, &h));
    uint8_t *dout = (uint8_t *)h->buf, *dq = dout + ob, *dx = dq + align256(qb);
    if (x) {
        QMV_TRY(t, hipMemcpyAsync(dx, x, (size_t)t->cols * 4, hipMemcpyHostToDevice, h->stream));
        float *o = (float *)dout;
        if (int rc = kore_qmv_mv_group_dev(1, &t, (const float *)dx, &o, avx2, h->stream)) return rc;
    } else {
        QMV_TRY(t, hipMemcpyAsync(dq, xq, qb, hipMemcpyHostToDevice, h->stream));
        if (int rc = launch_group(1, &t, dq, nullptr, (float *const *)&dout, avx2, h->stream)) return rc;
    }
    QMV_TRY(t, hipMemcpyAsync(out, dout, (size_t)t->rows * 4, hipMemcpyDeviceToHost, h->stream));
    QMV_TRY(t, hipStreamSynchronize(h->stream));
    return KORE_QMV_OK;
}

KORE_QMV_API int kore_qmv_matvec(kore_qmv_tensor_t t, const void *xq, float *out, int avx2) {
    if (!t) return fail(nullptr, KORE_QMV_E_INVALID, "tensor is NULL");
    if (!xq || !out) return fail(t, KORE_QMV_E_INVALID, "xq or out is NULL");
    int cur = -1;
    QMV_TRY(t, hipGetDevice(&cur));
    if (cur != t->device) QMV_TRY(t, hipSetDevice(t->device));
    const int rc = matvec_host(t, nullptr, xq, out, avx2);
    if (cur != t->device) (void)hipSetDevice(cur);
    return rc;
}

KORE_QMV_API int kore_qmv_mv(kore_qmv_tensor_t t, const float *x, float *out, int avx2) {
    if (!t) return fail(nullptr, KORE_QMV_E_INVALID, "tensor is NULL");
    if (!x || !out) return fail(t, KORE_QMV_E_INVALID, "x or out is NULL");
    int cur = -1;
    QMV_TRY(t, hipGetDevice(&cur));
    if (cur != t->device) QMV_TRY(t, hipSetDevice(t->device));
    const int rc = matvec_host(t, x, nullptr, out, avx2);
    if (cur != t->device) (void)hipSetDevice(cur);
    return rc;
}

namespace {

// The batched matmul of kore_qmv_matmul_batch_group_ex_dev, on x or (x16 set)
// on activations already split by kore_qmv_rmsnorm_rows_split_dev.
int matmul_group(int n, const kore_qmv_tensor_t *t, const float *x, const void *x16, int nb,
                 const kore_qmv_mv_opts *opts, float *const *out, void *stream, bool glu = false) {
    if (n < 1 || n > kMaxGroup || !t || !out) return fail(nullptr, KORE_QMV_E_INVALID, "n must be 1..4, t and out set");
    for (int k = 0; k < n; ++k)
        if (!t[k]) return fail(nullptr, KORE_QMV_E_INVALID, "tensor is NULL");
    kore_qmv_tensor *t0 = t[0];
    if (nb < 1 || nb > kGemmMaxB) return fail(t0, KORE_QMV_E_INVALID, "nb must be 1..64 (kore's KORE_BMAX)");
    if (opts && (opts->norm_w || opts->up))
        return fail(t0, KORE_QMV_E_INVALID, "the batched matmul takes bias and accumulate only (norm_w and up must be NULL)");
    for (int k = 0; opts && k < n; ++k)
        if (opts->bias[k])
            if (int rc = check_dev_ptr(t0, opts->bias[k], 4, "bias")) return rc;
    if (x16) {
        if (!gemm_fp16()) return fail(t0, KORE_QMV_E_UNSUPPORTED, "split activations need the fp16 matmul path");
        // a caller's split holds kore_qmv_split_bytes(cols) bytes: only tensors
        // whose cols have a split (at most 16 blocks) may read one
        if (kore_qmv_split_bytes(t0->cols) == 0)
            return fail(t0, KORE_QMV_E_UNSUPPORTED, "split activations exist only for cols 256..4096");
        if (int rc = check_dev_ptr(t0, x16, 16, "x16")) return rc;
    } else if (int rc = check_dev_ptr(t0, x, 16, "x")) {
        return rc;
    }
    GemmArgs a{};
    a.n_mat = n;
    a.x = x;
    a.B = nb;
    a.nblk = t0->nblk;
    for (int k = 0; k < n; ++k) {
        if (t[k]->device != t0->device || t[k]->cols != t0->cols)
            return fail(t0, KORE_QMV_E_INVALID, "grouped tensors must share device and cols");
        if (int rc = check_dev_ptr(t0, out[k], 4, "out")) return rc;
        a.m[k] = GemmMat{t[k]->w,        t[k]->wd,                      out[k],
                         (int)t[k]->rows, t[k]->type,                    a.tiles,
                         opts ? opts->bias[k] : nullptr, opts ? opts->accumulate : 0};
        a.tiles += row_tiles(t[k]->rows);
    }
    GemmScratch &g = g_gemm[t0->device & 63];
    bool q6 = false;
    for (int k = 0; k < n; ++k) q6 |= t[k]->type == KORE_QMV_Q6_K;
    a.glu = glu ? 1 : 0;
    a.halves = gemm_halves(a.tiles, a.nblk, nb, t0->num_cu);
    a.workers = gemm_workers(a.tiles * a.halves, a.nblk, nb, q6, t0->num_cu);
    a.partials = g.partials;
    a.x16 = x16 ? (uint8_t *)x16 : g.x16;
    a.presplit = x16 ? 1 : 0;
    hipError_t e = launch_gemm(a, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(t0, e, "matmul launch");
    return KORE_QMV_OK;
}

}  // namespace

KORE_QMV_API int kore_qmv_matmul_batch_group_ex_dev(int n, const kore_qmv_tensor_t *t, const float *x, int nb,
                                                    const kore_qmv_mv_opts *opts, float *const *out, void *stream) {
    return matmul_group(n, t, x, nullptr, nb, opts, out, stream);
}

KORE_QMV_API int kore_qmv_matmul_batch_group_split_dev(int n, const kore_qmv_tensor_t *t, const void *x16, int nb,
                                                       const kore_qmv_mv_opts *opts, float *const *out, void *stream) {
    if (!x16) return fail(nullptr, KORE_QMV_E_INVALID, "x16 is NULL");
    return matmul_group(n, t, nullptr, x16, nb, opts, out, stream);
}

KORE_QMV_API int kore_qmv_matmul_batch_glu_split_dev(const kore_qmv_tensor_t *gate_up, const void *x16, int nb,
                                                     float *out, float *tmp, void *stream) {
    if (!gate_up || !gate_up[0] || !gate_up[1] || !x16 || !out || !tmp)
        return fail(nullptr, KORE_QMV_E_INVALID, "gate_up[0..1], x16, out and tmp must be set");
    if (gate_up[0]->rows != gate_up[1]->rows)
        return fail(gate_up[0], KORE_QMV_E_INVALID, "gate and up must have the same rows");
    float *outs[2] = {out, tmp};
    return matmul_group(2, gate_up, nullptr, x16, nb, nullptr, outs, stream, true);
}

KORE_QMV_API size_t kore_qmv_split_bytes(int64_t cols) {
    if (!gemm_fp16() || cols < 256 || cols % 256 || cols > 16 * 256) return 0;
    return (size_t)(cols / 256) * kG16BlockBytes;
}

KORE_QMV_API int kore_qmv_rmsnorm_rows_split_dev(const float *x, const float *w, int64_t n, int rows, float eps,
                                                 float *out, void *x16, void *stream) {
    if (!x || !w || !out || !x16 || n < 1 || rows < 1)
        return fail(nullptr, KORE_QMV_E_INVALID, "x, w, out, x16 set, n >= 1 and rows >= 1 required");
    if (kore_qmv_split_bytes(n) == 0 || rows > kGemmMaxB)
        return fail(nullptr, KORE_QMV_E_UNSUPPORTED,
                    "split rows need the fp16 matmul path, n a multiple of 256 up to 4096 and rows <= 64");
    if (((uintptr_t)x | (uintptr_t)w | (uintptr_t)out | (uintptr_t)x16) & 15)
        return fail(nullptr, KORE_QMV_E_INVALID, "x, w, out and x16 must be 16-byte aligned");
    const hipError_t e = launch_rmsnorm_rows(x, w, (int)n, rows, eps, out, (hipStream_t)stream, (uint8_t *)x16);
    return e == hipSuccess ? KORE_QMV_OK : hip_fail(nullptr, e, "rmsnorm launch");
}

KORE_QMV_API int kore_qmv_matmul_batch_group_dev(int n, const kore_qmv_tensor_t *t, const float *x, int nb,
                                                 float *const *out, void *stream) {
    return kore_qmv_matmul_batch_group_ex_dev(n, t, x, nb, nullptr, out, stream);
}

KORE_QMV_API int kore_qmv_rmsnorm_rows_dev(const float *x, const float *w, int64_t n, int rows, float eps, float *out,
                                           void *stream) {
    if (!x || !w || !out || n < 1 || n > INT32_MAX || rows < 1)
        return fail(nullptr, KORE_QMV_E_INVALID, "x, w, out set, n >= 1 and rows >= 1 required");
    const hipError_t e = launch_rmsnorm_rows(x, w, (int)n, rows, eps, out, (hipStream_t)stream);
    return e == hipSuccess ? KORE_QMV_OK : hip_fail(nullptr, e, "rmsnorm launch");
}

KORE_QMV_API int kore_qmv_swiglu_dev(float *g, const float *u, int64_t n, void *stream) {
    if (!g || !u || n < 1) return fail(nullptr, KORE_QMV_E_INVALID, "g, u set and n >= 1 required");
    const hipError_t e = launch_swiglu(g, u, n, (hipStream_t)stream);
    return e == hipSuccess ? KORE_QMV_OK : hip_fail(nullptr, e, "swiglu launch");
}

KORE_QMV_API int kore_qmv_matmul_batch_dev(kore_qmv_tensor_t t, const float *x, int nb, float *out, void *stream) {
    if (!t) return fail(nullptr, KORE_QMV_E_INVALID, "tensor is NULL");
    return kore_qmv_matmul_batch_group_dev(1, &t, x, nb, &out, stream);
}

KORE_QMV_API int kore_qmv_matmul_batch(kore_qmv_tensor_t t, const float *x, int nb, float *out) {
    if (!t) return fail(nullptr, KORE_QMV_E_INVALID, "tensor is NULL");
    if (!x || !out) return fail(t, KORE_QMV_E_INVALID, "x or out is NULL");
    if (nb < 1 || nb > kGemmMaxB) return fail(t, KORE_QMV_E_INVALID, "nb must be 1..64 (kore's KORE_BMAX)");
    int cur = -1;
    QMV_TRY(t, hipGetDevice(&cur));
    if (cur != t->device) QMV_TRY(t, hipSetDevice(t->device));
    int rc = KORE_QMV_OK;
    {
        const size_t xb = align256((size_t)nb * t->cols * 4), ob = align256((size_t)nb * t->rows * 4);
        HostPath *h = nullptr;
        std::lock_guard<std::mutex> lock(g_host[t->device & 63].mu);
        hipError_t e = host_path(t->device, xb + ob, &h);
        if (e != hipSuccess) rc = hip_fail(t, e, "host staging");
        if (!rc) {
            float *dx = (float *)h->buf, *dout = (float *)((uint8_t *)h->buf + xb);
            if ((e = hipMemcpyAsync(dx, x, (size_t)nb * t->cols * 4, hipMemcpyHostToDevice, h->stream)) != hipSuccess)
                rc = hip_fail(t, e, "hipMemcpyAsync");
            if (!rc) rc = kore_qmv_matmul_batch_dev(t, dx, nb, dout, h->stream);
            if (!rc && (e = hipMemcpyAsync(out, dout, (size_t)nb * t->rows * 4, hipMemcpyDeviceToHost, h->stream)) != hipSuccess)
                rc = hip_fail(t, e, "hipMemcpyAsync");
            if (!rc && (e = hipStreamSynchronize(h->stream)) != hipSuccess) rc = hip_fail(t, e, "hipStreamSynchronize");
        }
    }
    if (cur != t->device) (void)hipSetDevice(cur);
    return rc;
}

KORE_QMV_API int kore_qmv_get_row_dev(int type, const void *table, int64_t row, int64_t n, float *out, void *stream) {
    if (!table || !out) return fail(nullptr, KORE_QMV_E_INVALID, "table or out is NULL");
    if (type != 0 && type != 1 && type != 30 && type != KORE_QMV_Q4_K && type != KORE_QMV_Q6_K)
        return fail(nullptr, KORE_QMV_E_UNSUPPORTED, "get_row takes F32, F16, BF16, Q4_K or Q6_K");
    const hipError_t e = launch_get_row(type, (const uint8_t *)table, row, n, out, (hipStream_t)stream);
    if (e != hipSuccess) return fail(nullptr, KORE_QMV_E_INVALID, std::string("get_row: ") + hipGetErrorString(e));
    return KORE_QMV_OK;
}

KORE_QMV_API const char *kore_qmv_last_error(kore_qmv_tensor_t t) {
    return t ? t->error.c_str() : g_error.c_str();
}

KORE_QMV_API int kore_qmv_get_info(kore_qmv_tensor_t t, kore_qmv_info *info) {
    if (!t || !info) return fail(t, KORE_QMV_E_INVALID, "tensor or info is NULL");
    info->type = t->type;
    info->device = t->device;
    info->rows = t->rows;
    info->cols = t->cols;
    info->weight_bytes = t->weight_bytes;
    info->rows_per_wave = t->rows_per_wave;
    return KORE_QMV_OK;
}

KORE_QMV_API int kore_qmv_synth_dev(int type, int64_t rows, int64_t cols, uint64_t seed, void *dst, void *stream) {
    if (type != KORE_QMV_Q4_K && type != KORE_QMV_Q6_K)
        return fail(nullptr, KORE_QMV_E_UNSUPPORTED, "weight type is not Q4_K (12) or Q6_K (14)");
    if (rows <= 0 || cols <= 0 || cols % 256 != 0)
        return fail(nullptr, KORE_QMV_E_INVALID, "rows must be > 0 and cols a positive multiple of 256");
    if (int rc = check_dev_ptr(nullptr, dst, 2, "dst")) return rc;
    hipError_t e = launch_synth_blocks(type, rows * (cols / 256), seed, (uint8_t *)dst, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(nullptr, e, "synth launch");
    return KORE_QMV_OK;
}

}  // extern "C"
