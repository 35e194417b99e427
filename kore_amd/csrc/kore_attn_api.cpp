// kore_attn_api.cpp - host side of libkore_attn.so (C++20): the KV-cache
// handle, argument checks with kore's error behaviour, the RoPE table, and
// the staging of host buffers for the synchronous entry points.
#include "kore_attn.h"
#include "kore_attn_synth.h"
#include "kore_attn_kernels.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <vector>

using namespace kore_attn_gpu;

struct kore_attn {
    int n_layer = 0, ctx = 0, n_head = 0, n_head_kv = 0, head_dim = 0, window = 0;
    float rope_base = 0;
    int device = 0, num_cu = 0;
    hipStream_t stream = nullptr;
    float *d_k = nullptr, *d_v = nullptr;    // [layer][kv_head][slot][head_dim]
    float2 *d_cs = nullptr;                  // RoPE table [ctx][head_dim/2] (prefill, append)
    std::vector<float> inv_freq;
    RopeRow dec_cs{};                        // (cos, sin) of the last decode position
    int dec_cs_pos = -1;
    float *d_part_o = nullptr;               // decode split partials (o, then max/sum), then
                                             // the roped q of the generic decode
    int max_split = 0;
    size_t part_floats = 0;
    bool fast_decode = false, fast_prefill = false;   // MFMA kernels for this geometry
    float *d_pf_part = nullptr;              // prefill key-segment partials
    size_t pf_part_floats = 0;
    float *d_scratch = nullptr;              // the device's fixed scratch (allocation-free decode)
    float *h_stage = nullptr;                // pinned staging of the host entry points
    size_t h_stage_floats = 0;
    float *d_io = nullptr;                   // device copies of q/k/v/out
    size_t d_io_floats = 0;
    std::string err;

    size_t kv_dim() const { return (size_t)n_head_kv * head_dim; }
    size_t layer_floats() const { return (size_t)n_head_kv * ctx * head_dim; }
};

namespace {

thread_local std::string g_create_error;

int fail(kore_attn *h, int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (h) h->err = buf;
    else g_create_error = buf;
    return code;
}

int hip_fail(kore_attn *h, hipError_t e, const char *what) {
    return fail(h, KORE_ATTN_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define HIP_TRY(h, expr)                                        \
    do {                                                        \
        hipError_t e_ = (expr);                                 \
        if (e_ != hipSuccess) return hip_fail((h), e_, #expr);  \
    } while (0)

// kore.cpp:1337-1339 and 1405-1410: inv_freq in double rounded to float,
// angle pos * inv_freq in double, cos/sin in double rounded to float.
void fill_rope_rows(const std::vector<float> &inv_freq, int p0, int p1, std::vector<float2> &out) {
    const int half = (int)inv_freq.size();
    out.resize((size_t)(p1 - p0) * half);
    for (int p = p0; p < p1; ++p)
        for (int i = 0; i < half; ++i) {
            const double ang = (double)p * inv_freq[(size_t)i];
            out[(size_t)(p - p0) * half + i] = make_float2((float)std::cos(ang), (float)std::sin(ang));
        }
}

// The table of positions 0..ctx-1, built once at create: prefill and append
// never reach past ctx (kore.cpp:1490), and a decode takes its one row by
// value (decode_row), so nothing on a per-call path grows or reallocates it.
int build_rope_table(kore_attn *h) {
    const int half = h->head_dim / 2;
    std::vector<float2> rows;
    fill_rope_rows(h->inv_freq, 0, h->ctx, rows);
    HIP_TRY(h, hipMalloc(&h->d_cs, sizeof(float2) * (size_t)h->ctx * half));
    HIP_TRY(h, hipMemcpy(h->d_cs, rows.data(), sizeof(float2) * rows.size(), hipMemcpyHostToDevice));
    return KORE_ATTN_OK;
}

// (cos, sin) of one decode position (kore.cpp:1405-1410), kept for the next
// call: kore's layer loop decodes every layer at the same position.
const RopeRow &decode_row(kore_attn *h, int pos) {
    if (pos != h->dec_cs_pos) {
        const int half = h->head_dim / 2;
        for (int i = 0; i < half; ++i) {
            const double ang = (double)pos * h->inv_freq[(size_t)i];
            h->dec_cs.cs[2 * i] = (float)std::cos(ang);
            h->dec_cs.cs[2 * i + 1] = (float)std::sin(ang);
        }
        h->dec_cs_pos = pos;
    }
    return h->dec_cs;
}

int check_geometry(kore_attn *h, int n_head, int n_head_kv, int head_dim) {
    if (n_head != h->n_head || n_head_kv != h->n_head_kv || head_dim != h->head_dim)
        return fail(h, KORE_ATTN_E_INVALID,
                    "geometry %d/%d/%d differs from the handle's %d/%d/%d (n_head/n_head_kv/head_dim)",
                    n_head, n_head_kv, head_dim, h->n_head, h->n_head_kv, h->head_dim);
    return KORE_ATTN_OK;
}

int ensure_io(kore_attn *h, size_t floats) {
    if (floats > h->h_stage_floats) {
        if (h->h_stage) (void)hipHostFree(h->h_stage);
        h->h_stage = nullptr;
        h->h_stage_floats = 0;
        HIP_TRY(h, hipHostMalloc((void **)&h->h_stage, floats * sizeof(float), hipHostMallocDefault));
        h->h_stage_floats = floats;
    }
    if (floats > h->d_io_floats) {
        if (h->d_io) (void)hipFree(h->d_io);
        h->d_io = nullptr;
        h->d_io_floats = 0;
        HIP_TRY(h, hipMalloc(&h->d_io, floats * sizeof(float)));
        h->d_io_floats = floats;
    }
    return KORE_ATTN_OK;
}

// Largest number of decode splits any number of cache rows can need.
int decode_max_split(int head_dim, int max_rows, int n_head_kv, int num_cu) {
    int m = 1;
    for (int n = 1; n <= max_rows; ++n) {
        const int t = decode_rows_per_split(head_dim, n, n_head_kv, num_cu);
        m = std::max(m, (n + t - 1) / t);
    }
    return m;
}

void release(kore_attn *h) {
    if (!h) return;
    (void)hipSetDevice(h->device);
    if (h->stream) (void)hipStreamSynchronize(h->stream);
    if (h->d_k) (void)hipFree(h->d_k);
    if (h->d_v) (void)hipFree(h->d_v);
    if (h->d_cs) (void)hipFree(h->d_cs);
    if (h->d_part_o) (void)hipFree(h->d_part_o);
    if (h->d_pf_part) (void)hipFree(h->d_pf_part);
    if (h->d_io) (void)hipFree(h->d_io);
    if (h->h_stage) (void)hipHostFree(h->h_stage);
    if (h->stream) (void)hipStreamDestroy(h->stream);
    delete h;
}

hipStream_t pick_stream(kore_attn *h, void *stream) {
    return stream ? (hipStream_t)stream : h->stream;
}

// The decode of a geometry without an MFMA kernel: a prep launch ropes q
// (into part, after the partials) and appends the new row, then the split
// attention reads every row up to and including it.
int generic_decode_enqueue(kore_attn *h, int layer, int pos, const float *q, const float *k, const float *v,
                           float *out, hipStream_t s, float *part, size_t part_floats) {
    const bool wrapped = h->window && pos >= h->window;
    GenericArgs a{};
    a.kc = h->d_k + (size_t)layer * h->layer_floats();
    a.vc = h->d_v + (size_t)layer * h->layer_floats();
    a.out = out;
    a.slots = h->ctx;
    a.hd = h->head_dim;
    a.n_head_kv = h->n_head_kv;
    a.n_rep = h->n_head / h->n_head_kv;
    generic_shape(a.hd, a.n_rep, &a.tile, &a.chunk, &a.n_chunks);
    a.n_rows = wrapped ? h->window : pos + 1;
    a.rows_per_split = generic_rows_per_split(a.hd, a.n_rep, a.n_rows, a.n_head_kv, h->num_cu);
    a.n_split = (a.n_rows + a.rows_per_split - 1) / a.rows_per_split;
    a.scale = 1.0f / std::sqrt((float)h->head_dim);   // kore.cpp:1411
    const size_t np = (size_t)h->n_head * a.n_split, hd = (size_t)h->head_dim;
    const size_t need = np * (hd + 2) + (size_t)h->n_head * hd;
    if (need > part_floats)
        return fail(h, KORE_ATTN_E_UNSUPPORTED, "decode partials need %zu floats, the scratch holds %zu", need,
                    part_floats);
    a.part_o = part;
    a.part_ml = part + np * hd;
    float *q_roped = part + np * (hd + 2);
    a.q = q_roped;
    float *kc = h->d_k + (size_t)layer * h->layer_floats(), *vc = h->d_v + (size_t)layer * h->layer_floats();
    HIP_TRY(h, launch_generic_decode(a, q, k, v, q_roped, kc, vc, h->n_head, h->window ? pos % h->window : pos,
                                     decode_row(h, pos), s));
    return KORE_ATTN_OK;
}

// Enqueues a decode with its split partials in part (part_floats floats; a
// decode needs n_head * splits * (head_dim + 2), the generic one n_head *
// head_dim more).
int decode_enqueue(kore_attn *h, int layer, int pos, const float *q, const float *k, const float *v,
                   float *out, hipStream_t s, float *part, size_t part_floats) {
    // Cache rows read besides the new one: positions 0..pos-1 (kore.cpp:1437),
    // or every slot of a ring that has wrapped (the new slot's stale copy is
    // masked by the kernel).
    const bool wrapped = h->window && pos >= h->window;
    const int n_rows = wrapped ? h->window : pos;
    const int slot = h->window ? pos % h->window : pos;
    if (!h->fast_decode) return generic_decode_enqueue(h, layer, pos, q, k, v, out, s, part, part_floats);
    DecodeArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.kc = h->d_k + (size_t)layer * h->layer_floats();
    a.vc = h->d_v + (size_t)layer * h->layer_floats();
    a.out = out;
    a.slots = h->ctx;
    a.n_rows = n_rows;
    a.new_slot = slot;
    a.rows_per_split = decode_rows_per_split(h->head_dim, n_rows, h->n_head_kv, h->num_cu);
    a.n_split = std::max(1, (n_rows + a.rows_per_split - 1) / a.rows_per_split);
    a.n_head_kv = h->n_head_kv;
    a.n_rep = h->n_head / h->n_head_kv;
    a.scale = 1.0f / std::sqrt((float)h->head_dim);   // kore.cpp:1411
    a.wg_per_cu = a.n_split * a.n_head_kv > h->num_cu ? 2 : 1;
    if (a.n_split > h->max_split)
        return fail(h, KORE_ATTN_E_UNSUPPORTED, "decode needs %d splits, scratch holds %d", a.n_split,
                    h->max_split);
    const size_t np = (size_t)h->n_head * a.n_split;
    if (np * ((size_t)h->head_dim + 2) > part_floats)
        return fail(h, KORE_ATTN_E_UNSUPPORTED, "decode partials need %zu floats, the scratch holds %zu",
                    np * ((size_t)h->head_dim + 2), part_floats);
    a.part_o = part;
    a.part_ml = part + np * h->head_dim;
    HIP_TRY(h, launch_decode(a, decode_row(h, pos), h->head_dim, s));
    return KORE_ATTN_OK;
}

int prefill_enqueue(kore_attn *h, int layer, int pos0, int n_tok, const float *q, const float *k,
                    const float *v, float *out, hipStream_t s) {
    AppendArgs ap{};
    ap.k = k;
    ap.v = v;
    ap.cs = h->d_cs;
    ap.kc = h->d_k + (size_t)layer * h->layer_floats();
    ap.vc = h->d_v + (size_t)layer * h->layer_floats();
    ap.slots = h->ctx;
    ap.pos0 = pos0;
    ap.n_tok = n_tok;
    ap.n_head_kv = h->n_head_kv;
    HIP_TRY(h, launch_append(ap, h->head_dim, s));
    if (!h->fast_prefill) {
        GenericArgs ga{};
        ga.q = q;
        ga.cs = h->d_cs;
        ga.kc = ap.kc;
        ga.vc = ap.vc;
        ga.out = out;
        ga.slots = h->ctx;
        ga.hd = h->head_dim;
        ga.n_head_kv = h->n_head_kv;
        ga.n_rep = h->n_head / h->n_head_kv;
        generic_shape(ga.hd, ga.n_rep, &ga.tile, &ga.chunk, &ga.n_chunks);
        ga.pos0 = pos0;
        ga.n_split = 1;
        ga.scale = 1.0f / std::sqrt((float)h->head_dim);   // kore.cpp:1411
        HIP_TRY(h, launch_generic_prefill(ga, n_tok, s));
        return KORE_ATTN_OK;
    }
    PrefillArgs pa{};
    pa.q = q;
    pa.cs = h->d_cs;
    pa.kc = ap.kc;
    pa.vc = ap.vc;
    pa.out = out;
    pa.slots = h->ctx;
    pa.pos0 = pos0;
    pa.n_tok = n_tok;
    pa.n_head_kv = h->n_head_kv;
    pa.n_rep = h->n_head / h->n_head_kv;
    pa.n_strips = (n_tok + 31) / 32;
    pa.scale_log2 = (1.0f / std::sqrt((float)h->head_dim)) * 1.4426950408889634f;
    pa.n_kseg = prefill_key_segments(n_tok, pos0, h->n_head_kv, pa.n_rep, h->num_cu, &pa.seg_tiles);
    pa.fold = h->num_cu;
    if (pa.n_kseg > 1) {
        const size_t entries = (size_t)h->n_head_kv * pa.n_rep * pa.n_strips * pa.n_kseg * 32;
        const size_t need = entries * ((size_t)h->head_dim + 2);
        if (need > h->pf_part_floats)   // cannot happen: sized at create for the largest split
            return fail(h, KORE_ATTN_E_UNSUPPORTED, "prefill partials need %zu floats, scratch holds %zu", need,
                        h->pf_part_floats);
        pa.part_o = h->d_pf_part;
        pa.part_ml = h->d_pf_part + entries * h->head_dim;
    } else {
        prefill_split_plan(pa, h->num_cu);
        if (pa.n_split > 0) {
            // n_head_kv * n_split < num_cu items, 4 waves x 2 halves x 32 rows each
            const size_t entries = (size_t)h->n_head_kv * pa.n_split * 8 * 32;
            const size_t need = entries * ((size_t)h->head_dim + 2);
            if (need > h->pf_part_floats)   // cannot happen: sized at create for 8 x num_cu x 32 rows
                return fail(h, KORE_ATTN_E_UNSUPPORTED, "prefill partials need %zu floats, scratch holds %zu",
                            need, h->pf_part_floats);
            pa.part_o = h->d_pf_part;
            pa.part_ml = h->d_pf_part + entries * h->head_dim;
        }
    }
    HIP_TRY(h, launch_prefill(pa, h->head_dim, s));
    return KORE_ATTN_OK;
}

int check_decode(kore_attn *h, int layer, int pos, int n_head, int n_head_kv, int head_dim,
                 const void *q, const void *k, const void *v, const void *out) {
    if (int rc = check_geometry(h, n_head, n_head_kv, head_dim)) return rc;
    if (!q || !k || !v || !out) return fail(h, KORE_ATTN_E_INVALID, "null buffer");
    if (layer < 0 || layer >= h->n_layer)
        return fail(h, KORE_ATTN_E_INVALID, "layer %d outside [0, %d)", layer, h->n_layer);
    if (pos < 0 || (h->window == 0 && pos >= h->ctx))
        return fail(h, KORE_ATTN_E_RANGE, "position %d outside the cache (ctx %d)", pos, h->ctx);
    return KORE_ATTN_OK;
}

int check_prefill(kore_attn *h, int layer, int pos0, int n_tok, int n_head, int n_head_kv,
                  int head_dim, const void *q, const void *k, const void *v, const void *out) {
    if (int rc = check_geometry(h, n_head, n_head_kv, head_dim)) return rc;
    if (!q || !k || !v || !out) return fail(h, KORE_ATTN_E_INVALID, "null buffer");
    if (layer < 0 || layer >= h->n_layer)
        return fail(h, KORE_ATTN_E_INVALID, "layer %d outside [0, %d)", layer, h->n_layer);
    if (n_tok <= 0 || pos0 < 0 || (long)pos0 + n_tok > (long)h->ctx)
        return fail(h, KORE_ATTN_E_RANGE, "rows [%d, %d + %d) outside the cache (ctx %d)", pos0, pos0,
                    n_tok, h->ctx);
    return KORE_ATTN_OK;
}

}  // namespace

extern "C" {

int kore_attn_create(kore_attn_t *out, int n_layer, int ctx, int n_head, int n_head_kv, int head_dim,
                     float rope_base, int window) {
    if (!out) return fail(nullptr, KORE_ATTN_E_INVALID, "null handle pointer");
    *out = nullptr;
    if (n_layer <= 0 || ctx <= 0 || n_head <= 0 || n_head_kv <= 0 || head_dim <= 0)
        return fail(nullptr, KORE_ATTN_E_INVALID, "non-positive geometry");
    if (n_head % n_head_kv != 0)
        return fail(nullptr, KORE_ATTN_E_INVALID, "n_head %d not a multiple of n_head_kv %d", n_head,
                    n_head_kv);
    if (head_dim % 2 != 0) return fail(nullptr, KORE_ATTN_E_INVALID, "odd head_dim %d", head_dim);
    if (!(rope_base > 0) || !std::isfinite(rope_base))
        return fail(nullptr, KORE_ATTN_E_INVALID, "rope_base must be positive");
    if (window < 0 || (window > 0 && window != ctx))
        return fail(nullptr, KORE_ATTN_E_INVALID, "window must be 0 or equal to ctx");
    const int n_rep = n_head / n_head_kv;
    if (!generic_supported(head_dim))
        return fail(nullptr, KORE_ATTN_E_UNSUPPORTED, "no gfx950 kernel for head_dim %d (supported: even, up to %d)",
                    head_dim, kMaxGenericHeadDim);
    const double kv_bytes = 2.0 * n_layer * (double)n_head_kv * ctx * head_dim * 4.0;
    if (kv_bytes > 1e15) return fail(nullptr, KORE_ATTN_E_INVALID, "cache size overflows");

    kore_attn *h = new (std::nothrow) kore_attn;
    if (!h) return fail(nullptr, KORE_ATTN_E_NOMEM, "out of host memory");
    h->n_layer = n_layer;
    h->ctx = ctx;
    h->n_head = n_head;
    h->n_head_kv = n_head_kv;
    h->head_dim = head_dim;
    h->window = window;
    h->rope_base = rope_base;
    h->fast_decode = decode_supported(head_dim, n_rep);
    h->fast_prefill = prefill_supported(head_dim, n_rep);
    auto bail = [&](hipError_t e, const char *what) {
        g_create_error = std::string(what) + ": " + hipGetErrorString(e);
        release(h);
        return KORE_ATTN_E_HIP;
    };
    hipError_t e = hipGetDevice(&h->device);
    if (e != hipSuccess) return bail(e, "hipGetDevice");
    e = hipDeviceGetAttribute(&h->num_cu, hipDeviceAttributeMultiprocessorCount, h->device);
    if (e != hipSuccess) return bail(e, "hipDeviceGetAttribute");
    e = hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking);
    if (e != hipSuccess) return bail(e, "hipStreamCreate");
    const size_t kvb = (size_t)n_layer * h->layer_floats() * sizeof(float);
    e = hipMalloc(&h->d_k, kvb);
    if (e != hipSuccess) { g_create_error = "K cache allocation failed"; release(h); return KORE_ATTN_E_NOMEM; }
    e = hipMalloc(&h->d_v, kvb);
    if (e != hipSuccess) { g_create_error = "V cache allocation failed"; release(h); return KORE_ATTN_E_NOMEM; }
    // kore zero-fills its cache (kore.cpp:1344-1345)
    if ((e = hipMemsetAsync(h->d_k, 0, kvb, h->stream)) != hipSuccess) return bail(e, "hipMemset");
    if ((e = hipMemsetAsync(h->d_v, 0, kvb, h->stream)) != hipSuccess) return bail(e, "hipMemset");

    h->inv_freq.resize((size_t)head_dim / 2);
    for (int i = 0; i < head_dim / 2; ++i)   // kore.cpp:1339
        h->inv_freq[(size_t)i] = (float)std::pow((double)rope_base, -2.0 * i / head_dim);
    if (build_rope_table(h) != KORE_ATTN_OK) {
        g_create_error = h->err;
        release(h);
        return KORE_ATTN_E_HIP;
    }
    // Decode split partials: n_head * max_split * (hd + 2) floats, and the
    // roped q of the generic decode.
    h->max_split = h->fast_decode ? decode_max_split(head_dim, window ? window : ctx, n_head_kv, h->num_cu)
                                  : generic_max_split(head_dim, n_rep, n_head_kv, h->num_cu);
    const size_t np = (size_t)n_head * h->max_split;
    h->part_floats = np * ((size_t)head_dim + 2) + (h->fast_decode ? 0 : (size_t)n_head * head_dim);
    if ((e = hipMalloc(&h->d_part_o, h->part_floats * sizeof(float))) != hipSuccess)
        return bail(e, "hipMalloc");
    // Prefill key-segment partials, sized for the largest split any chunk
    // gets: segments are only used while a chunk has fewer workgroups than
    // CUs, which bounds (heads x strips x segments) by 8 x num_cu
    // (prefill_key_segments), i.e. 8 x num_cu x 32 rows of (hd + 2) floats;
    // a split plan (prefill_split_plan) halves fewer than num_cu items of 4
    // entries: under 8 x num_cu entries as well.
    if (h->fast_prefill) {
        h->pf_part_floats = (size_t)8 * h->num_cu * 32 * ((size_t)head_dim + 2);
        if ((e = hipMalloc(&h->d_pf_part, h->pf_part_floats * sizeof(float))) != hipSuccess)
            return bail(e, "hipMalloc");
    }
    // the device's fixed scratch of kore_attn_decode_noalloc_dev, resolved
    // once per device with that device current
    if ((e = static_scratch(h->device, &h->d_scratch)) != hipSuccess) return bail(e, "hipGetSymbolAddress");
    if ((e = hipStreamSynchronize(h->stream)) != hipSuccess) return bail(e, "hipStreamSynchronize");
    *out = h;
    return KORE_ATTN_OK;
}

void kore_attn_destroy(kore_attn_t h) { release(h); }

int kore_attn_decode_dev(kore_attn_t h, int layer, int pos, int n_head, int n_head_kv, int head_dim,
                         const float *q, const float *k, const float *v, float *out, void *stream) {
    if (!h) return fail(nullptr, KORE_ATTN_E_INVALID, "null handle");
    if (int rc = check_decode(h, layer, pos, n_head, n_head_kv, head_dim, q, k, v, out)) return rc;
    HIP_TRY(h, hipSetDevice(h->device));
    return decode_enqueue(h, layer, pos, q, k, v, out, pick_stream(h, stream), h->d_part_o, h->part_floats);
}

int kore_attn_decode_noalloc_dev(kore_attn_t h, int layer, int pos, int n_head, int n_head_kv, int head_dim,
                                 const float *q, const float *k, const float *v, float *out, void *stream) {
    if (!h) return fail(nullptr, KORE_ATTN_E_INVALID, "null handle");
    if (int rc = check_decode(h, layer, pos, n_head, n_head_kv, head_dim, q, k, v, out)) return rc;
    HIP_TRY(h, hipSetDevice(h->device));
    return decode_enqueue(h, layer, pos, q, k, v, out, pick_stream(h, stream), h->d_scratch,
                          kStaticScratchFloats);
}

int kore_attn_decode(kore_attn_t h, int layer, int pos, int n_head, int n_head_kv, int head_dim,
                     const float *q, const float *k, const float *v, float *out) {
    if (!h) return fail(nullptr, KORE_ATTN_E_INVALID, "null handle");
    if (int rc = check_decode(h, layer, pos, n_head, n_head_kv, head_dim, q, k, v, out)) return rc;
    HIP_TRY(h, hipSetDevice(h->device));
    const size_t E = (size_t)h->n_head * h->head_dim, kvd = h->kv_dim();
    if (int rc = ensure_io(h, 2 * E + 2 * kvd)) return rc;
    float *hs = h->h_stage, *ds = h->d_io;
    std::memcpy(hs, q, E * sizeof(float));
    std::memcpy(hs + E, k, kvd * sizeof(float));
    std::memcpy(hs + E + kvd, v, kvd * sizeof(float));
    HIP_TRY(h, hipMemcpyAsync(ds, hs, (E + 2 * kvd) * sizeof(float), hipMemcpyHostToDevice, h->stream));
    if (int rc = decode_enqueue(h, layer, pos, ds, ds + E, ds + E + kvd, ds + E + 2 * kvd, h->stream,
                                h->d_part_o, h->part_floats))
        return rc;
    HIP_TRY(h, hipMemcpyAsync(hs + E + 2 * kvd, ds + E + 2 * kvd, E * sizeof(float), hipMemcpyDeviceToHost,
                              h->stream));
    HIP_TRY(h, hipStreamSynchronize(h->stream));
    std::memcpy(out, hs + E + 2 * kvd, E * sizeof(float));
    return KORE_ATTN_OK;
}

int kore_attn_prefill_dev(kore_attn_t h, int layer, int pos0, int n_tok, int n_head, int n_head_kv,
                          int head_dim, const float *q, const float *k, const float *v, float *out,
                          void *stream) {
    if (!h) return fail(nullptr, KORE_ATTN_E_INVALID, "null handle");
    if (int rc = check_prefill(h, layer, pos0, n_tok, n_head, n_head_kv, head_dim, q, k, v, out)) return rc;
    HIP_TRY(h, hipSetDevice(h->device));
    return prefill_enqueue(h, layer, pos0, n_tok, q, k, v, out, pick_stream(h, stream));
}

int kore_attn_append_dev(kore_attn_t h, int layer, int pos0, int n_tok, const float *k, const float *v,
                         void *stream) {
    if (!h) return fail(nullptr, KORE_ATTN_E_INVALID, "null handle");
    if (!k || !v) return fail(h, KORE_ATTN_E_INVALID, "null buffer");
    if (layer < 0 || layer >= h->n_layer)
        return fail(h, KORE_ATTN_E_INVALID, "layer %d outside [0, %d)", layer, h->n_layer);
    if (n_tok <= 0 || pos0 < 0 || (long)pos0 + n_tok > (long)h->ctx)
        return fail(h, KORE_ATTN_E_RANGE, "rows [%d, %d + %d) outside the cache (ctx %d)", pos0, pos0,
                    n_tok, h->ctx);
    HIP_TRY(h, hipSetDevice(h->device));
    AppendArgs ap{};
    ap.k = k;
    ap.v = v;
    ap.cs = h->d_cs;
    ap.kc = h->d_k + (size_t)layer * h->layer_floats();
    ap.vc = h->d_v + (size_t)layer * h->layer_floats();
    ap.slots = h->ctx;
    ap.pos0 = pos0;
    ap.n_tok = n_tok;
    ap.n_head_kv = h->n_head_kv;
    HIP_TRY(h, launch_append(ap, h->head_dim, pick_stream(h, stream)));
    return KORE_ATTN_OK;
}

int kore_attn_prefill(kore_attn_t h, int layer, int pos0, int n_tok, int n_head, int n_head_kv,
                      int head_dim, const float *q, const float *k, const float *v, float *out) {
    if (!h) return fail(nullptr, KORE_ATTN_E_INVALID, "null handle");
    if (int rc = check_prefill(h, layer, pos0, n_tok, n_head, n_head_kv, head_dim, q, k, v, out)) return rc;
    HIP_TRY(h, hipSetDevice(h->device));
    const size_t E = (size_t)h->n_head * h->head_dim, kvd = h->kv_dim(), n = (size_t)n_tok;
    const size_t in_f = n * (E + 2 * kvd);
    if (int rc = ensure_io(h, in_f + n * E)) return rc;
    float *hs = h->h_stage, *ds = h->d_io;
    std::memcpy(hs, q, n * E * sizeof(float));
    std::memcpy(hs + n * E, k, n * kvd * sizeof(float));
    std::memcpy(hs + n * (E + kvd), v, n * kvd * sizeof(float));
    HIP_TRY(h, hipMemcpyAsync(ds, hs, in_f * sizeof(float), hipMemcpyHostToDevice, h->stream));
    if (int rc = prefill_enqueue(h, layer, pos0, n_tok, ds, ds + n * E, ds + n * (E + kvd), ds + in_f,
                                 h->stream))
        return rc;
    HIP_TRY(h, hipMemcpyAsync(hs + in_f, ds + in_f, n * E * sizeof(float), hipMemcpyDeviceToHost, h->stream));
    HIP_TRY(h, hipStreamSynchronize(h->stream));
    std::memcpy(out, hs + in_f, n * E * sizeof(float));
    return KORE_ATTN_OK;
}

int kore_attn_read_kv(kore_attn_t h, int layer, int pos0, int n, float *k_out, float *v_out) {
    if (!h) return fail(nullptr, KORE_ATTN_E_INVALID, "null handle");
    if (!k_out || !v_out) return fail(h, KORE_ATTN_E_INVALID, "null buffer");
    if (layer < 0 || layer >= h->n_layer)
        return fail(h, KORE_ATTN_E_INVALID, "layer %d outside [0, %d)", layer, h->n_layer);
    if (n <= 0 || pos0 < 0 || (h->window == 0 && (long)pos0 + n > (long)h->ctx) ||
        (h->window > 0 && n > h->window))
        return fail(h, KORE_ATTN_E_RANGE, "rows [%d, %d + %d) outside the cache (ctx %d)", pos0, pos0, n,
                    h->ctx);
    HIP_TRY(h, hipSetDevice(h->device));
    // _dev calls may have been enqueued on any stream of the device: wait
    // for all of them (this export is not on kore's per-token path)
    HIP_TRY(h, hipDeviceSynchronize());
    const size_t hd = (size_t)h->head_dim, kvd = h->kv_dim();
    for (int which = 0; which < 2; ++which) {
        const float *base = (which ? h->d_v : h->d_k) + (size_t)layer * h->layer_floats();
        float *dst = which ? v_out : k_out;
        int done = 0;
        while (done < n) {   // runs of consecutive slots (a ring wraps once at most per run)
            const int p = pos0 + done;
            const int slot = h->window ? p % h->window : p;
            const int run = std::min(n - done, h->ctx - slot);
            for (int g = 0; g < h->n_head_kv; ++g) {
                HIP_TRY(h, hipMemcpy2D(dst + (size_t)done * kvd + g * hd, kvd * sizeof(float),
                                       base + ((size_t)g * h->ctx + slot) * hd, hd * sizeof(float),
                                       hd * sizeof(float), (size_t)run, hipMemcpyDeviceToHost));
            }
            done += run;
        }
    }
    return KORE_ATTN_OK;
}

const char *kore_attn_last_error(kore_attn_t h) {
    return h ? h->err.c_str() : g_create_error.c_str();
}

int kore_attn_sync(kore_attn_t h) {
    if (!h) return fail(nullptr, KORE_ATTN_E_INVALID, "null handle");
    HIP_TRY(h, hipSetDevice(h->device));
    HIP_TRY(h, hipStreamSynchronize(h->stream));
    return KORE_ATTN_OK;
}

int kore_attn_get_info(kore_attn_t h, kore_attn_info *info) {
    if (!h || !info) return fail(h, KORE_ATTN_E_INVALID, "null argument");
    info->n_layer = h->n_layer;
    info->ctx = h->ctx;
    info->n_head = h->n_head;
    info->n_head_kv = h->n_head_kv;
    info->head_dim = h->head_dim;
    info->window = h->window;
    info->device = h->device;
    info->num_cu = h->num_cu;
    info->kv_bytes = 2 * (size_t)h->n_layer * h->layer_floats() * sizeof(float);
    info->stream = (void *)h->stream;
    return KORE_ATTN_OK;
}

int kore_attn_synth_dev(float *dst, int rows, int dim, uint64_t seed, uint64_t stream_id, uint64_t row0,
                        uint64_t tensor, uint32_t per_mille, float outlier_scale, void *stream) {
    if (!dst || rows < 0 || dim < 0) return fail(nullptr, KORE_ATTN_E_INVALID, "bad synth arguments");
    SynthArgs a{};
    a.dst = dst;
    a.rows = rows;
    a.dim = dim;
    a.seed = seed;
    a.stream = stream_id;
    a.row0 = row0;
    a.tensor = tensor;
    a.per_mille = per_mille;
    a.outlier_scale = outlier_scale;
    hipError_t e = launch_synth(a, (hipStream_t)stream);
    if (e != hipSuccess) return fail(nullptr, KORE_ATTN_E_HIP, "synth launch: %s", hipGetErrorString(e));
    return KORE_ATTN_OK;
}

}  // extern "C"
