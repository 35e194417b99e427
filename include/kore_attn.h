/*
 * kore_attn.h - C ABI of the MI355X (gfx950) attention path for kore.
 *
 * kore has no attention function: RoPE, KV-cache append and attention are
 * inline in forward() (decode, kore.cpp:1405-1455) and forward_batch()
 * (prefill, kore.cpp:1503-1563), over the Engine's kcache/vcache
 * (kore.cpp:1260).  These entry points are cut at exactly the inputs and
 * outputs of those blocks, so a kore build can replace the blocks with one
 * call each and leave the matvec, tokenizer and servers untouched:
 *
 *   inputs   q, k, v after the bias add and before RoPE (kore.cpp:1422-1423,
 *            1533-1534), the layer index, the position (or first position and
 *            row count), the head geometry, a KV-cache handle;
 *   outputs  the attention rows kore leaves in e.att / e.batt and feeds to
 *            Wo (kore.cpp:1456-1457, 1566); the K/V rows appended to the
 *            cache, bit-identical to kore's.
 *
 * Conventions
 *   - 0 on success, a negative KORE_ATTN_E_* code otherwise; nothing throws
 *     across the ABI.  kore_attn_last_error() describes the last failure.
 *   - The host-pointer calls are synchronous like kore's loops: `out` is
 *     valid on return.  The caller owns every buffer it passes.
 *   - A handle owns the device K/V cache (zero-initialised, kore.cpp:1344),
 *     the RoPE table and scratch.  One thread at a time per handle; calls
 *     may come from different threads in turn (kore's web server serialises
 *     them with a mutex, kore.cpp:2512, 2600).  Several handles may coexist
 *     (kore keeps a second Engine for embeddings, kore.cpp:2513-2519).
 *   - Arithmetic: fp32.  K/V cache rows equal kore's bit for bit; attention
 *     outputs agree with kore's to max|d| <= 1e-4 * max|ref|.
 */
#ifndef KORE_ATTN_H
#define KORE_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifndef KORE_ATTN_API
#if defined(__GNUC__) || defined(__clang__)
#define KORE_ATTN_API __attribute__((visibility("default")))
#else
#define KORE_ATTN_API
#endif
#endif

#ifdef __cplusplus
extern "C" {
#endif

typedef struct kore_attn *kore_attn_t;

enum {
    KORE_ATTN_OK = 0,
    KORE_ATTN_E_INVALID = -1,      /* null pointer, bad layer, geometry mismatch  */
    KORE_ATTN_E_RANGE = -2,        /* position outside the cache: kore's forward()
                                      / forward_batch() return false here
                                      (kore.cpp:1400, 1490)                       */
    KORE_ATTN_E_UNSUPPORTED = -3,  /* geometry with no GPU kernel                  */
    KORE_ATTN_E_HIP = -4,          /* HIP runtime failure (no device, launch)      */
    KORE_ATTN_E_NOMEM = -5         /* device or host allocation failed             */
};

/* Create a KV-cache handle on the current HIP device.
 * Replaces Engine's cache/RoPE set-up in engine_init (kore.cpp:1287-1291,
 * 1337-1345): head_dim is even, n_head % n_head_kv == 0, rope_base > 0
 * (kore.cpp:1278-1288).  Every such geometry with head_dim <= 256 runs on the
 * GPU (head_dim 64 or 128 with at most 8 q-heads per kv-head on the MFMA
 * kernels, the rest on generic tiled kernels); a larger head_dim fails with
 * KORE_ATTN_E_UNSUPPORTED.  ctx is the number of positions per layer.
 * window = 0 keeps kore's semantics (a position must be < ctx).  window > 0
 * (must equal ctx) makes each layer a ring of `window` slots: position p is
 * stored in slot p % window and a decode at p >= window attends the last
 * `window` positions; a prefill must still end at or before `window`.
 * kore has no sliding window; this mode is an extension. */
KORE_ATTN_API int kore_attn_create(kore_attn_t *out, int n_layer, int ctx, int n_head, int n_head_kv,
                     int head_dim, float rope_base, int window);

/* Release the handle and its device memory (Engine destruction). */
KORE_ATTN_API void kore_attn_destroy(kore_attn_t h);

/* Single-token decode of one layer; replaces kore.cpp:1405-1455 (cos/sin of
 * pos, RoPE of q and k, append of k and v at pos, scalar GQA attention).
 *   q [n_head*head_dim], k/v [n_head_kv*head_dim]: post-bias, pre-RoPE.
 *   out [n_head*head_dim]: kore's e.att.
 * Fails with KORE_ATTN_E_RANGE when pos < 0 or (window == 0) pos >= ctx,
 * like forward() (kore.cpp:1400). */
KORE_ATTN_API int kore_attn_decode(kore_attn_t h, int layer, int pos, int n_head, int n_head_kv, int head_dim,
                     const float *q, const float *k, const float *v, float *out);

/* Batched causal prefill of n_tok rows at positions pos0..pos0+n_tok-1 of one
 * layer; replaces kore.cpp:1503-1563 (RoPE + append of every row, then
 * attention of row z over positions 0..pos0+z).  kore feeds at most 64 rows
 * (kore.cpp:690, 1490); any n_tok works here and gives the same rows.
 *   q [n_tok][n_head*head_dim], k/v [n_tok][n_head_kv*head_dim]: pre-RoPE.
 *   out [n_tok][n_head*head_dim]: kore's e.batt.
 * Fails with KORE_ATTN_E_RANGE when n_tok <= 0, pos0 < 0 or
 * pos0 + n_tok > ctx (kore.cpp:1490). */
KORE_ATTN_API int kore_attn_prefill(kore_attn_t h, int layer, int pos0, int n_tok, int n_head, int n_head_kv,
                      int head_dim, const float *q, const float *k, const float *v, float *out);

/* Copy n cache rows starting at position pos0 of one layer to the host in
 * kore's layout [n][n_head_kv*head_dim] (kore.cpp:1427-1428).  In window
 * mode positions map to slots p % window. */
KORE_ATTN_API int kore_attn_read_kv(kore_attn_t h, int layer, int pos0, int n, float *k_out, float *v_out);

/* Text of the last failure on this handle (or of the last failed create when
 * h is NULL, per thread).  Never NULL. */
KORE_ATTN_API const char *kore_attn_last_error(kore_attn_t h);

/* ---- device-pointer variants ---------------------------------------------
 * Same semantics with every buffer in device memory of the handle's device,
 * enqueued on `stream` (a hipStream_t; NULL = the handle's own stream) and
 * asynchronous: the result is ready when the stream reaches it.  Calls that
 * overlap on different streams of one handle race on its scratch. */
KORE_ATTN_API int kore_attn_decode_dev(kore_attn_t h, int layer, int pos, int n_head, int n_head_kv,
                         int head_dim, const float *q, const float *k, const float *v,
                         float *out, void *stream);
KORE_ATTN_API int kore_attn_prefill_dev(kore_attn_t h, int layer, int pos0, int n_tok, int n_head,
                          int n_head_kv, int head_dim, const float *q, const float *k,
                          const float *v, float *out, void *stream);

/* kore_attn_decode_dev with its split partials in a fixed device array of
 * the library (655,360 floats = 2.5 MiB per GPU, held until the process
 * ends) instead of the handle's scratch: after kore_attn_create, the call
 * allocates nothing, synchronises nothing and calls no allocating routine.
 * No counterpart in kore; it is for callers that cannot allocate (HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  A decode
 * needs n_head x splits x (head_dim + 2) floats, on the MFMA kernels at most
 * 16 x CUs x 130 (532,480 on a 256-CU MI355X), on the generic kernels
 * n_head x head_dim more; a larger need fails with KORE_ATTN_E_UNSUPPORTED.  Every call on one GPU shares the array (each call
 * writes every partial it reads, so nothing carries over): calls that overlap
 * on one GPU (other streams, other handles) race. */
KORE_ATTN_API int kore_attn_decode_noalloc_dev(kore_attn_t h, int layer, int pos, int n_head, int n_head_kv,
                         int head_dim, const float *q, const float *k, const float *v,
                         float *out, void *stream);

/* RoPE + append of n_tok rows at positions pos0.. of one layer, without
 * attention: the cache-row half of kore_attn_prefill_dev (kore.cpp:1535-1538).
 * kore has no counterpart (its forward_batch() always attends); it is for
 * restoring a cache from saved pre-RoPE k/v rows or filling one for a long
 * context.  k/v: device [n_tok][n_head_kv*head_dim].  Same range rules as
 * kore_attn_prefill. */
KORE_ATTN_API int kore_attn_append_dev(kore_attn_t h, int layer, int pos0, int n_tok, const float *k,
                         const float *v, void *stream);

/* Wait for all work enqueued on the handle's own stream. */
KORE_ATTN_API int kore_attn_sync(kore_attn_t h);

/* Geometry and resources of a handle. */
typedef struct kore_attn_info {
    int n_layer, ctx, n_head, n_head_kv, head_dim, window;
    int device;             /* HIP device ordinal                      */
    int num_cu;             /* compute units of that device            */
    size_t kv_bytes;        /* device bytes of the K and V caches      */
    void *stream;           /* the handle's own hipStream_t            */
} kore_attn_info;
KORE_ATTN_API int kore_attn_get_info(kore_attn_t h, kore_attn_info *info);

#ifdef __cplusplus
}
#endif
#endif
