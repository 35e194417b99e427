/* kore_layer.h - one layer of kore's forward() on an MI355X (gfx950), with the
 * residual stream, the activations and the KV cache resident in HBM.
 *
 * Replaces the body of kore's per-layer loop in forward() (kore.cpp:1415-1472,
 * the quantised path): rmsnorm -> quant -> q/k/v matvecs -> biases -> RoPE ->
 * append -> attention -> quant -> Wo -> x += o -> rmsnorm -> quant -> gate/up ->
 * SwiGLU -> quant -> down -> x += o, in five launches of libkore_qmv and the two
 * of libkore_attn's decode:
 *   1. rmsnorm (attn_norm), Q8_K quantisation and the wq/wk/wv matvecs with their
 *      biases in one launch (kore_qmv_mv_group_ex_dev);
 *   2. RoPE, the KV append and attention (kore_attn_decode_dev);
 *   3. quantisation of the attention rows and Wo, added into x;
 *   4. rmsnorm (ffn_norm), quantisation and the w_gate/w_up matvecs;
 *   5. SwiGLU and quantisation of the down input, then w_down added into x.
 * Every step is kore's arithmetic; all but attention's softmax and SwiGLU's exp
 * are bit-identical to kore's, those two hold to kore's tolerance (see
 * kore_attn.h, kore_qmv.h), so a layer's result agrees with kore's to that
 * tolerance.
 *
 * Link with -lkore_layer -lkore_qmv -lkore_attn.  No CPU fallback. */
#ifndef KORE_LAYER_H
#define KORE_LAYER_H

#include "kore_attn.h"
#include "kore_qmv.h"

#ifdef __cplusplus
extern "C" {
#endif

#ifndef KORE_LAYER_API
#if defined(__GNUC__)
#define KORE_LAYER_API __attribute__((visibility("default")))
#else
#define KORE_LAYER_API
#endif
#endif

#define KORE_LAYER_OK 0
#define KORE_LAYER_E_INVALID 1     /* bad geometry, pointer or tensor shape */
#define KORE_LAYER_E_HIP 2         /* a HIP call failed */
#define KORE_LAYER_E_STEP 3        /* a matvec or attention step failed (its library's error text) */

/* A layer's weights as kore's Layer holds them (kore.cpp:1246-1250): the seven
 * matrices as libkore_qmv tensors (Q4_K / Q6_K, rows x cols as in the GGUF:
 * wq E x E, wk/wv kv_dim x E, wo E x E, w_gate/w_up n_ff x E, w_down E x n_ff),
 * and device arrays: attn_norm, ffn_norm (E floats, 16-byte aligned), biases
 * bq (E), bk, bv (kv_dim), each NULL for a layer without it. */
typedef struct kore_layer_weights {
    kore_qmv_tensor_t wq, wk, wv, wo, w_gate, w_up, w_down;
    const float *attn_norm, *ffn_norm;
    const float *bq, *bk, *bv;
} kore_layer_weights;

typedef struct kore_layer *kore_layer_t;

/* Geometry (kore's Hparams, kore.cpp:172-176) and the device scratch of one
 * layer step: q, k, v, attention rows, gate, up (all on the current device). */
KORE_LAYER_API int kore_layer_create(kore_layer_t *out, int n_embd, int n_ff, int n_head, int n_head_kv,
                                     float rms_eps);
KORE_LAYER_API void kore_layer_destroy(kore_layer_t L);

/* kore's forward() body for layer `layer` at position `pos` (kore.cpp:1415-1472):
 * x (device, n_embd floats, 16-byte aligned) is the residual stream, updated in
 * place; attn holds the KV cache (created with the same n_head, n_head_kv and
 * head_dim = n_embd / n_head).  avx2 selects kore's matvec summation order.
 * Enqueued on `stream` (NULL: the layer's own stream, which is ordered with the
 * null stream like any stream created without flags); every launch goes to that
 * one stream.  Calls that overlap on one layer handle race on its scratch. */
KORE_LAYER_API int kore_layer_decode_dev(kore_layer_t L, const kore_layer_weights *w, kore_attn_t attn, int layer,
                                         int pos, float *x, int avx2, void *stream);

/* kore's forward_batch() body for layer `layer` over n_tok (1..64, kore's
 * KORE_BMAX) rows at positions pos0.. (kore.cpp:1518-1589): x (device,
 * [n_tok][n_embd], 16-byte aligned) is the rows' residual stream, updated in
 * place.  Batched rmsnorm, q/k/v matmul + biases, RoPE + append + causal
 * attention (kore_attn_prefill_dev), Wo + residual, rmsnorm, gate/up matmul,
 * SwiGLU, down + residual.  rmsnorm is bit-identical to kore's; the matmuls
 * and attention hold kore's tolerance (max|d| <= 1e-4 * max|ref|).  Fails
 * with KORE_LAYER_E_STEP (attention's range error) when pos0 < 0 or pos0 +
 * n_tok > ctx, like forward_batch() (kore.cpp:1490).  Same stream and scratch
 * rules as kore_layer_decode_dev. */
KORE_LAYER_API int kore_layer_prefill_dev(kore_layer_t L, const kore_layer_weights *w, kore_attn_t attn, int layer,
                                          int pos0, int n_tok, float *x, void *stream);

/* Wait for the layer's own stream. */
KORE_LAYER_API int kore_layer_sync(kore_layer_t L);

/* Text of the last failure on this handle (or of the last failed create when L
 * is NULL, per thread).  Never NULL. */
KORE_LAYER_API const char *kore_layer_last_error(kore_layer_t L);

#ifdef __cplusplus
}
#endif

#endif
