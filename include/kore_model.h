/* kore_model.h - a whole kore engine on an MI355X: kore's engine_init
 * (kore.cpp:1274-1365) over a GGUF file with every tensor in HBM, and its
 * forward() (kore.cpp:1397-1484) for one token on the GPU: the token's
 * embedding row (kore_qmv_get_row_dev), every layer (kore_layer_decode_dev)
 * and, when asked, the logits (rmsnorm with output_norm, quant, output head).
 *
 * Loading applies engine_init's checks (Qwen2 hyper-parameters present and
 * consistent, n_embd and n_ff multiples of 256, even head_dim, matrices Q4_K or
 * Q6_K, norms and biases F32, token_embd and output with the same vocabulary)
 * and its context: min(qwen2.context_length, ctx_max), or ctx_max when the file
 * has none.  Beyond kore, it refuses (KORE_MODEL_E_LOAD, before anything reaches
 * the device) a file whose tensors do not have the shapes the forward pass
 * reads: matrices [n_embd x n_embd], [kv_dim x n_embd], [n_ff x n_embd],
 * [n_embd x n_ff], token_embd and output.weight n_embd wide and 2-D, every norm
 * and attn_q.bias n_embd floats, attn_k.bias and attn_v.bias kv_dim floats.
 * The matvecs sum in the order kore's engine_init picks (e.avx2,
 * kore.cpp:1293): its AVX2 order on a host with AVX2 and FMA, its scalar order
 * elsewhere; kore_model_load_ex sets either.  Part of libkore_layer.so. */
#ifndef KORE_MODEL_H
#define KORE_MODEL_H

#include "kore_attn.h"
#include "kore_gguf.h"

#ifdef __cplusplus
extern "C" {
#endif

#ifndef KORE_MODEL_API
#if defined(__GNUC__)
#define KORE_MODEL_API __attribute__((visibility("default")))
#else
#define KORE_MODEL_API
#endif
#endif

#define KORE_MODEL_OK 0
#define KORE_MODEL_E_LOAD 1        /* the file: kore_gguf_open failed, or engine_init would refuse it */
#define KORE_MODEL_E_RANGE 2       /* token or position outside what forward() accepts (kore.cpp:1400) */
#define KORE_MODEL_E_DEVICE 3      /* a HIP call or a device step failed */

typedef struct kore_model *kore_model_t;

typedef struct kore_model_info {
    kore_gguf_hparams hp;
    int ctx;                 /* positions per layer of the KV cache */
    int n_vocab;             /* rows of output.weight */
    int head_dim, kv_dim;
    size_t weight_bytes;     /* device bytes of all tensors */
    int avx2;                /* 1: the matvecs sum in kore's AVX2 order, 0: its scalar order */
} kore_model_info;

/* engine_init(e, path, ctx_max) with the matvec order kore would pick on this
 * host: e.avx2 = KORE_HAVE_AVX2 && cpu_has_avx2() (kore.cpp:1293, 512-519). */
KORE_MODEL_API int kore_model_load(const char *gguf_path, int ctx_max, kore_model_t *out);

/* The same with e.avx2 given: 1 kore's AVX2 order (kore.cpp:521-632), 0 its
 * scalar order (kore.cpp:450-506), -1 kore's own choice on this host (as
 * kore_model_load); any other value is KORE_MODEL_E_LOAD. */
KORE_MODEL_API int kore_model_load_ex(const char *gguf_path, int ctx_max, int avx2, kore_model_t *out);
KORE_MODEL_API void kore_model_destroy(kore_model_t m);
KORE_MODEL_API int kore_model_get_info(kore_model_t m, kore_model_info *info);

/* kore's forward(e, token, pos, want_logits) with the result in HBM: the logits
 * (n_vocab floats) at kore_model_logits_dev when want_logits.  Enqueued on
 * `stream` (NULL: the model's own stream, ordered with the null stream). */
KORE_MODEL_API int kore_model_decode_dev(kore_model_t m, int token, int pos, int want_logits, void *stream);
KORE_MODEL_API const float *kore_model_logits_dev(kore_model_t m);

/* kore's forward_batch(e, tokens, n_tok, pos0, want_logits) (kore.cpp:1486-1598)
 * with the results in HBM: tokens is host memory; 1 <= n_tok <= min(64, ctx)
 * (kore's e.bsz) and pos0 + n_tok <= ctx, every token < n_vocab, else
 * KORE_MODEL_E_RANGE.  The rows' residual streams after the last layer are at
 * kore_model_rows_dev ([n_tok][n_embd], kore's e.bx) and, when want_logits,
 * the last row's logits at kore_model_logits_dev.  Matmuls and attention hold
 * kore's tolerance (max|d| <= 1e-4 * max|ref|); not bit for bit. */
KORE_MODEL_API int kore_model_prefill_dev(kore_model_t m, const int *tokens, int n_tok, int pos0, int want_logits,
                                          void *stream);
KORE_MODEL_API const float *kore_model_rows_dev(kore_model_t m);

/* Waits for the model's own stream. */
KORE_MODEL_API int kore_model_sync(kore_model_t m);

/* Same, synchronous, with the logits copied to host memory (NULL: no logits). */
KORE_MODEL_API int kore_model_decode(kore_model_t m, int token, int pos, float *logits);

/* The model's KV cache (for kore_attn_read_kv and the like). */
KORE_MODEL_API kore_attn_t kore_model_attn(kore_model_t m);

KORE_MODEL_API const char *kore_model_last_error(kore_model_t m);

#ifdef __cplusplus
}
#endif

#endif
