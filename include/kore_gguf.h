/* kore_gguf.h - kore's GGUF model loader (kore.cpp:188-285) with the weights
 * moved into HBM.
 *
 * kore maps the file and keeps pointers into the mapping (load_model): the
 * Qwen2 hyper-parameters from the metadata (qwen2.block_count,
 * embedding_length, feed_forward_length, attention.head_count(_kv),
 * context_length, rope.freq_base, attention.layer_norm_rms_epsilon, the vocab
 * size from the tokenizer.ggml.tokens array, general.alignment), and a table of
 * tensors by name (the first of a repeated name wins; a type kore does not
 * know has no bytes).  This parses the file by the same rules and rejects what
 * kore rejects (not GGUF, a read past the end, 0 or more than 4 dimensions, an
 * unknown metadata type or array, a tensor that leaves the file); then
 * kore_gguf_to_qmv / kore_gguf_to_device_f32 copy a tensor to the GPU, where
 * libkore_qmv and libkore_layer use it.  Part of libkore_layer.so. */
#ifndef KORE_GGUF_H
#define KORE_GGUF_H

#include <stdint.h>

#include "kore_qmv.h"

#ifdef __cplusplus
extern "C" {
#endif

#ifndef KORE_GGUF_API
#if defined(__GNUC__)
#define KORE_GGUF_API __attribute__((visibility("default")))
#else
#define KORE_GGUF_API
#endif
#endif

#define KORE_GGUF_OK 0
#define KORE_GGUF_E_IO 1           /* open / mmap failed */
#define KORE_GGUF_E_FORMAT 2       /* kore's load_model would return false */
#define KORE_GGUF_E_NOT_FOUND 3    /* no tensor of that name */
#define KORE_GGUF_E_TYPE 4         /* the tensor's type or shape does not fit the call */
#define KORE_GGUF_E_DEVICE 5       /* a HIP or libkore_qmv call failed */

typedef struct kore_gguf *kore_gguf_t;

/* kore's Hparams (kore.cpp:172-176; 0 where the file has no such key) and
 * what the parse found about the file. */
typedef struct kore_gguf_hparams {
    uint32_t n_layer, n_embd, n_ff, n_head, n_head_kv, n_ctx, n_vocab;
    float rope_base, rms_eps;
    uint32_t version;
    uint64_t alignment, data_start, file_size;
} kore_gguf_hparams;

/* kore's Tensor (kore.cpp:163-169): dims[0] is the contiguous dimension. */
typedef struct kore_gguf_tensor {
    const char *name;        /* valid until kore_gguf_close */
    uint32_t type, n_dims;
    uint64_t dims[4];
    uint64_t nbytes;         /* 0 for a type kore does not know */
    const uint8_t *data;     /* into the read-only mapping; NULL when nbytes is 0 */
} kore_gguf_tensor;

KORE_GGUF_API int kore_gguf_open(const char *path, kore_gguf_t *out);
KORE_GGUF_API void kore_gguf_close(kore_gguf_t g);
KORE_GGUF_API int kore_gguf_get_hparams(kore_gguf_t g, kore_gguf_hparams *hp);

/* Distinct tensor names, in the order of their first appearance in the file. */
KORE_GGUF_API int64_t kore_gguf_tensor_count(kore_gguf_t g);
KORE_GGUF_API int kore_gguf_tensor_at(kore_gguf_t g, int64_t i, kore_gguf_tensor *t);
KORE_GGUF_API int kore_gguf_find(kore_gguf_t g, const char *name, kore_gguf_tensor *t);

/* A Q4_K or Q6_K tensor as a libkore_qmv matrix on the current device: rows =
 * dims[1] * dims[2] * dims[3], cols = dims[0] (kore's matvec_mt, kore.cpp:677). */
KORE_GGUF_API int kore_gguf_to_qmv(kore_gguf_t g, const char *name, kore_qmv_tensor_t *out);

/* An F32 tensor (norms, biases) copied to a new device array of dims product
 * floats on the current device; release it with kore_gguf_free_device. */
KORE_GGUF_API int kore_gguf_to_device_f32(kore_gguf_t g, const char *name, float **dev);
KORE_GGUF_API void kore_gguf_free_device(void *dev);

/* Text of the last failure on this handle (or of the last failed open when g is
 * NULL, per thread).  Never NULL. */
KORE_GGUF_API const char *kore_gguf_last_error(kore_gguf_t g);

#ifdef __cplusplus
}
#endif

#endif
