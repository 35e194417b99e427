/*
 * kore_qmv.h - C ABI of the MI355X (gfx950) quantised matrix-vector product
 * for kore: the Q8_K activation quantiser and the Q4_K / Q6_K x Q8_K row dot
 * products that every weight matrix of kore's forward() goes through.
 *
 * kore's calls this replaces:
 *   quant(e, x, xq, n)        -> quantize_row_q8_K   (kore.cpp:1392-1394, 422-446)
 *   mv(e, t, x, xq, out)      -> matvec_mt / matvec_rows with
 *                                dot_q4_K_q8_K_* / dot_q6_K_q8_K_*
 *                                (kore.cpp:1387-1390, 649-682, 450-632)
 * A weight matrix is uploaded once (kore keeps it in the mmap'ed GGUF file,
 * Tensor::data); the activations and results move per call.
 *
 * Results are bit-identical to kore's on the same inputs, in either of
 * kore's two summation orders: `avx2` = 1 reproduces dot_*_avx2 (what kore
 * runs on a CPU with AVX2/FMA, kore.cpp:535-632), `avx2` = 0 the scalar
 * reference dot_*_ref (kore.cpp:450-506).  The Q8_K blocks are kore's
 * BlockQ8K records (292 bytes: float d, int8 qs[256], int16 bsums[16];
 * kore.cpp:415-420), bit for bit.
 *
 * Conventions (as kore_attn.h): 0 on success, a negative KORE_QMV_E_* code
 * otherwise; nothing throws across the ABI; kore_qmv_last_error() describes
 * the last failure.  Host-pointer calls are synchronous; *_dev calls take
 * device pointers on the tensor's device and are asynchronous on `stream`
 * (a hipStream_t; NULL = the null stream).
 */
#ifndef KORE_QMV_H
#define KORE_QMV_H

#include <stddef.h>
#include <stdint.h>

#ifndef KORE_QMV_API
#if defined(__GNUC__) || defined(__clang__)
#define KORE_QMV_API __attribute__((visibility("default")))
#else
#define KORE_QMV_API
#endif
#endif

#ifdef __cplusplus
extern "C" {
#endif

typedef struct kore_qmv_tensor *kore_qmv_tensor_t;

/* ggml type ids kore accepts in a matvec (kore.cpp:161, 650) */
enum { KORE_QMV_Q4_K = 12, KORE_QMV_Q6_K = 14 };

#define KORE_QMV_Q8K_BYTES 292   /* one BlockQ8K per 256 values */

enum {
    KORE_QMV_OK = 0,
    KORE_QMV_E_INVALID = -1,      /* null pointer, cols not a multiple of 256, size
                                     mismatch, misaligned device pointer        */
    KORE_QMV_E_UNSUPPORTED = -3,  /* weight type other than Q4_K / Q6_K: kore's
                                     matvec_rows() returns false (kore.cpp:650),
                                     or cols above 32768                         */
    KORE_QMV_E_HIP = -4,          /* HIP runtime failure                         */
    KORE_QMV_E_NOMEM = -5         /* device or host allocation failed            */
};

/* Upload one weight matrix to the current HIP device.  `data` holds kore's
 * Tensor::data for it: rows x (cols/256) blocks of 144 (Q4_K) or 210 (Q6_K)
 * bytes, row-major (kore.cpp:652: rows of cols/256 blocks; kore's dims[0] is
 * cols, dims[1]*dims[2]*dims[3] rows).  data_on_device = 1 when `data` is a
 * device pointer (then it must be 2-byte aligned).  The library keeps its own
 * copy (Q6_K blocks are stored split so every load is aligned). */
KORE_QMV_API int kore_qmv_tensor_create(kore_qmv_tensor_t *out, int type, int64_t rows, int64_t cols,
                                        const void *data, int data_on_device);

/* Release a matrix. */
KORE_QMV_API void kore_qmv_tensor_destroy(kore_qmv_tensor_t t);

/* quantize_row_q8_K (kore.cpp:422-446): x[n] (n a multiple of 256) ->
 * n/256 BlockQ8K records in xq.  Host buffers; runs on the current device. */
KORE_QMV_API int kore_qmv_quantize(const float *x, int64_t n, void *xq);

/* Same with device buffers on the current device; x and xq 16-byte aligned. */
KORE_QMV_API int kore_qmv_quantize_dev(const float *x, int64_t n, void *xq, void *stream);

/* out[r] = row r . xq for every row (matvec_mt, kore.cpp:677-682); xq holds
 * cols/256 BlockQ8K records.  Host buffers. */
KORE_QMV_API int kore_qmv_matvec(kore_qmv_tensor_t t, const void *xq, float *out, int avx2);

/* Same with device buffers on the tensor's device; xq 16-byte aligned. */
KORE_QMV_API int kore_qmv_matvec_dev(kore_qmv_tensor_t t, const void *xq, float *out, int avx2,
                                     void *stream);

/* mv() with quant() in front (kore.cpp:1387-1394): x[cols] floats in,
 * out[rows] out.  Host buffers. */
KORE_QMV_API int kore_qmv_mv(kore_qmv_tensor_t t, const float *x, float *out, int avx2);

/* Same with device buffers: x[cols] (16-byte aligned) -> out[rows].  The
 * quantisation runs inside the matvec launch when that is cheaper, else as a
 * launch of its own into a buffer of the tensor (so calls on one tensor from
 * different streams must not overlap).  Results equal quant() + mv(). */
KORE_QMV_API int kore_qmv_mv_dev(kore_qmv_tensor_t t, const float *x, float *out, int avx2, void *stream);

/* n (1..4) matrices with the same cols and input x in one launch: kore's
 * quant() followed by mv() of q, k and v (kore.cpp:1418-1421) or of gate and
 * up (kore.cpp:1462-1464).  outs[k] receives tensors[k]'s rows.  Same results
 * as n separate kore_qmv_mv_dev calls. */
KORE_QMV_API int kore_qmv_mv_group_dev(int n, const kore_qmv_tensor_t *tensors, const float *x,
                                       float *const *outs, int avx2, void *stream);

/* kore's batched prefill matmul, matmul_batch_float (kore.cpp:783-845), as
 * forward_batch() calls it for q/k/v, Wo, gate/up and down (kore.cpp:1524-1583):
 * x [nb][cols] fp32 activations, 1 <= nb <= 64 (kore's KORE_BMAX,
 * kore.cpp:690) -> out [nb][rows] (out[b * rows + r], kore's layout).  fp32
 * MFMA on weights dequantised as kore does (kore.cpp:337-381): the results
 * agree with kore's to fp32 rounding, max|d| <= 1e-4 * max|ref| + 1e-6 (kore's
 * own tolerance, kore_kernels.cpp:742), not bit for bit (kore sums each
 * output in one FMA chain over the columns).  Host buffers, synchronous. */
KORE_QMV_API int kore_qmv_matmul_batch(kore_qmv_tensor_t t, const float *x, int nb, float *out);

/* Same with device buffers (x 16-byte aligned; enqueued on `stream`, no
 * allocation).  Tiles of rows whose columns are split between workgroups pass
 * partial sums through a per-device workspace that tensor creation sizes:
 * calls that overlap on different streams of one device race on it. */
KORE_QMV_API int kore_qmv_matmul_batch_dev(kore_qmv_tensor_t t, const float *x, int nb, float *out,
                                           void *stream);

/* n (1..4) matrices of one device and equal cols multiplied with the same x
 * in one launch: out[k] = matmul_batch(t[k], x), as forward_batch() calls
 * matmul_batch_float for wq, wk, wv and for w_gate, w_up on the same input
 * (kore.cpp:1524-1526, 1575-1576).  Results equal n calls of
 * kore_qmv_matmul_batch_dev to fp32 rounding (the split of the sums between
 * workgroups depends on the launch).  Same workspace caveat. */
KORE_QMV_API int kore_qmv_matmul_batch_group_dev(int n, const kore_qmv_tensor_t *t, const float *x, int nb,
                                                 float *const *out, void *stream);

/* The matvec with kore's elementwise steps around it fused into the same
 * launches (kore's forward(), kore.cpp:1417-1471).  Before quantising x:
 *   norm_w  != NULL: kore's rmsnorm(x, norm_w, norm_eps) (kore.cpp:1367-1372),
 *                    bit-identical to kore's sequential double sum;
 *   up      != NULL: kore's SwiGLU, x / (1 + exp(-x)) * up (kore.cpp:1465-1468),
 *                    exp rounded from double (glibc's expf can differ in the last
 *                    bit on rare inputs, so this step holds to kore's tolerance);
 * and in the final store of matrix k:
 *   bias[k] != NULL: out = W.x + bias (kore's q/k/v biases, kore.cpp:1422-1423);
 *   accumulate:      out = out + W.x (kore's residual adds, kore.cpp:1458, 1471).
 * norm_w, up, bias are device arrays (norm_w and up 16-byte aligned, cols long;
 * bias rows long); at most one of norm_w and up. */
typedef struct kore_qmv_mv_opts {
    const float *norm_w;
    float norm_eps;
    const float *up;
    const float *bias[4];
    int accumulate;
} kore_qmv_mv_opts;

KORE_QMV_API int kore_qmv_mv_group_ex_dev(int n, const kore_qmv_tensor_t *t, const float *x,
                                          const kore_qmv_mv_opts *opts, float *const *out, int avx2,
                                          void *stream);

/* The batched matmul with kore's elementwise steps after it fused into the
 * final stores (forward_batch(), kore.cpp:1527-1532, 1567-1570, 1586-1589):
 * opts->bias[k] (q/k/v biases) and opts->accumulate (residual adds) as for
 * kore_qmv_mv_group_ex_dev; opts->norm_w and opts->up must be NULL (the batched
 * rmsnorm and SwiGLU are the two calls below).  opts may be NULL. */
KORE_QMV_API int kore_qmv_matmul_batch_group_ex_dev(int n, const kore_qmv_tensor_t *t, const float *x, int nb,
                                                    const kore_qmv_mv_opts *opts, float *const *out, void *stream);

/* kore's rmsnorm of each of `rows` rows of n floats (forward_batch(),
 * kore.cpp:1521-1522, 1572-1573; rmsnorm at kore.cpp:1367-1372): out[r] =
 * x[r] * scale_r * w, bit-identical to kore's sequential double sum.  Device
 * buffers (out may equal x), enqueued on `stream`. */
KORE_QMV_API int kore_qmv_rmsnorm_rows_dev(const float *x, const float *w, int64_t n, int rows, float eps, float *out,
                                           void *stream);

/* The batched matmul's fp16 activation split, for callers that produce the
 * activations with kore_qmv_rmsnorm_rows_split_dev (forward_batch()'s
 * attn_norm -> q/k/v and ffn_norm -> gate/up, kore.cpp:1521-1526, 1572-1576):
 * one pre-pass launch less per matmul.  kore_qmv_split_bytes(cols) is the
 * size of the split of up to 64 activations of cols values, or 0 when the
 * split is not available (cols not a multiple of 256 up to 4096, or the fp32
 * matmul path selected by KORE_GEMM=fp32); then use the plain calls. */
KORE_QMV_API size_t kore_qmv_split_bytes(int64_t cols);

/* kore_qmv_rmsnorm_rows_dev that also writes the normalised rows' split into
 * x16 (device, kore_qmv_split_bytes(n) bytes); rows <= 64; x, w, out and x16
 * 16-byte aligned. */
KORE_QMV_API int kore_qmv_rmsnorm_rows_split_dev(const float *x, const float *w, int64_t n, int rows, float eps,
                                                 float *out, void *x16, void *stream);

/* forward_batch()'s gate/up matmuls and SwiGLU (kore.cpp:1575-1581) in one call
 * on the split x16 of nb activations: out[b * rows + r] = SwiGLU(gate row r .
 * x_b, up row r . x_b), bit for bit kore_qmv_matmul_batch_group_split_dev of
 * {gate, up} followed by kore_qmv_swiglu_dev; the SwiGLU is applied where the
 * matmul adds its split tiles' partial sums (no launch of its own).  tmp
 * (device, nb * rows floats) is scratch; gate and up share rows and cols. */
KORE_QMV_API int kore_qmv_matmul_batch_glu_split_dev(const kore_qmv_tensor_t *gate_up, const void *x16, int nb,
                                                     float *out, float *tmp, void *stream);

/* kore_qmv_matmul_batch_group_ex_dev on the split x16 of nb activations
 * (written by kore_qmv_rmsnorm_rows_split_dev for the same cols as the
 * tensors', kept unchanged since) instead of x: the same results, bit for bit.
 * KORE_QMV_E_UNSUPPORTED when the tensors' cols have no split
 * (kore_qmv_split_bytes(cols) == 0); the same for the glu call above. */
KORE_QMV_API int kore_qmv_matmul_batch_group_split_dev(int n, const kore_qmv_tensor_t *t, const void *x16, int nb,
                                                       const kore_qmv_mv_opts *opts, float *const *out, void *stream);

/* kore's batched SwiGLU in place (kore.cpp:1577-1583): g[i] = g[i] / (1 +
 * exp(-g[i])) * u[i] over n floats, exp rounded from double as in
 * kore_qmv_mv_group_ex_dev.  Device buffers, enqueued on `stream`. */
KORE_QMV_API int kore_qmv_swiglu_dev(float *g, const float *u, int64_t n, void *stream);

/* kore's get_row (kore.cpp:384-407) on the device, as forward() uses it for the
 * token embedding: row `row` of `table` (device memory in the file's layout:
 * rows of n values of ggml type 0 F32, 1 F16, 30 BF16, 12 Q4_K or 14 Q6_K with
 * kore's 144 / 210-byte blocks) dequantised with kore's expressions into out[n]
 * (device), bit-identical to kore.  Enqueued on `stream`. */
KORE_QMV_API int kore_qmv_get_row_dev(int type, const void *table, int64_t row, int64_t n, float *out, void *stream);

/* Text of the last failure on this tensor (or, with NULL, of the last failed
 * call without a tensor on this thread).  Never NULL. */
KORE_QMV_API const char *kore_qmv_last_error(kore_qmv_tensor_t t);

/* Shape and resources of a matrix. */
typedef struct kore_qmv_info {
    int type;
    int device;
    int64_t rows, cols;
    size_t weight_bytes;     /* bytes one matvec streams from HBM (kore's block bytes) */
    int rows_per_wave;       /* rows one wave of the matvec kernel owns (1 .. 16)      */
} kore_qmv_info;
KORE_QMV_API int kore_qmv_get_info(kore_qmv_tensor_t t, kore_qmv_info *info);

#ifdef __cplusplus
}
#endif
#endif
