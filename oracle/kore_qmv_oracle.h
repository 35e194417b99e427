/*
 * kore_qmv_oracle.h - CPU restatement of kore's Q8_K activation quantisation
 * and Q4_K / Q6_K x Q8_K dot products (kore.cpp:295-316, 422-506, 535-682).
 *
 * TEST INFRASTRUCTURE ONLY (the parity oracle of the GPU matvec); see
 * kore_qmv_oracle.c for the kore.cpp lines each function follows and how
 * each is pinned.
 */
#ifndef KORE_QMV_ORACLE_H
#define KORE_QMV_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids of the two weight formats (kore.cpp GGML_Q4_K / GGML_Q6_K) */
#define KO_TYPE_Q4K 12
#define KO_TYPE_Q6K 14
#define KO_Q4K_BYTES 144   /* d f16, dmin f16, 12 bytes of 6-bit scales/mins, 128 bytes of nibbles */
#define KO_Q6K_BYTES 210   /* 128 bytes low nibbles, 64 bytes high bits, 16 int8 scales, d f16 */

/* kore's AVX2 Q6_K path subtracts d * 32 * bias from a scalar sum; the
 * compiler may fuse it (kore is built with GCC's default fp-contract inside a
 * target("avx2,fma") function).  Which form kore's build uses is fixed by the
 * golden fixtures written from kore's own dot product. */
#define KO_Q6K_FUSED_BIAS 1

/* kore's BlockQ8K (kore.cpp:415-420): 292 bytes */
typedef struct {
    float d;
    int8_t qs[256];
    int16_t bsums[16];
} KoQ8K;

float ko_f16(uint16_t h);
void  ko_quantize_q8K(const float *x, int64_t n, KoQ8K *y);
float ko_dot_q4K_ref(int64_t n, const uint8_t *w, const KoQ8K *y);
float ko_dot_q6K_ref(int64_t n, const uint8_t *w, const KoQ8K *y);
float ko_dot_q4K_avx2(int64_t n, const uint8_t *w, const KoQ8K *y);
float ko_dot_q6K_avx2(int64_t n, const uint8_t *w, const KoQ8K *y);
/* both readings of the AVX2 Q6_K bias step (fused_bias 0: rounded product,
 * then the subtraction; 1: one fused multiply-add) */
float ko_dot_q6K_avx2_v(int64_t n, const uint8_t *w, const KoQ8K *y, int fused_bias);
/* out[r] = row r of the weights (rows x cols, row-major blocks) . xq,
 * with the AVX2 (avx2 = 1) or scalar arithmetic; -1 for a bad type or cols */
int   ko_qmatvec(int type, int64_t rows, int64_t cols, const uint8_t *w, const KoQ8K *xq, float *out,
                 int avx2);

/* kore's dequantisers (kore.cpp:337-381): cols values of one row */
void  ko_dequant_row(int type, int64_t cols, const uint8_t *w, float *y);
/* kore's matmul_batch_float (kore.cpp:783-845): out[b * rows + r] for B
 * activations x[b * cols + j]; avx2 = 1: one fused multiply-add chain per
 * output, 0: per-block double sums; -1 for a bad type, cols or B */
int   ko_matmul_batch(int type, int64_t rows, int64_t cols, const uint8_t *w, const float *x, int B, float *out,
                      int avx2);

/* kore's rmsnorm (kore.cpp:1367-1372) and SwiGLU (kore.cpp:1465-1468, in place). */
void  ko_rmsnorm(float *out, const float *x, const float *w, int n, float eps);
void  ko_swiglu(float *g, const float *u, int n);

#ifdef __cplusplus
}
#endif

#endif
