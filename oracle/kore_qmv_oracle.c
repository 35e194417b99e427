/*
 * kore_qmv_oracle.c - CPU restatement of kore's quantised matrix-vector
 * product (activation quantisation to Q8_K and the Q4_K / Q6_K x Q8_K dot
 * products), the row that sits on either side of the attention call in
 * kore's forward() (kore.cpp:1387-1394, 1417-1421).
 *
 * TEST INFRASTRUCTURE ONLY: the parity oracle of the GPU matvec.  Only
 * tests/ and bench.py's cpu_baseline leg load it; the product library never
 * calls it.  Written from the arithmetic of kore.cpp in kore's operation
 * order so that the results are bit-identical to kore's own code:
 *   ko_f16             kore.cpp:295-316   (exact f16 -> f32 widening)
 *   ko_quantize_q8K    kore.cpp:422-446   (per 256 values: the first value of
 *                      largest magnitude maps to -127, round half to even)
 *   ko_dot_q4K_ref     kore.cpp:450-477   (scalar reference)
 *   ko_dot_q6K_ref     kore.cpp:480-506   (scalar reference)
 *   ko_dot_q4K_avx2    kore.cpp:535-587   (AVX2: 8 int32 lanes per block, one
 *                      FMA chain per lane over the blocks, 4 lanes for the
 *                      minimum terms, kore's horizontal sums kore.cpp:521-528,
 *                      537-541)
 *   ko_dot_q6K_avx2    kore.cpp:591-632
 *   ko_qmatvec         kore.cpp:649-682   (one dot product per row; the row
 *                      partition over threads does not change any result)
 *   ko_dequant_row     kore.cpp:337-381   (dequant_block_q4_K / _q6_K)
 *   ko_matmul_batch    kore.cpp:744-845   (matmul_batch_float, AVX2 and scalar)
 * Every AVX2 lane sum is an exact integer; the float steps are restated with
 * explicit fmaf() where kore uses _mm256_fmadd_ps / _mm_fmadd_ps, and the
 * file is compiled with -ffp-contract=off so no other product is fused.
 *
 * Pinning: bit-identical to kore's own quantize_row_q8_K and dot_*_{ref,avx2}
 * on the fixtures tests/golden/qmv_*.npz, written by driving those functions
 * (oracle/ref_qmv_harness.cpp); plus integer closed forms in the tests (an
 * all-equal block, a zero block, ties of the largest magnitude).
 */
#include "kore_qmv_oracle.h"

#include <math.h>
#include <stdint.h>
#include <string.h>

float ko_f16(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t ex = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu, bits;
    if (ex == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            int e = -1;
            do {
                e++;
                man <<= 1;
            } while (!(man & 0x400u));
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3FFu) << 13);
        }
    } else if (ex == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((ex + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static float rd16(const uint8_t *p) {
    uint16_t h;
    memcpy(&h, p, 2);
    return ko_f16(h);
}

void ko_quantize_q8K(const float *x, int64_t n, KoQ8K *y) {
    for (int64_t i = 0; i < n / 256; i++, x += 256) {
        float amax = 0.f, maxv = 0.f;
        for (int j = 0; j < 256; j++) {
            const float ax = fabsf(x[j]);
            if (ax > amax) {
                amax = ax;
                maxv = x[j];
            }
        }
        if (amax == 0.f) {
            memset(&y[i], 0, sizeof y[i]);
            continue;
        }
        const float iscale = -127.0f / maxv;
        for (int j = 0; j < 256; j++) {
            /* kore's (int) conversion of an out-of-range or NaN value is x86's
             * cvttss2si: 0x80000000, which the int8 store truncates to 0.  Only
             * blocks whose largest magnitude is below 127/FLT_MAX get there. */
            const float t = nearbyintf(iscale * x[j]);
            const int v = fabsf(t) < 2147483648.0f ? (int)t : INT32_MIN;
            y[i].qs[j] = (int8_t)(v > 127 ? 127 : v);
        }
        for (int j = 0; j < 16; j++) {
            int s = 0;
            for (int l = 0; l < 16; l++) s += y[i].qs[16 * j + l];
            y[i].bsums[j] = (int16_t)s;
        }
        y[i].d = 1.0f / iscale;
    }
}

/* 6-bit scale and minimum of sub-block j (0..7) of a Q4_K block, from its 12
 * packed bytes: j < 4 in the low 6 bits of bytes j and j + 4; j >= 4 as a low
 * nibble in byte j + 4 plus the two top bits of byte j - 4 (scale) / j (min). */
static void q4k_scale_min(int j, const uint8_t *q, int *sc, int *mn) {
    if (j < 4) {
        *sc = q[j] & 63;
        *mn = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4);
        *mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

float ko_dot_q4K_ref(int64_t n, const uint8_t *w, const KoQ8K *y) {
    float sumf = 0.f;
    for (int64_t i = 0; i < n / 256; i++) {
        const uint8_t *b = w + i * KO_Q4K_BYTES;
        const float d = rd16(b) * y[i].d;
        const float dmin = rd16(b + 2) * y[i].d;
        const uint8_t *q = b + 16;
        int32_t isum = 0, imin = 0;
        for (int c = 0; c < 4; c++) {
            int sc0, m0, sc1, m1;
            q4k_scale_min(2 * c, b + 4, &sc0, &m0);
            q4k_scale_min(2 * c + 1, b + 4, &sc1, &m1);
            const int8_t *q8 = y[i].qs + 64 * c;
            int32_t lo = 0, hi = 0;
            for (int l = 0; l < 32; l++) {
                lo += (q[32 * c + l] & 0x0F) * q8[l];
                hi += (q[32 * c + l] >> 4) * q8[32 + l];
            }
            isum += sc0 * lo + sc1 * hi;
            imin += m0 * (y[i].bsums[4 * c] + y[i].bsums[4 * c + 1]) +
                    m1 * (y[i].bsums[4 * c + 2] + y[i].bsums[4 * c + 3]);
        }
        const float t1 = d * (float)isum;
        const float t2 = dmin * (float)imin;
        sumf = sumf + (t1 - t2);
    }
    return sumf;
}

/* q6 value v (0..255) of a Q6_K block, unsigned 0..63: low nibble from
 * ql[64h + (v%64 < 32 ? l : l + 32)] (low for v%128 < 64, high above), two
 * high bits from qh[32h + l] at bit 2 * ((v % 128) / 32); l = v % 32. */
static int q6k_u6(const uint8_t *b, int v) {
    const uint8_t *ql = b, *qh = b + 128;
    const int h = v / 128, r = v % 128, k = r / 32, l = r % 32;
    const int lo = (k & 1) ? ql[64 * h + 32 + l] : ql[64 * h + l];
    const int nib = (k & 2) ? (lo >> 4) : (lo & 0x0F);
    return nib | (((qh[32 * h + l] >> (2 * k)) & 3) << 4);
}

float ko_dot_q6K_ref(int64_t n, const uint8_t *w, const KoQ8K *y) {
    float sumf = 0.f;
    for (int64_t i = 0; i < n / 256; i++) {
        const uint8_t *b = w + i * KO_Q6K_BYTES;
        const int8_t *sc = (const int8_t *)(b + 192);
        const float d = rd16(b + 208) * y[i].d;
        int32_t isum = 0;
        for (int j = 0; j < 16; j++) {
            int32_t s = 0;
            for (int l = 0; l < 16; l++) s += (q6k_u6(b, 16 * j + l) - 32) * y[i].qs[16 * j + l];
            isum += sc[j] * s;
        }
        sumf = sumf + d * (float)isum;
    }
    return sumf;
}

/* kore's 8-lane and 4-lane horizontal sums (kore.cpp:521-528, 537-541) */
static float hsum8(const float a[8]) {
    const float l0 = a[0] + a[4], l1 = a[1] + a[5], l2 = a[2] + a[6], l3 = a[3] + a[7];
    return (l0 + l2) + (l1 + l3);
}
static float hsum4(const float a[4]) { return (a[0] + a[2]) + (a[1] + a[3]); }

float ko_dot_q4K_avx2(int64_t n, const uint8_t *w, const KoQ8K *y) {
    float acc[8] = {0}, accm[4] = {0};
    for (int64_t i = 0; i < n / 256; i++) {
        const uint8_t *b = w + i * KO_Q4K_BYTES;
        const float d = rd16(b) * y[i].d;
        const float dmin = rd16(b + 2) * y[i].d;
        int sc[8], mn[8];
        for (int j = 0; j < 8; j++) q4k_scale_min(j, b + 4, &sc[j], &mn[j]);
        /* minimum terms: lane j of 4 gets sub-blocks 2j and 2j + 1 */
        for (int j = 0; j < 4; j++) {
            const int s0 = y[i].bsums[4 * j] + y[i].bsums[4 * j + 1];
            const int s1 = y[i].bsums[4 * j + 2] + y[i].bsums[4 * j + 3];
            const int32_t prod = mn[2 * j] * s0 + mn[2 * j + 1] * s1;
            accm[j] = fmaf(-dmin, (float)prod, accm[j]);
        }
        /* lane k of 8: bytes 4k .. 4k + 3 of every 32-byte group */
        const uint8_t *q4 = b + 16;
        for (int k = 0; k < 8; k++) {
            int32_t s = 0;
            for (int c = 0; c < 4; c++) {
                int32_t pl = 0, ph = 0;
                for (int e = 0; e < 4; e++) {
                    const int byte = q4[32 * c + 4 * k + e];
                    pl += (byte & 0x0F) * y[i].qs[64 * c + 4 * k + e];
                    ph += (byte >> 4) * y[i].qs[64 * c + 32 + 4 * k + e];
                }
                s += sc[2 * c] * pl + sc[2 * c + 1] * ph;
            }
            acc[k] = fmaf(d, (float)s, acc[k]);
        }
    }
    return hsum8(acc) + hsum4(accm);
}

float ko_dot_q6K_avx2_v(int64_t n, const uint8_t *w, const KoQ8K *y, int fused_bias) {
    float acc[8] = {0}, summ = 0.f;
    for (int64_t i = 0; i < n / 256; i++) {
        const uint8_t *b = w + i * KO_Q6K_BYTES;
        const int8_t *sc = (const int8_t *)(b + 192);
        const float d = rd16(b + 208) * y[i].d;
        int32_t ibias = 0;
        for (int j = 0; j < 16; j++) ibias += sc[j] * y[i].bsums[j];
        const float d32 = d * 32.0f;
        if (fused_bias) summ = fmaf(-d32, (float)ibias, summ);
        else summ = summ - d32 * (float)ibias;
        /* group (h, k): values 128h + 32k + (0..31); lane m of 8: bytes 4m .. 4m + 3
         * of the group, scale sc[8h + 2k] for m < 4, sc[8h + 2k + 1] above */
        int32_t s[8] = {0};
        for (int h = 0; h < 2; h++)
            for (int k = 0; k < 4; k++)
                for (int m = 0; m < 8; m++) {
                    int32_t p = 0;
                    for (int e = 0; e < 4; e++) {
                        const int v = 128 * h + 32 * k + 4 * m + e;
                        p += q6k_u6(b, v) * y[i].qs[v];
                    }
                    s[m] += sc[8 * h + 2 * k + (m >= 4)] * p;
                }
        for (int m = 0; m < 8; m++) acc[m] = fmaf(d, (float)s[m], acc[m]);
    }
    return hsum8(acc) + summ;
}

float ko_dot_q6K_avx2(int64_t n, const uint8_t *w, const KoQ8K *y) {
    return ko_dot_q6K_avx2_v(n, w, y, KO_Q6K_FUSED_BIAS);
}

int ko_qmatvec(int type, int64_t rows, int64_t cols, const uint8_t *w, const KoQ8K *xq, float *out,
               int avx2) {
    if (cols % 256 != 0 || (type != KO_TYPE_Q4K && type != KO_TYPE_Q6K)) return -1;
    const int64_t row_bytes = cols / 256 * (type == KO_TYPE_Q4K ? KO_Q4K_BYTES : KO_Q6K_BYTES);
    for (int64_t r = 0; r < rows; r++) {
        const uint8_t *wr = w + r * row_bytes;
        if (type == KO_TYPE_Q4K) out[r] = avx2 ? ko_dot_q4K_avx2(cols, wr, xq) : ko_dot_q4K_ref(cols, wr, xq);
        else out[r] = avx2 ? ko_dot_q6K_avx2(cols, wr, xq) : ko_dot_q6K_ref(cols, wr, xq);
    }
    return 0;
}

/* ------------------------------------------------------------------ batched
 * kore's matmul_batch_float (kore.cpp:783-845): out[b * rows + r] = row r of
 * the dequantised weights . x[b], B activations at once.
 *   dequantisation (kore.cpp:337-381): Q4_K value = d1 * q - m1 with
 *     d1 = d * scale, m1 = dmin * min (each product rounded); Q6_K value =
 *     (d * scale) * (q - 32); plain float arithmetic (no fused steps: the
 *     dequantisers are compiled without FMA).
 *   AVX2 (kore.cpp:744-779): per (row, b) one fused multiply-add chain over
 *     the columns in order, starting from 0.
 *   scalar (kore.cpp:820-839): per 256-column block a double sum in column
 *     order, added to a float accumulator.
 */
static void dequant_q4K_block(const uint8_t *b, float *y) {
    const float d = rd16(b), dmin = rd16(b + 2);
    const uint8_t *q = b + 16;
    for (int c = 0; c < 4; c++) {
        int sc, mn;
        q4k_scale_min(2 * c, b + 4, &sc, &mn);
        const float d1 = d * (float)sc, m1 = dmin * (float)mn;
        q4k_scale_min(2 * c + 1, b + 4, &sc, &mn);
        const float d2 = d * (float)sc, m2 = dmin * (float)mn;
        for (int l = 0; l < 32; l++) y[64 * c + l] = d1 * (float)(q[32 * c + l] & 0x0F) - m1;
        for (int l = 0; l < 32; l++) y[64 * c + 32 + l] = d2 * (float)(q[32 * c + l] >> 4) - m2;
    }
}

static void dequant_q6K_block(const uint8_t *b, float *y) {
    const int8_t *sc = (const int8_t *)(b + 192);
    const float d = rd16(b + 208);
    for (int v = 0; v < 256; v++) {
        const int h = v / 128, k = (v % 128) / 32, l = v % 32;
        const float ds = d * (float)sc[8 * h + 2 * k + l / 16];
        y[v] = ds * (float)(q6k_u6(b, v) - 32);
    }
}

void ko_dequant_row(int type, int64_t cols, const uint8_t *w, float *y) {
    const int64_t nb = cols / 256;
    for (int64_t i = 0; i < nb; i++) {
        if (type == KO_TYPE_Q4K) dequant_q4K_block(w + i * KO_Q4K_BYTES, y + 256 * i);
        else dequant_q6K_block(w + i * KO_Q6K_BYTES, y + 256 * i);
    }
}

int ko_matmul_batch(int type, int64_t rows, int64_t cols, const uint8_t *w, const float *x, int B, float *out,
                    int avx2) {
    if (cols % 256 != 0 || B <= 0 || (type != KO_TYPE_Q4K && type != KO_TYPE_Q6K)) return -1;
    const int64_t nb = cols / 256, rb = nb * (type == KO_TYPE_Q4K ? KO_Q4K_BYTES : KO_Q6K_BYTES);
    float wf[256];
    for (int64_t r = 0; r < rows; r++) {
        for (int b = 0; b < B; b++) out[(size_t)b * rows + r] = 0.f;
        for (int64_t i = 0; i < nb; i++) {
            ko_dequant_row(type, 256, w + r * rb + i * (rb / nb), wf);
            for (int b = 0; b < B; b++) {
                const float *xb = x + (size_t)b * cols + 256 * i;
                float *o = &out[(size_t)b * rows + r];
                if (avx2) {
                    float acc = *o;
                    for (int j = 0; j < 256; j++) acc = fmaf(wf[j], xb[j], acc);
                    *o = acc;
                } else {
                    double s = 0;
                    for (int j = 0; j < 256; j++) s += (double)wf[j] * xb[j];
                    *o = *o + (float)s;
                }
            }
        }
    }
    return 0;
}

/* ------------------------------------------------------------ around the matvecs */

/* kore.cpp:1367-1372 rmsnorm: double sum of (double)x[i] * x[i] in index order,
 * scale = 1.0f / std::sqrt((float)(ss / n) + eps), out[i] = x[i] * scale * w[i]. */
void ko_rmsnorm(float *out, const float *x, const float *w, int n, float eps) {
    double ss = 0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * x[i];
    const float scale = 1.0f / sqrtf((float)(ss / n) + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * scale * w[i];
}

/* kore.cpp:1465-1468 SwiGLU in place: g = g / (1.0f + exp(-g)) * u. */
void ko_swiglu(float *g, const float *u, int n) {
    for (int i = 0; i < n; i++) {
        const float gg = g[i];
        g[i] = gg / (1.0f + expf(-gg)) * u[i];
    }
}
