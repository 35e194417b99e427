/*
 * kore_oracle.c - CPU restatement of kore's RoPE-GQA attention path.
 *
 * TEST INFRASTRUCTURE ONLY (the parity oracle and the timed CPU baseline);
 * the product path never links or calls it.  Every function follows the
 * kore.cpp lines cited beside it in the same operation order.  The file is
 * compiled with -ffp-contract=off: kore's forward()/forward_batch() contain
 * no fused multiply-add (only its *_avx2 helpers do, through intrinsics), so
 * every product below is rounded before it is added unless fmaf() says
 * otherwise.
 */
#include "kore_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ RoPE */

/* kore.cpp:1337-1339: inv_freq[i] = (float)pow((double)base, -2.0*i/hd) */
void ko_inv_freq(int head_dim, float rope_base, float *inv_freq) {
    const int half = head_dim / 2;
    for (int i = 0; i < half; i++)
        inv_freq[i] = (float)pow((double)rope_base, -2.0 * i / head_dim);
}

/* kore.cpp:1405-1410 and 1503-1512: angle in double from the float inv_freq,
 * cos/sin in double (libm), rounded to float. */
void ko_rope_cs(int pos, int head_dim, const float *inv_freq, float *c, float *s) {
    const int half = head_dim / 2;
    for (int i = 0; i < half; i++) {
        const double a = (double)pos * inv_freq[i];
        c[i] = (float)cos(a);
        s[i] = (float)sin(a);
    }
}

/* kore.cpp:1411 / 1513 */
float ko_inv_sqrt(int head_dim) { return 1.0f / sqrtf((float)head_dim); }

/* kore.cpp:1374-1384: NEOX pairs (i, i + hd/2); each product rounded, then
 * the difference / sum rounded. */
void ko_rope_neox(float *vec, int n_heads, int head_dim, const float *c, const float *s) {
    const int half = head_dim / 2;
    for (int h = 0; h < n_heads; h++) {
        float *p = vec + (size_t)h * head_dim;
        for (int i = 0; i < half; i++) {
            const float x0 = p[i], x1 = p[i + half];
            const float a = x0 * c[i], b = x1 * s[i];
            const float d = x0 * s[i], e = x1 * c[i];
            p[i] = a - b;
            p[i + half] = d + e;
        }
    }
}

void ko_rope_rows(float *x, int n_rows, int n_heads, int head_dim, const int *pos,
                  const float *inv_freq) {
    const int half = head_dim / 2;
    float *c = (float *)malloc(sizeof(float) * (size_t)half * 2);
    if (!c) return;
    for (int r = 0; r < n_rows; r++) {
        ko_rope_cs(pos[r], head_dim, inv_freq, c, c + half);
        ko_rope_neox(x + (size_t)r * n_heads * head_dim, n_heads, head_dim, c, c + half);
    }
    free(c);
}

/* ------------------------------------------------------- decode attention */

/* kore.cpp:1432-1455 generalised to a run of positions t0..t1 stored at
 * slot t % mod (mod = ctx for kore semantics, where t1 < ctx so no wrap). */
static void attn_decode_range(const float *q_roped, const float *kc, const float *vc,
                              int t0, int t1, int mod, int n_head, int n_head_kv, int hd,
                              float inv_sqrt, float *sc, float *att) {
    const int kvd = n_head_kv * hd;
    const int n_rep = n_head / n_head_kv;
    const int n = t1 - t0 + 1;
    for (int hh = 0; hh < n_head; hh++) {
        const float *qh = q_roped + (size_t)hh * hd;
        const int kvh = hh / n_rep;
        float mx = -INFINITY;
        for (int j = 0; j < n; j++) {
            const int slot = (t0 + j) % mod;
            const float *kt = kc + (size_t)slot * kvd + (size_t)kvh * hd;
            float s = 0;
            for (int i = 0; i < hd; i++) s += qh[i] * kt[i];
            s *= inv_sqrt;
            sc[j] = s;
            if (s > mx) mx = s;
        }
        float sum = 0;
        for (int j = 0; j < n; j++) { sc[j] = expf(sc[j] - mx); sum += sc[j]; }
        const float inv = 1.0f / sum;
        float *oh = att + (size_t)hh * hd;
        for (int i = 0; i < hd; i++) oh[i] = 0;
        for (int j = 0; j < n; j++) {
            const int slot = (t0 + j) % mod;
            const float p = sc[j] * inv;
            const float *vt = vc + (size_t)slot * kvd + (size_t)kvh * hd;
            for (int i = 0; i < hd; i++) oh[i] += p * vt[i];
        }
    }
}

void ko_attn_decode(const float *q_roped, const float *kc, const float *vc, int pos,
                    int n_head, int n_head_kv, int head_dim, float inv_sqrt,
                    float *scores, float *att) {
    attn_decode_range(q_roped, kc, vc, 0, pos, pos + 1, n_head, n_head_kv, head_dim,
                      inv_sqrt, scores, att);
}

/* ----------------------------------------- hd_dot / hd_fma (kore.cpp:690-725)
 * The AVX2 variants keep two 8-lane FMA accumulators over 16-float steps and
 * reduce them with hsum256 (kore.cpp:521-528): lanes j and j+4 of
 * (acc0+acc1) are added, then (l0+l2) + (l1+l3).  The scalar tails (head_dim
 * not a multiple of 16 / 8) behave differently in kore's g++ -O3 build: the
 * hd_dot tail is a rounded product then a rounded add, the hd_fma tail is a
 * fused multiply-add.  Both were established against kore itself (the
 * hd=40 and hd=36 golden fixtures fail with the other choice).  Written as
 * 8-lane arrays with fmaf(); the "fma" build of the same code only lets the
 * compiler use the hardware instruction, fmaf() is exact either way. */
#define KO_DOT_BODY                                                            \
    float acc0[8] = {0, 0, 0, 0, 0, 0, 0, 0}, acc1[8] = {0, 0, 0, 0, 0, 0, 0, 0}; \
    int i = 0;                                                                 \
    for (; i + 16 <= n; i += 16)                                               \
        for (int j = 0; j < 8; j++) {                                          \
            acc0[j] = fmaf(a[i + j], b[i + j], acc0[j]);                       \
            acc1[j] = fmaf(a[i + 8 + j], b[i + 8 + j], acc1[j]);               \
        }                                                                      \
    float v[8];                                                                \
    for (int j = 0; j < 8; j++) v[j] = acc0[j] + acc1[j];                      \
    float l[4];                                                                \
    for (int j = 0; j < 4; j++) l[j] = v[j] + v[j + 4];                        \
    const float l02 = l[0] + l[2], l13 = l[1] + l[3];                          \
    float s = l02 + l13;                                                       \
    for (; i < n; i++) s += a[i] * b[i];                                       \
    return s;

#define KO_AXPY_BODY                                                           \
    int i = 0;                                                                 \
    for (; i + 8 <= n; i += 8)                                                 \
        for (int j = 0; j < 8; j++) o[i + j] = fmaf(p, v[i + j], o[i + j]);    \
    for (; i < n; i++) o[i] = fmaf(p, v[i], o[i]);

static float dot_lanes_generic(const float *a, const float *b, int n) { KO_DOT_BODY }
static void axpy_lanes_generic(float *o, const float *v, float p, int n) { KO_AXPY_BODY }

#if defined(__x86_64__)
__attribute__((target("avx2,fma"))) static float dot_lanes_fma(const float *a, const float *b, int n) { KO_DOT_BODY }
__attribute__((target("avx2,fma"))) static void axpy_lanes_fma(float *o, const float *v, float p, int n) { KO_AXPY_BODY }
static int g_has_fma = -1;
int ko_cpu_has_fma(void) {
    if (g_has_fma < 0) {
        __builtin_cpu_init();
        g_has_fma = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
    }
    return g_has_fma;
}
#else
static float dot_lanes_fma(const float *a, const float *b, int n) { return dot_lanes_generic(a, b, n); }
static void axpy_lanes_fma(float *o, const float *v, float p, int n) { axpy_lanes_generic(o, v, p, n); }
int ko_cpu_has_fma(void) { return 0; }
#endif

/* kore.cpp:705-710 (avx2 = 0) and 693-703 (avx2 = 1) */
float ko_hd_dot(const float *a, const float *b, int n, int avx2) {
    if (avx2) return ko_cpu_has_fma() ? dot_lanes_fma(a, b, n) : dot_lanes_generic(a, b, n);
    float s = 0;
    for (int i = 0; i < n; i++) s += a[i] * b[i];
    return s;
}

/* kore.cpp:722-725 (avx2 = 0) and 712-720 (avx2 = 1) */
void ko_hd_fma(float *o, const float *v, float p, int n, int avx2) {
    if (avx2) {
        if (ko_cpu_has_fma()) axpy_lanes_fma(o, v, p, n);
        else axpy_lanes_generic(o, v, p, n);
        return;
    }
    for (int i = 0; i < n; i++) o[i] += p * v[i];
}

/* ------------------------------------------------ batched causal attention */

/* kore.cpp:1542-1563: query row z (position pos0+z) attends cache rows
 * 0..pos0+z; `scores` holds at least pos0+nb floats. */
void ko_attn_batch(const float *bq_roped, int nb, int pos0, const float *kc, const float *vc,
                   int n_head, int n_head_kv, int head_dim, float inv_sqrt, int avx2,
                   float *scores, float *batt) {
    const int hd = head_dim, kvd = n_head_kv * hd, E = n_head * hd;
    const int n_rep = n_head / n_head_kv;
    for (int hh = 0; hh < n_head; hh++) {
        const int kvh = hh / n_rep;
        for (int z = 0; z < nb; z++) {
            const int lim = pos0 + z;
            const float *qh = bq_roped + (size_t)z * E + (size_t)hh * hd;
            float *sc = scores;
            float mx = -INFINITY;
            for (int t = 0; t <= lim; t++) {
                const float *kt = kc + (size_t)t * kvd + (size_t)kvh * hd;
                const float s = ko_hd_dot(qh, kt, hd, avx2) * inv_sqrt;
                sc[t] = s;
                if (s > mx) mx = s;
            }
            float sum = 0;
            for (int t = 0; t <= lim; t++) { sc[t] = expf(sc[t] - mx); sum += sc[t]; }
            const float inv = 1.0f / sum;
            float *oh = batt + (size_t)z * E + (size_t)hh * hd;
            memset(oh, 0, (size_t)hd * sizeof(float));
            for (int t = 0; t <= lim; t++)
                ko_hd_fma(oh, vc + (size_t)t * kvd + (size_t)kvh * hd, sc[t] * inv, hd, avx2);
        }
    }
}

/* ------------------------------------------------------------- KV store */

int ko_kv_init(ko_kv *kv, int n_layer, int ctx, int n_head, int n_head_kv, int head_dim,
               float rope_base, int window) {
    memset(kv, 0, sizeof(*kv));
    /* kore.cpp:1278-1288 geometry guards */
    if (n_layer <= 0 || ctx <= 0 || n_head <= 0 || n_head_kv <= 0 || head_dim <= 0) return -1;
    if (n_head % n_head_kv != 0 || head_dim % 2 != 0 || !(rope_base > 0)) return -1;
    if (window < 0 || (window > 0 && window != ctx)) return -1;
    const size_t kvd = (size_t)n_head_kv * head_dim;
    const size_t n = (size_t)n_layer * ctx * kvd;
    kv->n_layer = n_layer; kv->ctx = ctx; kv->n_head = n_head; kv->n_head_kv = n_head_kv;
    kv->head_dim = head_dim; kv->window = window; kv->rope_base = rope_base;
    kv->kcache = (float *)calloc(n, sizeof(float));     /* zero-filled, kore.cpp:1344-1345 */
    kv->vcache = (float *)calloc(n, sizeof(float));
    kv->inv_freq = (float *)malloc(sizeof(float) * (size_t)(head_dim / 2 + 1));
    kv->scores = (float *)malloc(sizeof(float) * (size_t)ctx);
    if (!kv->kcache || !kv->vcache || !kv->inv_freq || !kv->scores) { ko_kv_free(kv); return -2; }
    ko_inv_freq(head_dim, rope_base, kv->inv_freq);
    return 0;
}

void ko_kv_free(ko_kv *kv) {
    free(kv->kcache); free(kv->vcache); free(kv->inv_freq); free(kv->scores);
    memset(kv, 0, sizeof(*kv));
}

/* forward() hot path for one layer: kore.cpp:1405-1411 (cos/sin, inv_sqrt),
 * 1424-1425 (RoPE), 1427-1430 (append), 1432-1455 (attention). */
int ko_decode(ko_kv *kv, int layer, int pos, const float *q, const float *k, const float *v,
              float *out) {
    const int hd = kv->head_dim, half = hd / 2, kvd = kv->n_head_kv * hd, E = kv->n_head * hd;
    if (layer < 0 || layer >= kv->n_layer || pos < 0) return -1;
    if (kv->window == 0 && pos >= kv->ctx) return -1;         /* kore.cpp:1400 */
    float *c = (float *)malloc(sizeof(float) * (size_t)half * 2);
    float *qr = (float *)malloc(sizeof(float) * (size_t)(E + kvd));
    if (!c || !qr) { free(c); free(qr); return -2; }
    float *s = c + half, *kr = qr + E;
    ko_rope_cs(pos, hd, kv->inv_freq, c, s);
    const float inv_sqrt = ko_inv_sqrt(hd);
    memcpy(qr, q, sizeof(float) * (size_t)E);
    memcpy(kr, k, sizeof(float) * (size_t)kvd);
    ko_rope_neox(qr, kv->n_head, hd, c, s);
    ko_rope_neox(kr, kv->n_head_kv, hd, c, s);
    float *kc = kv->kcache + (size_t)layer * kv->ctx * kvd;
    float *vc = kv->vcache + (size_t)layer * kv->ctx * kvd;
    const int slot = pos % kv->ctx;
    memcpy(kc + (size_t)slot * kvd, kr, sizeof(float) * (size_t)kvd);
    memcpy(vc + (size_t)slot * kvd, v, sizeof(float) * (size_t)kvd);
    const int t0 = (kv->window > 0 && pos >= kv->window) ? pos - kv->window + 1 : 0;
    attn_decode_range(qr, kc, vc, t0, pos, kv->ctx, kv->n_head, kv->n_head_kv, hd, inv_sqrt,
                      kv->scores, out);
    free(c); free(qr);
    return 0;
}

/* forward_batch() hot path for one layer: kore.cpp:1503-1513, 1535-1539
 * (RoPE + append of every row first), 1542-1563 (causal attention).  kore
 * feeds at most 64 rows per call (kore.cpp:690, 1490); since a row only
 * attends positions <= its own, one call over n rows gives the same bits as
 * kore's 64-row chunks. */
int ko_prefill(ko_kv *kv, int layer, int pos0, int n, const float *q, const float *k,
               const float *v, float *out, int avx2) {
    const int hd = kv->head_dim, half = hd / 2, kvd = kv->n_head_kv * hd, E = kv->n_head * hd;
    if (layer < 0 || layer >= kv->n_layer) return -1;
    if (n <= 0 || pos0 < 0 || pos0 + n > kv->ctx) return -1;   /* kore.cpp:1490 */
    float *c = (float *)malloc(sizeof(float) * (size_t)half * 2);
    float *bq = (float *)malloc(sizeof(float) * (size_t)n * E);
    float *kr = (float *)malloc(sizeof(float) * (size_t)kvd);
    if (!c || !bq || !kr) { free(c); free(bq); free(kr); return -2; }
    float *s = c + half;
    float *kc = kv->kcache + (size_t)layer * kv->ctx * kvd;
    float *vc = kv->vcache + (size_t)layer * kv->ctx * kvd;
    for (int z = 0; z < n; z++) {
        ko_rope_cs(pos0 + z, hd, kv->inv_freq, c, s);
        memcpy(bq + (size_t)z * E, q + (size_t)z * E, sizeof(float) * (size_t)E);
        memcpy(kr, k + (size_t)z * kvd, sizeof(float) * (size_t)kvd);
        ko_rope_neox(bq + (size_t)z * E, kv->n_head, hd, c, s);
        ko_rope_neox(kr, kv->n_head_kv, hd, c, s);
        memcpy(kc + (size_t)(pos0 + z) * kvd, kr, sizeof(float) * (size_t)kvd);
        memcpy(vc + (size_t)(pos0 + z) * kvd, v + (size_t)z * kvd, sizeof(float) * (size_t)kvd);
    }
    ko_attn_batch(bq, n, pos0, kc, vc, kv->n_head, kv->n_head_kv, hd, ko_inv_sqrt(hd), avx2,
                  kv->scores, out);
    free(c); free(bq); free(kr);
    return 0;
}

/* --------------------------------------------------- double brute force */

void ko_attn_ref64(const float *q_roped, const float *kc, const float *vc, const int *rows,
                   int n_rows, int n_head, int n_head_kv, int head_dim, double *out) {
    const int hd = head_dim, kvd = n_head_kv * hd, n_rep = n_head / n_head_kv;
    const double scale = 1.0 / sqrt((double)hd);
    double *sc = (double *)malloc(sizeof(double) * (size_t)(n_rows > 0 ? n_rows : 1));
    if (!sc) return;
    for (int h = 0; h < n_head; h++) {
        const int g = h / n_rep;
        const float *qh = q_roped + (size_t)h * hd;
        double mx = -INFINITY;
        for (int j = 0; j < n_rows; j++) {
            const float *kt = kc + (size_t)rows[j] * kvd + (size_t)g * hd;
            double s = 0;
            for (int i = 0; i < hd; i++) s += (double)qh[i] * (double)kt[i];
            sc[j] = s * scale;
            if (sc[j] > mx) mx = sc[j];
        }
        double sum = 0;
        for (int j = 0; j < n_rows; j++) { sc[j] = exp(sc[j] - mx); sum += sc[j]; }
        double *oh = out + (size_t)h * hd;
        for (int i = 0; i < hd; i++) oh[i] = 0;
        for (int j = 0; j < n_rows; j++) {
            const float *vt = vc + (size_t)rows[j] * kvd + (size_t)g * hd;
            const double p = sc[j] / sum;
            for (int i = 0; i < hd; i++) oh[i] += p * (double)vt[i];
        }
    }
    free(sc);
}

/* ------------------------------------------------------ synthetic inputs */

uint64_t ko_splitmix64(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline uint64_t synth_key(uint64_t seed, uint64_t stream) {
    return ko_splitmix64(ko_splitmix64(seed) ^ stream);
}

/* Irwin-Hall(12): six 64-bit hashes, two 24-bit uniforms from each (bits
 * 0..23 and 32..55).  S - 6*2^24 is an exact integer below 2^28 in
 * magnitude; one rounding to float, then an exact scaling by 2^-24. */
static inline float synth_from_key(uint64_t key, uint64_t idx) {
    int64_t sum = 0;
    for (uint64_t k = 0; k < 6; k++) {
        const uint64_t h = ko_splitmix64(key ^ (idx * 8u + k));
        sum += (int64_t)(h & 0xFFFFFFu) + (int64_t)((h >> 32) & 0xFFFFFFu);
    }
    const int32_t centred = (int32_t)(sum - 6 * (int64_t)0x1000000);
    return (float)centred * (1.0f / 16777216.0f);
}

float ko_synth_value(uint64_t seed, uint64_t stream, uint64_t idx) {
    return synth_from_key(synth_key(seed, stream), idx);
}

int ko_synth_is_outlier(uint64_t seed, uint64_t tensor, uint64_t ch, uint32_t per_mille) {
    if (per_mille == 0) return 0;
    const uint64_t h = ko_splitmix64(ko_splitmix64(seed ^ 0x00571E50ull) ^ (tensor << 32) ^ ch);
    return (uint32_t)(h % 1000u) < per_mille;
}

void ko_synth_fill(float *dst, int rows, int dim, uint64_t seed, uint64_t stream, uint64_t row0,
                   uint64_t tensor, uint32_t per_mille, float outlier_scale) {
    const uint64_t key = synth_key(seed, stream);
    for (int c = 0; c < dim; c++) {
        const int out = ko_synth_is_outlier(seed, tensor, (uint64_t)c, per_mille);
        for (int r = 0; r < rows; r++) {
            float x = synth_from_key(key, (row0 + (uint64_t)r) * (uint64_t)dim + (uint64_t)c);
            if (out) x *= outlier_scale;
            dst[(size_t)r * dim + c] = x;
        }
    }
}
