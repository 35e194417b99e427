// kore_attn_kernels.hip - gfx950 (CDNA4) kernels of kore's attention path.
//
//   decode_kernel   single-token decode of one layer: RoPE of q and k
//                   (kore.cpp:1424-1425), append of the new k/v row
//                   (kore.cpp:1427-1430), split-K attention over the cache
//                   (kore.cpp:1432-1455) and the combine of the splits, all in
//                   one launch.  HBM-bound: every K/V byte is read once per
//                   kv-head (not once per q-head as kore's head-outer loop
//                   does) with 16-byte loads issued before any arithmetic.
//   append_kernel   RoPE + append of a prefill chunk (kore.cpp:1535-1538).
//   prefill_kernel  causal attention of a prefill chunk (kore.cpp:1542-1563)
//                   on fp32 MFMA (v_mfma_f32_32x32x2_f32) with LDS-staged K and
//                   transposed V tiles shared by the four waves of a
//                   workgroup, which all belong to one kv-head (GQA sharing).
//   synth_kernel    counter-based synthetic inputs for benchmarks and tests.
//
// RoPE is bit-exact with kore: cos/sin come from the host-built table (the
// same double-precision libm expression as kore.cpp:1407-1409) and the
// rotation is evaluated without contraction (each product rounded, then the
// sum), so the cache rows equal kore's bit for bit.  The whole library is
// built with -ffp-contract=off; fused multiply-adds below are explicit
// fmaf() calls or MFMA instructions.
#include "kore_attn_kernels.h"

#include <cmath>

namespace kore_attn_gpu {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;

typedef float floatx16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }
__device__ __forceinline__ void st4(float *p, float4 v) { *reinterpret_cast<float4 *>(p) = v; }
__device__ __forceinline__ float4 zero4() { return make_float4(0.f, 0.f, 0.f, 0.f); }
__device__ __forceinline__ float comp(const float4 &v, int e) {
    return e == 0 ? v.x : (e == 1 ? v.y : (e == 2 ? v.z : v.w));
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
    return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
    return x;
}

// NEOX rotation of the pair (x0, x1) = (x[i], x[i + hd/2]) by (c, s)
// (kore.cpp:1379-1382): products rounded, then difference / sum rounded.
__device__ __forceinline__ void rope_pair(float x0, float x1, float2 cs, float &y0, float &y1) {
#pragma clang fp contract(off)
    const float a = x0 * cs.x, b = x1 * cs.y;
    const float c = x0 * cs.y, d = x1 * cs.x;
    y0 = a - b;
    y1 = c + d;
}

// ------------------------------------------------------------------ decode

template <int HD>
struct DecodeGeom {
    static constexpr int LPR = HD / 16;       // lanes sharing one K row in the score pass
    static constexpr int RPW = 64 / LPR;      // K rows per wave per pass
    static constexpr int RPP = RPW * kWaves;  // K rows per workgroup per pass
    static constexpr int VL = HD / 4;         // lanes sharing one V row in the PV pass
    static constexpr int VRW = 64 / VL;       // V rows per wave per load
    static constexpr int SMAX = kWaves * HD;  // splits the combine can hold (LDS reuse)
};

// Workgroup (split, kv-head g): rows [split*T, split*T + T) of kv-head g for
// the NR q-heads of g.  Score pass: LPR lanes per K row, each lane holds 16
// of the row's floats (4 x 16 B loads, dims j*4*LPR + 4c + e) and the same
// dims of the NR roped queries; partial dots are reduced over the LPR lanes.
// The split's softmax is exact (two passes over LDS-resident scores, no
// rescaling); the PV pass puts VL lanes on a V row (one float4 each).  Split
// partials (o, max, sum) go to HBM; the last workgroup of kv-head g to
// finish (device-scope counter) merges them.
template <int HD, int NR, int NPASS>
__global__ __launch_bounds__(kThreads) void decode_kernel(DecodeArgs a) {
    using G = DecodeGeom<HD>;
    constexpr int T = G::RPP * NPASS;
    constexpr int HALF = HD / 2;
    constexpr int NV = T / (kWaves * G::VRW);
    static_assert(T <= kThreads, "one thread per row in the softmax pass");
    static_assert(NR >= 1 && NR <= 8, "at most 8 q-heads per workgroup");

    __shared__ __align__(16) float s_q[NR * HD];
    __shared__ __align__(16) float s_knew[HD];
    __shared__ __align__(16) float s_vnew[HD];
    __shared__ __align__(16) float s_p[T * 8];
    __shared__ __align__(16) float s_red[kWaves * NR * HD > G::SMAX * NR ? kWaves * NR * HD : G::SMAX * NR];
    __shared__ float s_stat[2 * kWaves * 8];
    __shared__ float s_m[8], s_l[8];
    __shared__ unsigned s_ticket;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int split = blockIdx.x, g = blockIdx.y;
    const int r0 = split * a.rows_per_split;
    const int nrows = min(T, a.n_attend - r0);
    const size_t head_base = (size_t)g * a.slots * HD;
    const float *kbase = a.kc + head_base + (size_t)r0 * HD;
    const float *vbase = a.vc + head_base + (size_t)r0 * HD;
    const int new_local = a.new_slot - r0;
    const bool has_new = new_local >= 0 && new_local < nrows;

    // ---- all K and V loads of the split first: the HBM latency overlaps
    // the RoPE work below.
    const int c = lane % G::LPR, rw = lane / G::LPR;
    float4 kreg[NPASS][4];
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
        const int row = ps * G::RPP + wave * G::RPW + rw;
        const bool ok = row < nrows;
        const float *kp = kbase + (size_t)(ok ? row : 0) * HD + c * 4;
#pragma unroll
        for (int j = 0; j < 4; ++j) kreg[ps][j] = ok ? ld4(kp + j * (G::LPR * 4)) : zero4();
    }
    const int vc4 = lane % G::VL, vr = lane / G::VL;
    float4 vreg[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int row = wave * (T / kWaves) + i * G::VRW + vr;
        const bool ok = row < nrows;
        vreg[i] = ok ? ld4(vbase + (size_t)(ok ? row : 0) * HD + vc4 * 4) : zero4();
    }

    // ---- RoPE of this group's q heads; RoPE + append of the new k/v row.
    for (int idx = tid; idx < NR * HALF; idx += kThreads) {
        const int h = idx / HALF, i = idx - h * HALF;
        const float *qh = a.q + (size_t)(g * a.n_rep + h) * HD;
        float y0, y1;
        rope_pair(qh[i], qh[i + HALF], a.cs[i], y0, y1);
        s_q[h * HD + i] = y0;
        s_q[h * HD + i + HALF] = y1;
    }
    if (has_new) {
        const float *kh = a.k + (size_t)g * HD;
        float *kd = a.kc + head_base + (size_t)a.new_slot * HD;
        for (int i = tid; i < HALF; i += kThreads) {
            float y0, y1;
            rope_pair(kh[i], kh[i + HALF], a.cs[i], y0, y1);
            s_knew[i] = y0;
            s_knew[i + HALF] = y1;
            kd[i] = y0;
            kd[i + HALF] = y1;
        }
        float *vd = a.vc + head_base + (size_t)a.new_slot * HD;
        for (int i = tid; i < HD; i += kThreads) {
            const float x = a.v[(size_t)g * HD + i];
            s_vnew[i] = x;
            vd[i] = x;
        }
    }
    __syncthreads();

    // ---- scores s = (q . k) * scale, as kore (kore.cpp:1438-1440)
    float qv[NR][16];
#pragma unroll
    for (int h = 0; h < NR; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float4 t = ld4(&s_q[h * HD + j * (G::LPR * 4) + c * 4]);
            qv[h][4 * j + 0] = t.x;
            qv[h][4 * j + 1] = t.y;
            qv[h][4 * j + 2] = t.z;
            qv[h][4 * j + 3] = t.w;
        }
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
        const int row = ps * G::RPP + wave * G::RPW + rw;
        float4 kk[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) kk[j] = kreg[ps][j];
        if (row == new_local) {
#pragma unroll
            for (int j = 0; j < 4; ++j) kk[j] = ld4(&s_knew[j * (G::LPR * 4) + c * 4]);
        }
        float acc[NR];
#pragma unroll
        for (int h = 0; h < NR; ++h) {
            float s = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                s = fmaf(qv[h][4 * j + 0], kk[j].x, s);
                s = fmaf(qv[h][4 * j + 1], kk[j].y, s);
                s = fmaf(qv[h][4 * j + 2], kk[j].z, s);
                s = fmaf(qv[h][4 * j + 3], kk[j].w, s);
            }
            acc[h] = s;
        }
#pragma unroll
        for (int off = 1; off < G::LPR; off <<= 1)
#pragma unroll
            for (int h = 0; h < NR; ++h) acc[h] += __shfl_xor(acc[h], off);
        if (row < nrows) {
#pragma unroll
            for (int h = 0; h < NR; ++h)
                if (h % G::LPR == c) s_p[row * 8 + h] = acc[h] * a.scale;
        }
    }
    __syncthreads();

    // ---- split softmax: exact max, then exp and sum (one thread per row)
    {
        const bool ok = tid < nrows;
#pragma unroll
        for (int h = 0; h < NR; ++h) {
            const float m = wave_max(ok ? s_p[tid * 8 + h] : -INFINITY);
            if (lane == 0) s_stat[wave * 8 + h] = m;
        }
        __syncthreads();
        if (tid < NR) {
            float m = s_stat[tid];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) m = fmaxf(m, s_stat[w * 8 + tid]);
            s_m[tid] = m;
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < NR; ++h) {
            float p = 0.f;
            if (ok) {
                p = __expf(s_p[tid * 8 + h] - s_m[h]);
                s_p[tid * 8 + h] = p;
            }
            p = wave_sum(p);
            if (lane == 0) s_stat[kWaves * 8 + wave * 8 + h] = p;
        }
        __syncthreads();
        if (tid < NR) {
            float l = 0.f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) l += s_stat[kWaves * 8 + w * 8 + tid];
            s_l[tid] = l;
        }
    }

    // ---- o = sum_t p_t v_t over the split's rows (PV pass)
    float o[NR][4];
#pragma unroll
    for (int h = 0; h < NR; ++h) o[h][0] = o[h][1] = o[h][2] = o[h][3] = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int row = wave * (T / kWaves) + i * G::VRW + vr;
        if (row < nrows) {
            float4 vv = vreg[i];
            if (row == new_local) vv = ld4(&s_vnew[vc4 * 4]);
            const float4 p0 = ld4(&s_p[row * 8]);
            const float4 p1 = ld4(&s_p[row * 8 + 4]);
            const float pp[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
            for (int h = 0; h < NR; ++h) {
                o[h][0] = fmaf(pp[h], vv.x, o[h][0]);
                o[h][1] = fmaf(pp[h], vv.y, o[h][1]);
                o[h][2] = fmaf(pp[h], vv.z, o[h][2]);
                o[h][3] = fmaf(pp[h], vv.w, o[h][3]);
            }
        }
    }
#pragma unroll
    for (int off = G::VL; off < 64; off <<= 1)
#pragma unroll
        for (int h = 0; h < NR; ++h)
#pragma unroll
            for (int e = 0; e < 4; ++e) o[h][e] += __shfl_xor(o[h][e], off);
    if (vr == 0) {
#pragma unroll
        for (int h = 0; h < NR; ++h)
            st4(&s_red[(wave * NR + h) * HD + vc4 * 4], make_float4(o[h][0], o[h][1], o[h][2], o[h][3]));
    }
    __syncthreads();

    const bool single = a.n_split == 1;
    for (int idx = tid; idx < NR * HD; idx += kThreads) {
        float sum = s_red[idx];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) sum += s_red[w * NR * HD + idx];
        const int h = idx / HD, d = idx - h * HD;
        const size_t hg = (size_t)g * a.n_rep + h;
        if (single) a.out[hg * HD + d] = sum / s_l[h];
        else a.part_o[(hg * a.n_split + split) * HD + d] = sum;
    }
    if (single) return;
    if (tid < NR) {
        const size_t hg = (size_t)g * a.n_rep + tid;
        a.part_ml[(hg * a.n_split + split) * 2 + 0] = s_m[tid];
        a.part_ml[(hg * a.n_split + split) * 2 + 1] = s_l[tid];
    }

    // ---- last workgroup of this kv-head merges the splits
    __threadfence();
    __syncthreads();
    if (tid == 0) s_ticket = atomicAdd(&a.counters[g], 1u);
    __syncthreads();
    if (s_ticket != (unsigned)(a.n_split - 1)) return;
    __threadfence();

    const int S = a.n_split;
    float *s_w = s_red;  // [NR][SMAX] normalised split weights
    for (int h = wave; h < NR; h += kWaves) {
        const float *ml = a.part_ml + ((size_t)g * a.n_rep + h) * S * 2;
        float m = -INFINITY;
        for (int s = lane; s < S; s += 64) m = fmaxf(m, ml[2 * s]);
        m = wave_max(m);
        float den = 0.f;
        for (int s = lane; s < S; s += 64) {
            const float w = __expf(ml[2 * s] - m);
            s_w[h * G::SMAX + s] = w;
            den = fmaf(w, ml[2 * s + 1], den);
        }
        den = wave_sum(den);
        const float inv = 1.f / den;
        for (int s = lane; s < S; s += 64) s_w[h * G::SMAX + s] *= inv;
    }
    __syncthreads();
    for (int idx = tid; idx < NR * (HD / 4); idx += kThreads) {
        const int h = idx / (HD / 4), d4 = idx - h * (HD / 4);
        const size_t hg = (size_t)g * a.n_rep + h;
        const float *po = a.part_o + hg * S * HD + d4 * 4;
        float4 acc = zero4();
#pragma unroll 8
        for (int s = 0; s < S; ++s) {
            const float w = s_w[h * G::SMAX + s];
            const float4 x = ld4(po + (size_t)s * HD);
            acc.x = fmaf(w, x.x, acc.x);
            acc.y = fmaf(w, x.y, acc.y);
            acc.z = fmaf(w, x.z, acc.z);
            acc.w = fmaf(w, x.w, acc.w);
        }
        st4(a.out + hg * HD + d4 * 4, acc);
    }
    if (tid == 0) atomicExch(&a.counters[g], 0u);
}

// ------------------------------------------------------------------ append

// Block (token z, kv-head g): k row rotated at position pos0+z and stored,
// v row copied (kore.cpp:1536-1538).  Slot = position (a prefill never wraps).
__global__ void append_kernel(AppendArgs a, int hd) {
    const int z = blockIdx.x, g = blockIdx.y, half = hd / 2;
    const int pos = a.pos0 + z;
    const float *kin = a.k + ((size_t)z * a.n_head_kv + g) * hd;
    const float *vin = a.v + ((size_t)z * a.n_head_kv + g) * hd;
    const float2 *cs = a.cs + (size_t)pos * half;
    float *kd = a.kc + ((size_t)g * a.slots + pos) * hd;
    float *vd = a.vc + ((size_t)g * a.slots + pos) * hd;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        float y0, y1;
        rope_pair(kin[i], kin[i + half], cs[i], y0, y1);
        kd[i] = y0;
        kd[i + half] = y1;
    }
    for (int i = threadIdx.x; i < hd; i += blockDim.x) vd[i] = vin[i];
}

// ----------------------------------------------------------------- prefill

// v_mfma_f32_32x32x2_f32, one block: lane l supplies A[l%32][l/32] and
// B[l/32][l%32]; D register r of lane l is D[8(r/4) + 4(l/32) + r%4][l%32].
__device__ __forceinline__ floatx16 mfma32(float a, float b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Workgroup = 4 waves of one kv-head g; wave w takes entry 4*item + w of g's
// list of (strip, q-head) pairs ordered by strip descending, so the waves of
// a workgroup attend the same key range (to within one tile) and share each
// K / V tile from LDS.  A strip is 32 query rows.  Per 32-key tile a wave
// computes S^T = K Q^T (keys x queries, 64 MFMAs for hd 128) so that every
// lane owns the scores of one query, runs the online softmax in base 2 on
// them, and accumulates O^T += V^T P^T (64 MFMAs), whose D layout again gives
// each lane one query; the softmax statistics need one cross-lane exchange.
// K tile rows are padded to HD+4 floats and V^T rows to 36 floats so the
// 16-byte LDS reads of 32 different rows fall in different banks.
template <int HD>
__global__ __launch_bounds__(kThreads) void prefill_kernel(PrefillArgs a) {
    constexpr int BK = 32;
    constexpr int KSTR = HD + 4;
    constexpr int VSTR = BK + 4;
    constexpr int NT = HD / 32;
    constexpr int HALF = HD / 2;
    __shared__ __align__(16) float sK[BK * KSTR];
    __shared__ __align__(16) float sV[HD * VSTR];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nkv = a.n_head_kv;
    const int g = blockIdx.x % nkv;
    const int item = blockIdx.x / nkv;
    const int total = a.n_rep * a.n_strips;
    const int e = item * 4 + wave;
    const bool active = e < total;
    const int ee = active ? e : total - 1;
    const int strip = a.n_strips - 1 - ee / a.n_rep;
    const int h = g * a.n_rep + ee % a.n_rep;
    const int strip0 = a.n_strips - 1 - (item * 4) / a.n_rep;
    const int n_keys = a.pos0 + a.n_tok;
    const int wg_kmax = min(a.pos0 + 32 * strip0 + 31, n_keys - 1);
    const int my_kmax = active ? min(a.pos0 + 32 * strip + 31, n_keys - 1) : -1;
    const int n_tiles = wg_kmax / BK + 1;
    const int n_head = nkv * a.n_rep;

    const int qi = lane & 31, qg = lane >> 5;
    const int qrow = 32 * strip + qi;
    const bool qvalid = active && qrow < a.n_tok;
    const int qrow_c = min(qrow, a.n_tok - 1);
    const int qpos = a.pos0 + qrow_c;

    // Q^T operand: qreg[4j+e] = roped q[qrow][8j + 4qg + e]
    float qreg[HD / 2];
    {
        const float *qp = a.q + ((size_t)qrow_c * n_head + h) * HD;
        const float2 *cs = a.cs + (size_t)qpos * HALF;
#pragma unroll
        for (int j = 0; j < HD / 16; ++j) {
            const int d = 8 * j + 4 * qg;
            const float4 lo = qvalid ? ld4(qp + d) : zero4();
            const float4 hi = qvalid ? ld4(qp + HALF + d) : zero4();
#pragma unroll
            for (int e2 = 0; e2 < 4; ++e2) {
                float y0, y1;
                rope_pair(comp(lo, e2), comp(hi, e2), cs[d + e2], y0, y1);
                qreg[4 * j + e2] = y0;
                qreg[4 * (j + HD / 16) + e2] = y1;
            }
        }
    }

    floatx16 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;

    for (int t = 0; t < n_tiles; ++t) {
        const int k0 = t * BK;
        __syncthreads();
        for (int idx = tid; idx < BK * HD / 4; idx += kThreads) {
            const int key = idx / (HD / 4), c4 = idx - key * (HD / 4);
            const int kp = k0 + key;
            float4 kv = zero4(), vv = zero4();
            if (kp < n_keys) {
                const size_t off = ((size_t)g * a.slots + kp) * HD + c4 * 4;
                kv = ld4(a.kc + off);
                vv = ld4(a.vc + off);
            }
            st4(&sK[key * KSTR + c4 * 4], kv);
            sV[(c4 * 4 + 0) * VSTR + key] = vv.x;
            sV[(c4 * 4 + 1) * VSTR + key] = vv.y;
            sV[(c4 * 4 + 2) * VSTR + key] = vv.z;
            sV[(c4 * 4 + 3) * VSTR + key] = vv.w;
        }
        __syncthreads();
        if (k0 > my_kmax) continue;

        floatx16 s;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
        for (int j = 0; j < HD / 8; ++j) {
            const float4 a4 = ld4(&sK[qi * KSTR + 8 * j + 4 * qg]);
            s = mfma32(a4.x, qreg[4 * j + 0], s);
            s = mfma32(a4.y, qreg[4 * j + 1], s);
            s = mfma32(a4.z, qreg[4 * j + 2], s);
            s = mfma32(a4.w, qreg[4 * j + 3], s);
        }
        // s[r] = score(query qi, key k0 + 8(r/4) + 4qg + r%4)
        float mt = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = k0 + 8 * (r / 4) + 4 * qg + (r % 4);
            const float x = key > qpos ? -INFINITY : s[r] * a.scale_log2;
            s[r] = x;
            mt = fmaxf(mt, x);
        }
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float m_new = fmaxf(m_run, mt);
        const float alpha = exp2f(m_run - m_new);
        float psum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            s[r] = exp2f(s[r] - m_new);
            psum += s[r];
        }
        psum += __shfl_xor(psum, 32);
        l_run = fmaf(l_run, alpha, psum);
        m_run = m_new;
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[tt][r] *= alpha;
#pragma unroll
            for (int sb = 0; sb < 4; ++sb) {
                const float4 a4 = ld4(&sV[(32 * tt + qi) * VSTR + 8 * sb + 4 * qg]);
                acc[tt] = mfma32(a4.x, s[4 * sb + 0], acc[tt]);
                acc[tt] = mfma32(a4.y, s[4 * sb + 1], acc[tt]);
                acc[tt] = mfma32(a4.z, s[4 * sb + 2], acc[tt]);
                acc[tt] = mfma32(a4.w, s[4 * sb + 3], acc[tt]);
            }
        }
    }

    if (qvalid) {
        const float inv = 1.f / l_run;
        float *op = a.out + ((size_t)qrow * n_head + h) * HD;
#pragma unroll
        for (int tt = 0; tt < NT; ++tt)
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
                st4(op + 32 * tt + 8 * rb + 4 * qg,
                    make_float4(acc[tt][4 * rb + 0] * inv, acc[tt][4 * rb + 1] * inv,
                                acc[tt][4 * rb + 2] * inv, acc[tt][4 * rb + 3] * inv));
    }
}

// ------------------------------------------------------------------- synth

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Irwin-Hall(12) of splitmix64 24-bit uniforms; the exact construction is
// stated with the CPU generator (oracle/kore_oracle.c) and both must agree
// bit for bit.
__global__ void synth_kernel(SynthArgs a, uint64_t key, uint64_t okey) {
    const size_t n = (size_t)a.rows * a.dim;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        const uint64_t r = i / (uint64_t)a.dim, c = i - r * (uint64_t)a.dim;
        const uint64_t idx = (a.row0 + r) * (uint64_t)a.dim + c;
        int64_t sum = 0;
#pragma unroll
        for (uint64_t k = 0; k < 6; ++k) {
            const uint64_t h = splitmix64(key ^ (idx * 8u + k));
            sum += (int64_t)(h & 0xFFFFFFu) + (int64_t)((h >> 32) & 0xFFFFFFu);
        }
        const int32_t centred = (int32_t)(sum - 6 * (int64_t)0x1000000);
        float x = (float)centred * (1.0f / 16777216.0f);
        if (a.per_mille) {
            const uint64_t h = splitmix64(okey ^ (a.tensor << 32) ^ c);
            if ((uint32_t)(h % 1000u) < a.per_mille) x *= a.outlier_scale;
        }
        a.dst[i] = x;
    }
}

// --------------------------------------------------------------- dispatch

template <int HD, int NR>
hipError_t launch_decode_nr(const DecodeArgs &a, hipStream_t s) {
    using G = DecodeGeom<HD>;
    const dim3 grid(a.n_split, a.n_head_kv);
    const int npass = a.rows_per_split / G::RPP;
    switch (npass) {
        case 1: hipLaunchKernelGGL((decode_kernel<HD, NR, 1>), grid, dim3(kThreads), 0, s, a); break;
        case 2: hipLaunchKernelGGL((decode_kernel<HD, NR, 2>), grid, dim3(kThreads), 0, s, a); break;
        case 4:
            if constexpr (G::RPP * 4 <= kThreads) {
                hipLaunchKernelGGL((decode_kernel<HD, NR, 4>), grid, dim3(kThreads), 0, s, a);
                break;
            }
            return hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int HD>
hipError_t launch_decode_hd(const DecodeArgs &a, hipStream_t s) {
    switch (a.n_rep) {
        case 1: return launch_decode_nr<HD, 1>(a, s);
        case 2: return launch_decode_nr<HD, 2>(a, s);
        case 3: return launch_decode_nr<HD, 3>(a, s);
        case 4: return launch_decode_nr<HD, 4>(a, s);
        case 5: return launch_decode_nr<HD, 5>(a, s);
        case 6: return launch_decode_nr<HD, 6>(a, s);
        case 7: return launch_decode_nr<HD, 7>(a, s);
        case 8: return launch_decode_nr<HD, 8>(a, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool decode_supported(int head_dim, int n_rep) {
    return (head_dim == 64 || head_dim == 128) && n_rep >= 1 && n_rep <= 8;
}

bool prefill_supported(int head_dim, int n_rep) {
    return (head_dim == 64 || head_dim == 128) && n_rep >= 1;
}

int decode_rows_per_split(int head_dim, int n_attend, int n_head_kv, int num_cu) {
    // Candidates (rows per workgroup) in decreasing order; take the largest
    // that still gives at least one workgroup per CU, and never more splits
    // than the merge can hold.
    const int rpp = head_dim == 128 ? DecodeGeom<128>::RPP : DecodeGeom<64>::RPP;
    const int smax = head_dim == 128 ? DecodeGeom<128>::SMAX : DecodeGeom<64>::SMAX;
    const int maxpass = (rpp * 4 <= kThreads) ? 4 : 2;
    int best = rpp;
    for (int np = maxpass; np >= 1; np >>= 1) {
        const int t = rpp * np;
        const int splits = (n_attend + t - 1) / t;
        if ((long)splits * n_head_kv >= num_cu) { best = t; break; }
        best = t;
    }
    while ((n_attend + best - 1) / best > smax && best < rpp * maxpass) best *= 2;
    return best;
}

hipError_t launch_decode(const DecodeArgs &a, int head_dim, hipStream_t s) {
    if (head_dim == 128) return launch_decode_hd<128>(a, s);
    if (head_dim == 64) return launch_decode_hd<64>(a, s);
    return hipErrorInvalidValue;
}

hipError_t launch_append(const AppendArgs &a, int head_dim, hipStream_t s) {
    const dim3 grid(a.n_tok, a.n_head_kv);
    const int threads = head_dim / 2 >= 64 ? 64 : (head_dim / 2 > 0 ? head_dim / 2 : 1);
    hipLaunchKernelGGL(append_kernel, grid, dim3(threads), 0, s, a, head_dim);
    return hipGetLastError();
}

hipError_t launch_prefill(const PrefillArgs &a, int head_dim, hipStream_t s) {
    const int items = (a.n_rep * a.n_strips + 3) / 4;
    const dim3 grid(items * a.n_head_kv);
    if (head_dim == 128) hipLaunchKernelGGL(prefill_kernel<128>, grid, dim3(kThreads), 0, s, a);
    else if (head_dim == 64) hipLaunchKernelGGL(prefill_kernel<64>, grid, dim3(kThreads), 0, s, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_synth(const SynthArgs &a, hipStream_t s) {
    auto mix = [](uint64_t x) {
        uint64_t z = x + 0x9E3779B97F4A7C15ull;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    };
    const uint64_t key = mix(mix(a.seed) ^ a.stream);
    const uint64_t okey = mix(a.seed ^ 0x00571E50ull);
    const size_t n = (size_t)a.rows * a.dim;
    if (n == 0) return hipSuccess;
    size_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(synth_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a, key, okey);
    return hipGetLastError();
}

}  // namespace kore_attn_gpu
