// kore_attn_kernels.hip - gfx950 (CDNA4) kernels of kore's attention path.
//
//   decode_split_kernel    single-token decode of one layer: RoPE of q and k
//                          (kore.cpp:1424-1425), append of the new k/v row
//                          (kore.cpp:1427-1430) and flash-decoding attention
//                          (kore.cpp:1432-1455) of each (kv-head, split) of
//                          the cache.  HBM-bound: every K/V byte is read once
//                          per kv-head (not once per q-head as kore's
//                          head-outer loop does) with 16-byte loads issued
//                          before any arithmetic.
//   decode_combine_kernel  log-sum-exp merge of the split partials, one
//                          workgroup per (q-head, 16 dims): a second launch
//                          instead of a last-workgroup merge, because a
//                          device-scope fence costs an L2 write-back on every
//                          workgroup and one workgroup reading every partial
//                          serialises the merge.
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

#include <algorithm>
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


// Cross-lane moves inside a 16-lane DPP row (no LDS traffic).  CTRL is a
// DPP control word: 0x121..0x12F rotate the row right by 1..15 lanes,
// 0x141 mirrors each half-row of 8 lanes, 0x00..0xFF permute within quads.
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
// Sum over the aligned group of N lanes (N = 4, 8 or 16) that contains this
// lane; every lane of the group receives it.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
    static_assert(N == 4 || N == 8 || N == 16, "DPP group of 4, 8 or 16 lanes");
    if constexpr (N == 16) {
        x += dpp<0x128>(x);   // row_ror:8
        x += dpp<0x124>(x);   // row_ror:4
    } else if constexpr (N == 8) {
        x += dpp<0x141>(x);   // row_half_mirror: lane i + lane 7-i of each half-row
    }
    if constexpr (N == 16) {
        x += dpp<0x122>(x);   // row_ror:2
        x += dpp<0x121>(x);   // row_ror:1
    } else {
        x += dpp<0xB1>(x);    // quad_perm [1,0,3,2]
        x += dpp<0x4E>(x);    // quad_perm [2,3,0,1]
    }
    return x;
}

// Max / sum over the 64 lanes of a value that is uniform within each aligned
// group of N lanes (N = 8 or 16); every lane receives the result.  The
// groups of a 16-lane row are folded with DPP, the four rows with v_readlane
// (no LDS traffic).
template <int N>
__device__ __forceinline__ float wave_max_groups(float x) {
    static_assert(N == 8 || N == 16, "groups of 8 or 16 lanes");
    if constexpr (N == 8) x = fmaxf(x, dpp<0x128>(x));   // row_ror:8 pairs the two half-rows
    const int i = __builtin_bit_cast(int, x);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}
template <int N>
__device__ __forceinline__ float wave_sum_groups(float x) {
    static_assert(N == 8 || N == 16, "groups of 8 or 16 lanes");
    if constexpr (N == 8) x += dpp<0x128>(x);
    const int i = __builtin_bit_cast(int, x);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(i, 48));
    return (r0 + r1) + (r2 + r3);
}
// Max over each 16-lane row; every lane of the row receives it.
__device__ __forceinline__ float row16_max(float x) {
    x = fmaxf(x, dpp<0x128>(x));
    x = fmaxf(x, dpp<0x124>(x));
    x = fmaxf(x, dpp<0x122>(x));
    return fmaxf(x, dpp<0x121>(x));
}
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
constexpr float kLog2e = 1.4426950408889634f;

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
    static constexpr int RW = kDecodeTile / kWaves;               // rows of a full tile per wave
    static constexpr int LPR = HD / 8;                            // lanes per K row (8 floats each)
    static constexpr int RPW = 64 / LPR;                          // K rows per wave per pass
    static constexpr int KPASS = RW / RPW;                        // K passes of a full tile
    static constexpr int VL = HD / 4;                             // lanes per V row (one float4 each)
    static constexpr int VRW = 64 / VL;                           // V rows per wave per load
    static constexpr int VLD = RW / VRW;                          // V loads per thread of a full tile
    static_assert(KPASS >= 1 && VLD >= 1 && (LPR == 8 || LPR == 16), "unsupported head_dim");
};

// Workgroup (split, kv-head g): cache slots [r0, r_end) of kv-head g for the
// NR q-heads of g, so every K/V byte is read once per kv-head (kore's
// head-outer loop, kore.cpp:1432, reads it once per q-head).  The slots are
// processed in tiles of kDecodeTile rows, the last of which may carry up to
// kWaves extra rows (row 64 + w goes to wave w as one more, mostly masked
// pass); that lets the host give every CU exactly one workgroup when the row
// count is a little above a multiple of 64 per CU.  Wave w owns rows
// [16w, 16w + 16) of a tile and keeps its own online softmax (max, sum,
// output) over them, so the tile loop has no workgroup barrier.  A tile's K
// and V rows are loaded into registers by unconditional 16-byte loads (rows
// past the end are clamped to the last row and masked afterwards), issued
// before any arithmetic and consumed in issue order.
//   score pass: LPR lanes per K row, each lane 8 of the row's floats (2 x
//               16 B loads at dims 4c + j*4*LPR) and the same dims of the NR
//               roped queries, pre-multiplied by 1/sqrt(hd) * log2(e) so the
//               softmax runs in base 2 on v_exp_f32; the partial dots are
//               summed over the LPR lanes with DPP, which leaves every lane
//               of a row group with the scores of its row.
//   softmax:    the running max of each head is wave-uniform (a max over the
//               row groups by v_readlane); the running sums stay per row
//               group until the end.
//   PV pass:    VL lanes per V row (one float4 each), VRW rows per wave per
//               load; the weights go through a wave-private LDS slice.
// The new token's row is not read from the cache: the owner workgroup ropes
// it, appends it, and adds it as one more softmax state (its own score, sum
// 1, output v) when the four wave states are merged.  Slots [0, n_rows) never
// include it except in a wrapped ring, where its stale slot is masked.
template <int HD, int NR>
__global__ __launch_bounds__(kThreads) void decode_split_kernel(DecodeArgs a) {
    using G = DecodeGeom<HD>;
    constexpr int TILE = kDecodeTile;
    constexpr int HALF = HD / 2;
    constexpr int NPAIR = (NR * HALF + kThreads - 1) / kThreads;   // q RoPE pairs per thread
    constexpr int NST = kWaves + 1;                                // softmax states merged at the end
    constexpr int KP = G::KPASS + 1;                               // passes incl. the extra-row pass
    constexpr int VP = G::VLD + 1;
    static_assert(NR >= 1 && NR <= 8, "at most 8 q-heads per workgroup");

    __shared__ __align__(16) float s_q[NR * HD];           // roped q * scale * log2(e)
    __shared__ __align__(16) float s_knew[HD];
    __shared__ __align__(16) float s_p[(TILE + kWaves) * 8];   // [row][head] weights, wave-private rows
    __shared__ __align__(16) float s_red[NST * NR * HD];   // per state: unnormalised output
    __shared__ float s_wm[NST * 8], s_wl[NST * 8], s_we[NST * 8], s_hm[8], s_hl[8];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int split = blockIdx.x, g = blockIdx.y;
    const int r0 = split * a.rows_per_split;
    const int r_end = min(r0 + a.rows_per_split, a.n_rows);
    const int n_own = max(r_end - r0, 0);
    const int n_tiles = n_own == 0 ? 0 : max(1, (n_own - kWaves + TILE - 1) / TILE);
    const int last_row = max(r_end - 1, 0);
    const int owner = a.n_rows == 0 ? 0 : min(a.new_slot, a.n_rows - 1) / a.rows_per_split;
    const bool is_owner = split == owner;
    const size_t head_base = (size_t)g * a.slots * HD;
    const float *kg = a.kc + head_base;
    const float *vg = a.vc + head_base;
    const int c = lane % G::LPR, rw = lane / G::LPR;
    const int vc4 = lane % G::VL, vr = lane / G::VL;
    const float qscale = a.scale * kLog2e;

    // ---- loads: q pairs and their cos/sin first (needed first), then the
    // first tile of K and V (every load in bounds, consumed in issue order).
    float qx0[NPAIR], qx1[NPAIR];
    float2 qcs[NPAIR];
#pragma unroll
    for (int it = 0; it < NPAIR; ++it) {
        const int idx = min(tid + it * kThreads, NR * HALF - 1);
        const int h = idx / HALF, i = idx - h * HALF;
        const float *qh = a.q + (size_t)(g * a.n_rep + h) * HD;
        qx0[it] = qh[i];
        qx1[it] = qh[i + HALF];
        qcs[it] = a.cs[i];
    }
    // the new k/v row (used by the owner workgroup only; loaded by all so
    // that no load is conditional): thread i < HALF takes pair i of k and
    // elements i, i + HALF of v
    const int ni = tid % HALF;
    const float nk0 = a.k[(size_t)g * HD + ni], nk1 = a.k[(size_t)g * HD + ni + HALF];
    const float2 ncs = a.cs[ni];
    const float nv0 = a.v[(size_t)g * HD + ni], nv1 = a.v[(size_t)g * HD + ni + HALF];
    __builtin_amdgcn_sched_barrier(0);   // keep these loads ahead of the K/V tile
    float4 kreg[KP][2];
    float4 vreg[VP];
    // tile row of K pass ps (the last pass is row TILE + wave) / of V load i
    auto krow = [&](int ps) { return ps < G::KPASS ? wave * G::RW + ps * G::RPW + rw : TILE + wave; };
    auto vrow = [&](int i) { return i < G::VLD ? wave * G::RW + i * G::VRW + vr : TILE + wave; };
    // The extra-row loads are issued even when the tile has no extra rows:
    // they are then clamped to the tile's last row, which the tile loads
    // anyway, so they cost cache hits only, and the loads stay unconditional
    // (exact in-order wait counts).
    auto load_tile = [&](int t0) {
#pragma unroll
        for (int ps = 0; ps < KP; ++ps) {
            const int r = min(t0 + krow(ps), last_row);
            const float *p = kg + (size_t)r * HD + c * 4;
#pragma unroll
            for (int j = 0; j < 2; ++j) kreg[ps][j] = ld4(p + j * (G::LPR * 4));
        }
#pragma unroll
        for (int i = 0; i < VP; ++i) {
            const int r = min(t0 + vrow(i), last_row);
            vreg[i] = ld4(vg + (size_t)r * HD + vc4 * 4);
        }
    };
    load_tile(r0);

    // ---- RoPE of this group's q heads (stored pre-scaled for the scores);
    // RoPE + append of the new k/v row.
#pragma unroll
    for (int it = 0; it < NPAIR; ++it) {
        const int idx = tid + it * kThreads;
        if (idx < NR * HALF) {
            const int h = idx / HALF, i = idx - h * HALF;
            float y0, y1;
            rope_pair(qx0[it], qx1[it], qcs[it], y0, y1);
            s_q[h * HD + i] = y0 * qscale;
            s_q[h * HD + i + HALF] = y1 * qscale;
        }
    }
    if (is_owner && tid < HALF) {
        float *kd = a.kc + head_base + (size_t)a.new_slot * HD;
        float *vd = a.vc + head_base + (size_t)a.new_slot * HD;
        float y0, y1;
        rope_pair(nk0, nk1, ncs, y0, y1);
        s_knew[ni] = y0;
        s_knew[ni + HALF] = y1;
        kd[ni] = y0;
        kd[ni + HALF] = y1;
        s_red[(kWaves * NR) * HD + ni] = nv0;          // state kWaves: v of the new row
        s_red[(kWaves * NR) * HD + ni + HALF] = nv1;
        vd[ni] = nv0;
        vd[ni + HALF] = nv1;
    }
    __syncthreads();

    float qv[NR][8];
#pragma unroll
    for (int h = 0; h < NR; ++h)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const float4 t = ld4(&s_q[h * HD + j * (G::LPR * 4) + c * 4]);
            qv[h][4 * j + 0] = t.x;
            qv[h][4 * j + 1] = t.y;
            qv[h][4 * j + 2] = t.z;
            qv[h][4 * j + 3] = t.w;
        }
    float o[NR][4];
    float m_run[NR], l_run[NR];
#pragma unroll
    for (int h = 0; h < NR; ++h) {
        o[h][0] = o[h][1] = o[h][2] = o[h][3] = 0.f;
        m_run[h] = -INFINITY;
        l_run[h] = 0.f;
    }

    for (int t = 0; t < n_tiles; ++t) {
        const int t0 = r0 + t * TILE;
        const bool last = t + 1 == n_tiles;
        const bool extra = last && n_own - t * TILE > TILE;
        if (t > 0) load_tile(t0);
        const int nrows = last ? r_end - t0 : TILE;
        const int skip = a.new_slot - t0;   // a wrapped ring's stale copy of the new slot
        const int npass = extra ? KP : G::KPASS;

        // ---- scores (log2 domain): s = (q . k) / sqrt(hd) * log2(e)
        float sc[KP][NR];
#pragma unroll
        for (int ps = 0; ps < KP; ++ps) {
            if (ps >= npass) {
#pragma unroll
                for (int h = 0; h < NR; ++h) sc[ps][h] = -INFINITY;
                continue;
            }
            const int row = krow(ps);
            const bool ok = row < nrows && row != skip && (ps < G::KPASS || rw == 0);
#pragma unroll
            for (int h = 0; h < NR; ++h) {
                float s = 0.f;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    s = fmaf(qv[h][4 * j + 0], kreg[ps][j].x, s);
                    s = fmaf(qv[h][4 * j + 1], kreg[ps][j].y, s);
                    s = fmaf(qv[h][4 * j + 2], kreg[ps][j].z, s);
                    s = fmaf(qv[h][4 * j + 3], kreg[ps][j].w, s);
                }
                s = group_sum<G::LPR>(s);
                sc[ps][h] = ok ? s : -INFINITY;
            }
        }

        // ---- online softmax: wave-uniform running max, per-group sums
        float alpha[NR];
#pragma unroll
        for (int h = 0; h < NR; ++h) {
            float mt = sc[0][h];
#pragma unroll
            for (int ps = 1; ps < KP; ++ps) mt = fmaxf(mt, sc[ps][h]);
            const float m_new = fmaxf(m_run[h], wave_max_groups<G::LPR>(mt));
            float lt = 0.f;
#pragma unroll
            for (int ps = 0; ps < KP; ++ps) {
                const float p = sc[ps][h] == -INFINITY ? 0.f : fast_exp2(sc[ps][h] - m_new);
                sc[ps][h] = p;
                lt += p;
            }
            alpha[h] = m_run[h] == -INFINITY ? 0.f : fast_exp2(m_run[h] - m_new);
            l_run[h] = fmaf(l_run[h], alpha[h], lt);
            m_run[h] = m_new;
        }
        // weights of the wave's rows to its LDS slice: lane c == 0 of each row
        if (c == 0) {
#pragma unroll
            for (int ps = 0; ps < KP; ++ps) {
                if (ps < npass && (ps < G::KPASS || rw == 0)) {
                    float pw[8];
#pragma unroll
                    for (int h = 0; h < 8; ++h) pw[h] = h < NR ? sc[ps][h] : 0.f;
                    float *dst = &s_p[krow(ps) * 8];
                    st4(dst, make_float4(pw[0], pw[1], pw[2], pw[3]));
                    st4(dst + 4, make_float4(pw[4], pw[5], pw[6], pw[7]));
                }
            }
        }

        // ---- o = alpha * o + sum_t p_t v_t over the wave's rows
        if (t > 0) {
#pragma unroll
            for (int h = 0; h < NR; ++h) {
                o[h][0] *= alpha[h];
                o[h][1] *= alpha[h];
                o[h][2] *= alpha[h];
                o[h][3] *= alpha[h];
            }
        }
#pragma unroll
        for (int i = 0; i < VP; ++i) {
            if (i < G::VLD || (extra && vr == 0)) {
                const int row = vrow(i);
                const float4 vv = vreg[i];
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
    }

    // ---- the wave's state: o summed over the lanes sharing dims, l over
    // the row groups; then the four wave states and the new row's are merged
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
#pragma unroll
    for (int h = 0; h < NR; ++h) {
        const float lw = wave_sum_groups<G::LPR>(l_run[h]);
        if (lane == 0) {
            s_wm[wave * 8 + h] = m_run[h];
            s_wl[wave * 8 + h] = lw;
        }
    }
    if (is_owner) {
        // score of the new row for head h (wave w takes heads w, w + 4):
        // lane-strided dot over the scaled roped q and the roped k, then a
        // wave sum
        for (int h = wave; h < NR; h += kWaves) {
            float s = 0.f;
            for (int d = lane; d < HD; d += 64) s = fmaf(s_q[h * HD + d], s_knew[d], s);
            s = wave_sum_groups<16>(group_sum<16>(s));
            if (lane == 0) {
                s_wm[kWaves * 8 + h] = s;
                s_wl[kWaves * 8 + h] = 1.f;
            }
        }
    }
    __syncthreads();
    const bool single = a.n_split == 1;
    if (tid < NR) {
        const int h = tid, nst = is_owner ? NST : kWaves;
        float m = -INFINITY;
        for (int w = 0; w < nst; ++w) m = fmaxf(m, s_wm[w * 8 + h]);
        float l = 0.f;
        for (int w = 0; w < NST; ++w) {
            const float mw = s_wm[w * 8 + h];
            const float e = (w >= nst || mw == -INFINITY) ? 0.f : fast_exp2(mw - m);
            s_we[w * 8 + h] = e;
            l = fmaf(e, s_wl[w * 8 + h], l);
        }
        if (single) {
            const float inv = 1.f / l;
            for (int w = 0; w < NST; ++w) s_we[w * 8 + h] *= inv;
        }
        s_hm[h] = m;
        s_hl[h] = l;
    }
    __syncthreads();
    for (int idx = tid; idx < NR * (HD / 4); idx += kThreads) {
        const int h = idx / (HD / 4), d4 = idx - h * (HD / 4);
        float4 acc = zero4();
#pragma unroll
        for (int w = 0; w < NST; ++w) {
            const float e = s_we[w * 8 + h];
            const float4 x = ld4(&s_red[(w < kWaves ? (w * NR + h) * HD : (kWaves * NR) * HD) + d4 * 4]);
            acc.x = fmaf(e, x.x, acc.x);
            acc.y = fmaf(e, x.y, acc.y);
            acc.z = fmaf(e, x.z, acc.z);
            acc.w = fmaf(e, x.w, acc.w);
        }
        const size_t hg = (size_t)g * a.n_rep + h;
        if (single) {
            st4(a.out + hg * HD + d4 * 4, acc);
        } else {
            st4(a.part_o + (hg * a.n_split + split) * HD + d4 * 4, acc);
            if (d4 == 0) {
                a.part_ml[(hg * a.n_split + split) * 2 + 0] = s_hm[h];
                a.part_ml[(hg * a.n_split + split) * 2 + 1] = s_hl[h];
            }
        }
    }
}

// Block (q-head h, 16-dim chunk): out[h][chunk] = sum_s w_s o_s / sum_s w_s l_s
// with w_s = 2^(m_s - max_s m_s) (split maxima are in the log2 domain), the
// log-sum-exp merge of the splits.  Lane (sub, c) takes splits sub + 16 i
// (i < 8, so n_split <= 128) and float4 c of the chunk; every load is issued
// before the first use.
template <int HD>
__global__ __launch_bounds__(64) void decode_combine_kernel(DecodeArgs a) {
    constexpr int PER = kMaxDecodeSplits / 16;
    const int h = blockIdx.x, chunk = blockIdx.y, lane = threadIdx.x;
    const int S = a.n_split;
    const int sub = lane >> 2, c = lane & 3;
    const float2 *ml = reinterpret_cast<const float2 *>(a.part_ml) + (size_t)h * S;
    const float *po = a.part_o + (size_t)h * S * HD + chunk * 16 + c * 4;
    float4 x[PER];
    float2 st[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int s = min(sub + 16 * i, S - 1);
        x[i] = ld4(po + (size_t)s * HD);
        st[i] = ml[s];
    }
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER; ++i) m = fmaxf(m, st[i].x);
    m = wave_max_groups<16>(row16_max(m));
    float4 acc = zero4();
    float den = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const float w = (sub + 16 * i < S) ? fast_exp2(st[i].x - m) : 0.f;
        den = fmaf(w, st[i].y, den);
        acc.x = fmaf(w, x[i].x, acc.x);
        acc.y = fmaf(w, x[i].y, acc.y);
        acc.z = fmaf(w, x[i].z, acc.z);
        acc.w = fmaf(w, x[i].w, acc.w);
    }
    // sum over sub (lane bits 2..5): the four subs of a row by DPP (rotations
    // by 8 and 4 keep c), the four rows by shuffles
    acc.x += dpp<0x128>(acc.x); acc.y += dpp<0x128>(acc.y); acc.z += dpp<0x128>(acc.z); acc.w += dpp<0x128>(acc.w);
    den += dpp<0x128>(den);
    acc.x += dpp<0x124>(acc.x); acc.y += dpp<0x124>(acc.y); acc.z += dpp<0x124>(acc.z); acc.w += dpp<0x124>(acc.w);
    den += dpp<0x124>(den);
#pragma unroll
    for (int off = 16; off < 64; off <<= 1) {
        acc.x += __shfl_xor(acc.x, off);
        acc.y += __shfl_xor(acc.y, off);
        acc.z += __shfl_xor(acc.z, off);
        acc.w += __shfl_xor(acc.w, off);
        den += __shfl_xor(den, off);
    }
    if (sub == 0) {
        const float inv = 1.f / den;
        st4(a.out + (size_t)h * HD + chunk * 16 + c * 4,
            make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv));
    }
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
// 16-byte LDS reads of 32 different rows fall in different banks.  With key
// segments (a short chunk over a long cache has too few workgroups to fill the
// GPU) a workgroup covers one range of key tiles and writes its rows'
// unnormalised output with their max and sum instead.
template <int HD>
__global__ __launch_bounds__(kThreads, 2) void prefill_kernel(PrefillArgs a) {
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
    const int seg = (blockIdx.x / nkv) % a.n_kseg;
    const int item = blockIdx.x / nkv / a.n_kseg;
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

    const int t_begin = seg * a.seg_tiles;
    const int t_end = a.n_kseg == 1 ? n_tiles : min(n_tiles, t_begin + a.seg_tiles);
    for (int t = t_begin; t < t_end; ++t) {
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
        // a segment may start with a tile that is all masked for a row
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        const float alpha = exp2f(m_run - m_use);
        float psum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            s[r] = exp2f(s[r] - m_use);
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

    if (a.n_kseg > 1) {
        if (!active) return;
        const size_t pe = ((size_t)g * total + ee) * a.n_kseg + seg;
        float *po = a.part_o + (pe * 32 + qi) * HD;
#pragma unroll
        for (int tt = 0; tt < NT; ++tt)
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
                st4(po + 32 * tt + 8 * rb + 4 * qg,
                    make_float4(acc[tt][4 * rb + 0], acc[tt][4 * rb + 1], acc[tt][4 * rb + 2], acc[tt][4 * rb + 3]));
        if (qg == 0) {
            a.part_ml[(pe * 32 + qi) * 2 + 0] = m_run;
            a.part_ml[(pe * 32 + qi) * 2 + 1] = l_run;
        }
        return;
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

// Block = one (kv-head, strip, q-head) entry of the prefill: the log-sum-exp
// merge of its key segments for 32 query rows; thread (row r, chunk c) owns
// 16 dims of one row.
template <int HD>
__global__ __launch_bounds__(256) void prefill_combine_kernel(PrefillArgs a) {
    constexpr int CH = HD / 8;                          // dims per thread
    const int entry = blockIdx.x;
    const int total = a.n_rep * a.n_strips;
    const int g = entry / total, e = entry - g * total;
    const int strip = a.n_strips - 1 - e / a.n_rep;
    const int h = g * a.n_rep + e % a.n_rep;
    const int r = threadIdx.x >> 3, c = threadIdx.x & 7;
    const int qrow = 32 * strip + r;
    if (qrow >= a.n_tok) return;
    const int S = a.n_kseg;
    const size_t base = (size_t)entry * S;
    float m = -INFINITY;
    for (int s = 0; s < S; ++s) m = fmaxf(m, a.part_ml[((base + s) * 32 + r) * 2]);
    float den = 0.f;
    float4 acc[CH / 4];
#pragma unroll
    for (int j = 0; j < CH / 4; ++j) acc[j] = zero4();
    for (int s = 0; s < S; ++s) {
        const float ms = a.part_ml[((base + s) * 32 + r) * 2];
        const float w = ms == -INFINITY ? 0.f : exp2f(ms - m);
        den = fmaf(w, a.part_ml[((base + s) * 32 + r) * 2 + 1], den);
        const float *po = a.part_o + ((base + s) * 32 + r) * HD + c * CH;
#pragma unroll
        for (int j = 0; j < CH / 4; ++j) {
            const float4 x = ld4(po + 4 * j);
            acc[j].x = fmaf(w, x.x, acc[j].x);
            acc[j].y = fmaf(w, x.y, acc[j].y);
            acc[j].z = fmaf(w, x.z, acc[j].z);
            acc[j].w = fmaf(w, x.w, acc[j].w);
        }
    }
    const float inv = 1.f / den;
    float *op = a.out + ((size_t)qrow * a.n_head_kv * a.n_rep + h) * HD + c * CH;
#pragma unroll
    for (int j = 0; j < CH / 4; ++j)
        st4(op + 4 * j, make_float4(acc[j].x * inv, acc[j].y * inv, acc[j].z * inv, acc[j].w * inv));
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
    hipLaunchKernelGGL((decode_split_kernel<HD, NR>), dim3(a.n_split, a.n_head_kv), dim3(kThreads), 0, s, a);
    if (a.n_split > 1)
        hipLaunchKernelGGL(decode_combine_kernel<HD>, dim3(a.n_head_kv * a.n_rep, HD / 16), dim3(64), 0, s, a);
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

int decode_rows_per_split(int head_dim, int n_rows, int n_head_kv, int num_cu) {
    // One workgroup per CU where the rows allow it: S splits per kv-head with
    // S = min(num_cu / n_head_kv, kMaxDecodeSplits).  Up to 64 * S rows use
    // 64-row splits; a little more gives S splits of 65..68 rows (one tile
    // plus an extra row per wave); beyond that the split grows to the next
    // size whose remainder over whole tiles is at most kWaves rows.
    (void)head_dim;
    const int S = std::max(1, std::min(num_cu / std::max(n_head_kv, 1), kMaxDecodeSplits));
    if (n_rows <= kDecodeTile * S) return kDecodeTile;
    int rps = (n_rows + S - 1) / S;
    if (rps % kDecodeTile > kWaves) rps = (rps + kDecodeTile - 1) / kDecodeTile * kDecodeTile;
    return rps;
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

int prefill_key_segments(int n_tok, int pos0, int n_head_kv, int n_rep, int num_cu, int *seg_tiles) {
    // Split the key range when the workgroups of a chunk do not fill every
    // CU (two fit per CU): as many segments as keep all of them in one wave
    // of two per CU, each of at least 8 key tiles.
    const int n_strips = (n_tok + 31) / 32;
    const int n_wg = (n_rep * n_strips + 3) / 4 * n_head_kv;
    const int n_tiles = (pos0 + n_tok - 1) / 32 + 1;
    int n_kseg = 1;
    if (n_wg < num_cu)
        n_kseg = std::max(1, std::min(2 * num_cu / n_wg, n_tiles / 8));
    *seg_tiles = (n_tiles + n_kseg - 1) / n_kseg;
    return n_kseg;
}

hipError_t launch_prefill(const PrefillArgs &a, int head_dim, hipStream_t s) {
    const int items = (a.n_rep * a.n_strips + 3) / 4;
    const dim3 grid(items * a.n_head_kv * a.n_kseg);
    if (head_dim == 128) hipLaunchKernelGGL(prefill_kernel<128>, grid, dim3(kThreads), 0, s, a);
    else if (head_dim == 64) hipLaunchKernelGGL(prefill_kernel<64>, grid, dim3(kThreads), 0, s, a);
    else return hipErrorInvalidValue;
    if (a.n_kseg > 1) {
        const dim3 cgrid(a.n_head_kv * a.n_rep * a.n_strips);
        if (head_dim == 128) hipLaunchKernelGGL(prefill_combine_kernel<128>, cgrid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL(prefill_combine_kernel<64>, cgrid, dim3(256), 0, s, a);
    }
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
