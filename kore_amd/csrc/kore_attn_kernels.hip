// kore_attn_kernels.hip - gfx950 (CDNA4) kernels of kore's attention path.
//
//   decode_split_kernel    single-token decode of one layer: RoPE of q and k
//                          (kore.cpp:1424-1425), append of the new k/v row
//                          (kore.cpp:1427-1430) and flash-decoding attention
//                          (kore.cpp:1432-1455) of each (kv-head, split) of
//                          the cache on fp32 MFMA (v_mfma_f32_16x16x4f32),
//                          16 rows per wave and block.  HBM-bound: every K/V
//                          byte is read once per kv-head (not once per q-head
//                          as kore's head-outer loop does) with 16-byte loads
//                          straight into the MFMA operands.
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
//   generic_*       every other geometry kore accepts (any even head_dim up
//                   to 256, any q-heads per kv-head): a decode prep launch
//                   (RoPE of q, RoPE + append of the new row), LDS-tiled
//                   attention on VALU with fp64 scores for decode splits and
//                   prefill rows, and the merge of the decode's split partials.
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
#include <mutex>
#include <vector>

namespace kore_attn_gpu {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr size_t kLdsPerCu = 160 * 1024;   // gfx950

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

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
// Max over each 16-lane row; every lane of the row receives it.
__device__ __forceinline__ float row16_max(float x) {
    x = fmaxf(x, dpp<0x128>(x));
    x = fmaxf(x, dpp<0x124>(x));
    x = fmaxf(x, dpp<0x122>(x));
    return fmaxf(x, dpp<0x121>(x));
}
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Timing build only (libkore_attn_tl.so, compiled with -DKORE_DECODE_TIMELINE;
// never the product library): every wave of the latest decode_split_kernel
// launch and every workgroup of the latest decode_combine_kernel launch keep
// s_memrealtime stamps (a 100 MHz counter shared by the whole device) in
// scalar registers and write them when they end, so the stamps add no memory
// operation between a kernel's loads and their uses.  kore_attn_tl_read()
// copies them out.
#ifdef KORE_DECODE_TIMELINE
constexpr int kTlStamps = 11;     // per split wave
constexpr int kTlWaves = 4096;
constexpr int kTlCombStamps = 3;  // per combine workgroup
constexpr int kTlComb = 2048;
__device__ unsigned long long g_tl_split[kTlWaves * kTlStamps];
__device__ unsigned long long g_tl_comb[kTlComb * kTlCombStamps];
#define TL_DECL(n) unsigned long long tl_[n] = {}
#define TL(i)                                      \
    do {                                           \
        __builtin_amdgcn_sched_barrier(0);         \
        tl_[i] = __builtin_amdgcn_s_memrealtime(); \
        __builtin_amdgcn_sched_barrier(0);         \
    } while (0)
#define TL_WRITE(buf, cap, id, n)                                                    \
    do {                                                                             \
        if ((threadIdx.x & 63) == 0 && (id) < (cap))                                 \
            for (int i_ = 0; i_ < (n); ++i_) buf[(size_t)(id) * (n) + i_] = tl_[i_]; \
    } while (0)
#else
#define TL_DECL(n) ((void)0)
#define TL(i) ((void)0)
#define TL_WRITE(buf, cap, id, n) ((void)0)
#endif

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

// v_mfma_f32_16x16x4f32, one block: lane l supplies A[l%16][l/16] and
// B[l/16][l%16]; D register v of lane l is D[4(l/16) + v][l%16].
__device__ __forceinline__ floatx4 mfma16(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// x of lane l and of lane l ^ 16 (v_permlane16_swap with x as both operands
// returns the even 16-lane rows in one result and the odd rows in the other),
// and likewise of lane l ^ 32 (v_permlane32_swap).  The results are copied
// to integers before the bit casts: a bit cast applied to an element of the
// returned vector directly is compiled as the first element by this hipcc
// (ROCm 7.2) for either index.
__device__ __forceinline__ void pair16(float x, float &a, float &b) {
    const unsigned xb = __builtin_bit_cast(unsigned, x);
    const auto r = __builtin_amdgcn_permlane16_swap(xb, xb, false, false);
    const unsigned r0 = r[0], r1 = r[1];
    a = __builtin_bit_cast(float, r0);
    b = __builtin_bit_cast(float, r1);
}
__device__ __forceinline__ void pair32(float x, float &a, float &b) {
    const unsigned xb = __builtin_bit_cast(unsigned, x);
    const auto r = __builtin_amdgcn_permlane32_swap(xb, xb, false, false);
    const unsigned r0 = r[0], r1 = r[1];
    a = __builtin_bit_cast(float, r0);
    b = __builtin_bit_cast(float, r1);
}
// Max / sum over the four lanes l % 16 + 16 k (k = 0..3); every one of them
// receives the same value (the operands are the same in all four lanes).
__device__ __forceinline__ float max4rows(float x) {
    float a, b;
    pair16(x, a, b);
    x = fmaxf(a, b);
    pair32(x, a, b);
    return fmaxf(a, b);
}
__device__ __forceinline__ float sum4rows(float x) {
    float a, b;
    pair16(x, a, b);
    x = a + b;
    pair32(x, a, b);
    return a + b;
}

// v_mfma_f64_4x4x4f64: four 4x4x4 blocks b; lane 16k + 4b + i supplies
// A_b[i][k], lane 16k + 4b + j supplies B_b[k][j], and lane 16i + 4b + j
// holds D_b[i][j] (checked on the GPU).  One instruction does a quarter of
// the products of v_mfma_f64_16x16x4f64 in under a third of its time.
__device__ __forceinline__ double mfma4d(double a, double b, double c) {
    return __builtin_amdgcn_mfma_f64_4x4x4f64(a, b, c, 0, 0, 0);
}

// Sum over the four lanes l % 16 + 16 k of a double (both 32-bit halves go
// through the permlane swaps).
__device__ __forceinline__ double sum4rows_d(double x) {
    auto pair = [](double v, bool p32, double &a, double &b) {
        const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
        const unsigned lo = (unsigned)u, hi = (unsigned)(u >> 32);
        const auto rl = p32 ? __builtin_amdgcn_permlane32_swap(lo, lo, false, false)
                            : __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
        const auto rh = p32 ? __builtin_amdgcn_permlane32_swap(hi, hi, false, false)
                            : __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
        const unsigned l0 = rl[0], l1 = rl[1], h0 = rh[0], h1 = rh[1];
        a = __builtin_bit_cast(double, ((unsigned long long)h0 << 32) | l0);
        b = __builtin_bit_cast(double, ((unsigned long long)h1 << 32) | l1);
    };
    double a, b;
    pair(x, false, a, b);
    x = a + b;
    pair(x, true, a, b);
    return a + b;
}

// Workgroup (split, kv-head g): cache slots [r0, r_end) of kv-head g for the
// NR q-heads of g, so every K/V byte is read once per kv-head (kore's
// head-outer loop, kore.cpp:1432, reads it once per q-head).  The slots are
// cut into blocks of 16 rows; wave w takes blocks w, w + 4, ... and keeps its
// own online softmax (max, sum, output) for all NR heads, so the block loop
// has no workgroup barrier.  Per block:
//   scores  S[row][head] = K[16 rows][hd] . q^T on fp64 MFMA
//           (v_mfma_f64_4x4x4f64): the four 4x4 blocks are the four groups
//           of 4 rows, the block columns 4 heads (two chains cover heads
//           0..3 and 4..7), and the k index picks one of four hd/4-dim
//           chunks, so lane l gives K[row l % 16][(hd/4)(l / 16) + 4t + e]
//           (contiguous 16-byte loads) and the roped q of heads l % 4 and
//           4 + l % 4 at the same dims, all widened to double (their products
//           are exact); the sums are scaled by kore's 1/sqrt(hd) and log2(e)
//           in double.  The scores reach a few hundred in the log2 domain on
//           heavy-tailed inputs, where an fp32 accumulation chain loses more
//           than kore's own rounding; in fp64 the products are exact and the
//           sum loses nothing that matters.  Lane l ends up with row
//           4((l / 4) % 4) + l / 16 of heads l % 4 and 4 + l % 4.
//   softmax the running max (fp32) and sum of each head over the 16 rows are
//           reductions over the 16 lanes that hold the head (DPP rotations
//           inside a 16-lane row, permlane swaps across rows); each weight is
//           2^(score - max) with the difference taken in fp64, then v_exp_f32.
//   values  O^T[dim][head] += V^T[dim][16 rows] . P on fp32 MFMA
//           (v_mfma_f32_16x16x4f32): k-step s takes rows 4s + k for lane
//           (m, k) = (l % 16, l / 16), which gives V[row 4s + k][64j + 4m + e]
//           (16-byte loads) for the output block 4j + e and P[row][head m];
//           the weights and the heads' rescale factors reach that layout
//           through 0.5 KB of the wave's LDS.
// Issue order of a wave: its q and the new k/v row, the K rows of its first
// block, then (once q has returned) the RoPE of q through the wave's own LDS
// rows, then the V rows, so the score MFMAs run while V streams in.  Every
// load before the first MFMA is unconditional (rows past the split's end
// are clamped to its last row and masked): a load under a branch makes the
// compiler's wait counts for everything after it conservative.  This kernel
// takes splits of at most one block per wave (plus kWaves extra rows);
// decode_multi_kernel takes the longer ones.
// The new token's row is not read from the cache: the owner workgroup ropes
// it, appends it, and adds it as one more softmax state (its own score, sum
// 1, output v).  Slots [0, n_rows) never include it except in a wrapped ring,
// where its stale slot is masked.  The four wave states (each started from
// the wave's single row) are merged in LDS into one partial per q-head, or
// into `out` when the kv-head has a single split.  Compiled for two
// workgroups per CU (at most 256 registers a wave: 240 at 7 q-heads per
// kv-head, no spills), which also runs faster at one workgroup per CU than
// the build with the whole register file (280 there): 7B at 4096 rows 8.14-
// 8.20 against 8.32-8.34 us per layer.
template <int HD, int NR>
__global__ __launch_bounds__(kThreads, 2) void decode_split_kernel(const float *__restrict__ q_in, float *kc_in,
                                                                float *vc_in, const float *__restrict__ k_in,
                                                                const float *__restrict__ v_in, int n_rows,
                                                                int rows_per_split, int new_slot, int slots,
                                                                DecodeArgs a, RopeRow rr) {
    constexpr int NT = HD / 16;    // K float4 per lane per block (MFMA k-steps / 4)
    constexpr int NJ = HD / 64;    // V float4 per lane per row
    constexpr int NMB = HD / 16;   // 16-dim output blocks
    constexpr int HALF = HD / 2;
    constexpr int NST = kWaves + 1;       // wave states, then single entry kWaves
    constexpr int CH = HD / 4;            // dims per lane of a K row (one k chunk)
    constexpr int NHG = NR > 4 ? 2 : 1;   // groups of 4 heads (score chains)
    constexpr int NEW_WAVE = kWaves - 1;  // the wave that takes the new row
    static_assert(NR >= 1 && NR <= 8, "at most 8 q-heads per workgroup");
    static_assert(HD == 64 || HD == 128, "head_dim 64 or 128");
    TL_DECL(kTlStamps);
    TL(0);

    constexpr int OST = HD + 4;    // LDS stride of a head's output (bank spread)
    __shared__ __align__(16) float s_o[kWaves * NR * OST];  // unnormalised wave outputs
    // single entries e = 0 .. kWaves: the extra rows, then the new row
    __shared__ __align__(16) float s_kx[(kWaves + 1) * HD];  // k (roped)
    __shared__ __align__(16) float s_vx[(kWaves + 1) * HD];  // v (zero where absent)
    __shared__ float s_m[NST * 8], s_l[NST * 8];
    __shared__ __align__(16) float s_p[kWaves * (8 * 16 + 8)];   // per wave: weights, rescale factors

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m16 = lane & 15, kq = lane >> 4;
    const int jq = lane & 3, bq = (lane >> 2) & 3, iq = lane >> 4;   // score layout: head, row group, row
    const int split = blockIdx.x, g = blockIdx.y;
    const int r0 = split * rows_per_split;
    const int r_end = min(r0 + rows_per_split, n_rows);
    const int n_own = max(r_end - r0, 0);
    // whole blocks, plus a last partial block of more than kWaves rows; a
    // remainder of at most kWaves rows is taken as extra rows, one per wave
    const int rem = n_own % kDecodeBlock;
    const int n_blk = n_own / kDecodeBlock + (rem > kWaves ? 1 : 0);
    const int n_extra = rem > kWaves ? 0 : rem;
    const int last_row = max(r_end - 1, 0);
    const int owner = n_rows == 0 ? 0 : min(new_slot, n_rows - 1) / rows_per_split;
    const bool is_owner = split == owner;
    const size_t head_base = (size_t)g * slots * HD;
    const float *kg = kc_in + head_base;
    const float *vg = vc_in + head_base;

    // ---- q of the NR heads of kv-head g, roped and pre-scaled by every wave
    // for itself and staged through the wave's own LDS rows, so no
    // workgroup barrier stands between a wave's loads and its first MFMA.
    // Pair p < NR * hd/8 of the wave is (q[h][4c..4c+3], q[h][hd/2 + 4c..])
    // with h = p / NC, c = p % NC; lane l takes pairs l and l + 64, which
    // share c = l % NC and so the four (cos, sin) pairs of dims 4c..4c+3.
    // The MFMA operand layout repeats every q value in 16/NR lanes and every
    // (cos, sin) pair in 16, so loading the operands directly would cost each
    // wave as much vector-memory traffic as its cache rows.
    constexpr int QS = HD + 4;                 // s_q row stride (bank spread)
    constexpr int NC = HALF / 4;               // float4 per half row
    constexpr int NP = (NR * NC + 63) / 64;    // pairs per lane
    static_assert(64 % NC == 0 && NP <= 2, "a lane's pairs share their (cos, sin) values");
    // per wave NR rows of roped q * 1/sqrt(hd) * log2(e), and one row that
    // takes the stores of lanes without a pair (so the stores need no branch)
    __shared__ __align__(16) float s_q[kWaves * (NR + 1) * QS];
    float *wq = s_q + wave * (NR + 1) * QS;
    const int sc = lane % NC;
    float4 sx0[NP], sx1[NP];
    const float4 scs01 = ld4(&rr.cs[8 * sc]), scs23 = ld4(&rr.cs[8 * sc + 4]);
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        const int sh = min((lane + 64 * i) / NC, NR - 1);
        const float *qh = q_in + (size_t)(g * NR + sh) * HD + 4 * sc;
        sx0[i] = ld4(qh);
        sx1[i] = ld4(qh + HALF);
    }
    TL(10);
    // the new k/v row and this wave's extra row, pair (i, i + hd/2) in lane
    // i: loaded by every lane of every wave (clamped rows), so that no load
    // is conditional, and ahead of the K rows, so that their scores are taken
    // while the cache rows stream in
    const int ni = min(lane, HALF - 1);
    const float nk0 = k_in[(size_t)g * HD + ni], nk1 = k_in[(size_t)g * HD + ni + HALF];
    const float nv0 = v_in[(size_t)g * HD + ni], nv1 = v_in[(size_t)g * HD + ni + HALF];
    const float2 ncs = *reinterpret_cast<const float2 *>(&rr.cs[2 * ni]);
    const int xrow = min(r0 + (n_own - n_extra) + wave, last_row);
    const float xk0 = kg[(size_t)xrow * HD + ni], xk1 = kg[(size_t)xrow * HD + ni + HALF];
    const float xv0 = vg[(size_t)xrow * HD + ni], xv1 = vg[(size_t)xrow * HD + ni + HALF];
    // the arguments the merge needs (read from the kernel-argument segment,
    // not preloaded)
    float *const out_p = a.out, *const part_o = a.part_o, *const part_ml = a.part_ml;
    const int n_split = a.n_split, n_rep = a.n_rep;

    float4 kA[NT], vA[4][NJ];
    auto load_k = [&](float4 *kf, int b) {
        const float *kr = kg + (size_t)min(r0 + 16 * b + m16, last_row) * HD + CH * kq;
#pragma unroll
        for (int t = 0; t < NT; ++t) kf[t] = ld4(kr + 4 * t);
    };
    auto load_v = [&](float4 (*vf)[NJ], int b) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const float *vr = vg + (size_t)min(r0 + 16 * b + 4 * s + kq, last_row) * HD + 4 * m16;
#pragma unroll
            for (int j = 0; j < NJ; ++j) vf[s][j] = ld4(vr + 64 * j);
        }
    };
    __builtin_amdgcn_sched_barrier(0);
    load_k(kA, wave);
    __builtin_amdgcn_sched_barrier(0);
    TL(1);
    // the merge arguments are waited for here, behind the K rows' requests: a
    // first read after the block loop would wait for a kernel-argument fetch
    // at the end of the kernel
    asm volatile("" ::"s"(out_p), "s"(part_o), "s"(part_ml), "s"(n_split), "s"(n_rep));

    // RoPE of the staged pairs into the wave's LDS rows, then the B operand:
    // lane l holds heads jq and jq + 4 (jq = l % 4) at dims CH kq + 4t + e
    // (heads past NR are zero); the dot products are widened to double and
    // scaled by kore's 1/sqrt(hd) and log2(e) there.
    const double qscale = (double)a.scale * 1.4426950408889634;
    float qb[NHG][NT][4];
    {
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int p = lane + 64 * i;
            const int row = p < NR * NC ? p / NC : NR;
            float y0[4], y1[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float4 c4 = e < 2 ? scs01 : scs23;
                const float2 cs = (e & 1) ? make_float2(c4.z, c4.w) : make_float2(c4.x, c4.y);
                rope_pair(comp(sx0[i], e), comp(sx1[i], e), cs, y0[e], y1[e]);
            }
            st4(&wq[row * QS + 4 * sc], make_float4(y0[0], y0[1], y0[2], y0[3]));
            st4(&wq[row * QS + HALF + 4 * sc], make_float4(y1[0], y1[1], y1[2], y1[3]));
        }
        __builtin_amdgcn_wave_barrier();
        // heads past NR read head NR - 1 and are zeroed by a bit mask: a
        // select of the loaded value became a read under a lane mask, each
        // waited for before the next
#pragma unroll
        for (int hg = 0; hg < NHG; ++hg) {
            const int h = jq + 4 * hg;
            const unsigned keep = h < NR ? 0xFFFFFFFFu : 0u;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const float4 qv = ld4(&wq[min(h, NR - 1) * QS + CH * kq + 4 * t]);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    qb[hg][t][e] = __builtin_bit_cast(float, __builtin_bit_cast(unsigned, comp(qv, e)) & keep);
            }
        }
    }
    TL(2);

    // dot of q (operand layout) with a k row staged in LDS, for heads jq + 4hg:
    // lane l sums its dims CH kq + 4t + e, then the four lanes of its chunk
    // row (l, l ^ 16, l ^ 32, l ^ 48) add up; every lane ends with the scores
    // (four independent partial sums per head group: a single chain of
    // dependent fp64 FMAs would take most of a microsecond)
    auto row_scores = [&](const float *kr, double (&out)[NHG]) {
        double sx[NHG][4];
#pragma unroll
        for (int hg = 0; hg < NHG; ++hg)
#pragma unroll
            for (int e = 0; e < 4; ++e) sx[hg][e] = 0.0;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float4 kx = ld4(&kr[CH * kq + 4 * t]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const double kd = (double)comp(kx, e);
#pragma unroll
                for (int hg = 0; hg < NHG; ++hg) sx[hg][e] = fma((double)qb[hg][t][e], kd, sx[hg][e]);
            }
        }
#pragma unroll
        for (int hg = 0; hg < NHG; ++hg)
            out[hg] = sum4rows_d((sx[hg][0] + sx[hg][1]) + (sx[hg][2] + sx[hg][3])) * qscale;
    };
    // A single row as a softmax state: max = its score rounded to fp32, sum
    // = 2^(score - max) with the difference in fp64 (about 1), output = that
    // sum times the row (the merge applies the sum to the stored v row).
    // ---- single entry `wave` (state kWaves + wave): extra row `wave` (from
    // the cache, roped already) while wave < n_extra, the new row (roped
    // here; it counts in the owner workgroup only) at wave == n_extra, none
    // after; entry kWaves (state 2 kWaves: the new row behind kWaves extra
    // rows) in NEW_WAVE.  So a wave scores one single row, NEW_WAVE a second
    // one only when the split ends in kWaves extra rows.  Absent entries hold
    // max -inf, sum 0 and a zero v row.  Only LDS and register work: no
    // memory operation under these branches.  The merge weighs each stored v
    // row with the state's sum.
    float nky0, nky1;
    rope_pair(nk0, nk1, ncs, nky0, nky1);
    auto single_state = [&](int st, bool on, const double (&sc)[NHG]) {
#pragma unroll
        for (int hg = 0; hg < NHG; ++hg) {
            const double sx = sc[hg];
            const int h = jq + 4 * hg;
            if (lane < 4 && h < NR) {
                const float mx = (float)sx;
                s_m[st * 8 + h] = on ? mx : -INFINITY;
                s_l[st * 8 + h] = on ? fast_exp2((float)(sx - (double)mx)) : 0.f;
            }
        }
    };
    // the wave's own entry: its scores stay in registers and become the
    // wave's initial softmax state below
    const bool e_on = (wave < n_extra && xrow != new_slot) || (wave == n_extra && is_owner);
    double sxs[NHG];
    {
        const bool x_is = wave < n_extra;
        if (lane < HALF) {
            s_kx[wave * HD + lane] = x_is ? xk0 : nky0;
            s_kx[wave * HD + lane + HALF] = x_is ? xk1 : nky1;
            s_vx[wave * HD + lane] = e_on ? (x_is ? xv0 : nv0) : 0.f;
            s_vx[wave * HD + lane + HALF] = e_on ? (x_is ? xv1 : nv1) : 0.f;
        }
        __builtin_amdgcn_wave_barrier();
        row_scores(&s_kx[wave * HD], sxs);
    }
    // entry kWaves exists only behind kWaves extra rows (uniform in the
    // workgroup); absent, nothing of it is written: the merge reads it but
    // uses it only when present
    if (wave == NEW_WAVE && n_extra == kWaves) {
        if (lane < HALF) {
            s_kx[kWaves * HD + lane] = nky0;
            s_kx[kWaves * HD + lane + HALF] = nky1;
            s_vx[kWaves * HD + lane] = is_owner ? nv0 : 0.f;
            s_vx[kWaves * HD + lane + HALF] = is_owner ? nv1 : 0.f;
        }
        __builtin_amdgcn_wave_barrier();
        double sns[NHG];
        row_scores(&s_kx[kWaves * HD], sns);
        single_state(kWaves, is_owner, sns);
    }
    TL(3);
    __builtin_amdgcn_sched_barrier(0);
    load_v(vA, wave);
    __builtin_amdgcn_sched_barrier(0);
    TL(4);

    // ---- the wave's initial softmax state: its single entry (max = the
    // score rounded to fp32, sum = 2^(score - max) with the difference in
    // fp64, output = sum * v row), or the empty state (-inf, 0, 0).  Heads
    // jq + 4hg are in every lane that holds them; the output goes into the
    // value layout by one MFMA k-step per output block whose only nonzero
    // weights are in lanes kq = 0: lane (m16, 0) takes head m16's sum.
    float m_run[NHG], l_run[NHG];
#pragma unroll
    for (int hg = 0; hg < NHG; ++hg) {
        const float mx = (float)sxs[hg];
        m_run[hg] = e_on ? mx : -INFINITY;
        l_run[hg] = e_on ? fast_exp2((float)(sxs[hg] - (double)mx)) : 0.f;
    }
    floatx4 o[NMB];
    {
        const float pw = (kq == 0 && m16 < NR) ? (m16 < 4 ? l_run[0] : l_run[NHG - 1]) : 0.f;
        float4 xv[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j) xv[j] = ld4(&s_vx[wave * HD + 64 * j + 4 * m16]);
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb)
            o[mb] = mfma16(comp(xv[mb / 4], mb % 4), pw, floatx4{0.f, 0.f, 0.f, 0.f});
    }
    float *wp = s_p + wave * (8 * 16 + 8);   // the wave's weights [head][k][s], then rescale factors [head]
    const int rD = 4 * bq + iq;              // this lane's row of the block in the score layout

    auto process = [&](const float4 *kf, const float4 (*vf)[NJ], int b) {
        const int rb = r0 + 16 * b;
        double acc[NHG];
#pragma unroll
        for (int hg = 0; hg < NHG; ++hg) acc[hg] = 0.0;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const double kv = (double)comp(kf[t], e);
#pragma unroll
                for (int hg = 0; hg < NHG; ++hg) acc[hg] = mfma4d(kv, (double)qb[hg][t][e], acc[hg]);
            }
        const int row = rb + rD;
        const bool ok = b < n_blk && row < r_end && row != new_slot;
#pragma unroll
        for (int hg = 0; hg < NHG; ++hg) {
            const double sc = acc[hg] * qscale;
            float mt = ok ? (float)sc : -INFINITY;
            mt = fmaxf(mt, dpp<0x124>(mt));           // the four row groups of a 16-lane row
            mt = fmaxf(mt, dpp<0x128>(mt));
            const float m_new = fmaxf(m_run[hg], max4rows(mt));
            const float m_use = m_new == -INFINITY ? 0.f : m_new;   // a block with every row masked
            const float alpha = fast_exp2(m_run[hg] - m_use);
            const float p = ok ? fast_exp2((float)(sc - (double)m_use)) : 0.f;
            float ps = p + dpp<0x124>(p);
            ps += dpp<0x128>(ps);
            l_run[hg] = fmaf(l_run[hg], alpha, sum4rows(ps));
            m_run[hg] = m_new;
            const int h = jq + 4 * hg;
            wp[h * 16 + iq * 4 + bq] = p;
            if (lane < 4) wp[8 * 16 + h] = alpha;
        }
        __builtin_amdgcn_wave_barrier();
        // to the value layout: lane (m16, kq) takes rows 4s + kq of head m16
        const bool hv = m16 < 4 * NHG;
        const float4 pv = hv ? ld4(&wp[min(m16, 4 * NHG - 1) * 16 + kq * 4]) : zero4();
        {
            const float al = hv ? wp[8 * 16 + min(m16, 4 * NHG - 1)] : 1.f;
#pragma unroll
            for (int mb = 0; mb < NMB; ++mb) o[mb] *= al;
        }
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
            for (int sk = 0; sk < 4; ++sk) o[mb] = mfma16(comp(vf[sk][mb / 4], mb % 4), comp(pv, sk), o[mb]);
        __builtin_amdgcn_wave_barrier();
    };
    // one block per wave at most: the block's loads are exact and it runs
    // unconditionally (a wave without one masks its rows)
    process(kA, vA, wave);

    TL(5);
    // ---- the wave's state to LDS: o[mb][v] is head m16 at dim
    // 64(mb / 4) + 16kq + 4v + mb % 4; the max and sum of head jq + 4hg
    // come from lane jq
    if (m16 < NR) {
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v)
                st4(&s_o[(wave * NR + m16) * OST + 64 * j + 16 * kq + 4 * v],
                    make_float4(o[4 * j][v], o[4 * j + 1][v], o[4 * j + 2][v], o[4 * j + 3][v]));
    }
#pragma unroll
    for (int hg = 0; hg < NHG; ++hg) {
        const int h = jq + 4 * hg;
        if (lane < 4 && h < NR) {
            s_m[wave * 8 + h] = m_run[hg];
            s_l[wave * 8 + h] = l_run[hg];
        }
    }
    TL(6);
    __syncthreads();
    TL(7);

    // ---- merge of the wave states (each holds its wave's single entry) and
    // of entry kWaves per (head, float4): thread (h, d4) for h < NR, d4 <
    // hd/4 (NR * hd/4 <= kThreads)
    static_assert(8 * (HD / 4) <= kThreads, "one merge thread per output float4");
    if (tid < NR * (HD / 4)) {
        const int h = tid / (HD / 4), d4 = tid - h * (HD / 4);
        float mw[kWaves], lw[kWaves];
        float4 xw[kWaves];
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            mw[w] = s_m[w * 8 + h];
            lw[w] = s_l[w * 8 + h];
            xw[w] = ld4(&s_o[(w * NR + h) * OST + 4 * d4]);
        }
        // entry kWaves (the new row behind kWaves extra rows; it holds the
        // bare v row, weighed here with its sum): read in every workgroup so
        // that all the LDS reads are issued together, used only where it was
        // written and counts (its max masked by bits: a select of the loaded
        // value would become a read under a branch)
        const bool on5 = n_extra == kWaves && is_owner;
        const unsigned keep5 = on5 ? 0xFFFFFFFFu : 0u;
        const float m5 = __builtin_bit_cast(float, (__builtin_bit_cast(unsigned, s_m[kWaves * 8 + h]) & keep5) |
                                                       (__builtin_bit_cast(unsigned, -INFINITY) & ~keep5));
        const float l5 = s_l[kWaves * 8 + h];
        const float4 x5 = ld4(&s_vx[kWaves * HD + 4 * d4]);
        const float m = fmaxf(fmaxf(fmaxf(mw[0], mw[1]), fmaxf(mw[2], mw[3])), m5);
        float l = 0.f;
        float4 acc = zero4();
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float e = mw[w] == -INFINITY ? 0.f : fast_exp2(mw[w] - m);
            l = fmaf(e, lw[w], l);
            acc.x = fmaf(e, xw[w].x, acc.x);
            acc.y = fmaf(e, xw[w].y, acc.y);
            acc.z = fmaf(e, xw[w].z, acc.z);
            acc.w = fmaf(e, xw[w].w, acc.w);
        }
        if (on5) {   // uniform in the workgroup; no memory operation inside
            const float e = fast_exp2(m5 - m) * l5;
            l += e;
            acc.x = fmaf(e, x5.x, acc.x);
            acc.y = fmaf(e, x5.y, acc.y);
            acc.z = fmaf(e, x5.z, acc.z);
            acc.w = fmaf(e, x5.w, acc.w);
        }
        const size_t hg = (size_t)g * n_rep + h;
        if (n_split == 1) {
            const float inv = 1.f / l;
            st4(out_p + hg * HD + 4 * d4, make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv));
        } else {
            st4(part_o + (hg * n_split + split) * HD + 4 * d4, acc);
            if (d4 == 0) {
                part_ml[(hg * n_split + split) * 2 + 0] = m;
                part_ml[(hg * n_split + split) * 2 + 1] = l;
            }
        }
    }
    TL(8);
    // ---- append of the new row (owner workgroup), last: no load waits
    // behind these stores
    if (is_owner && wave == NEW_WAVE && lane < HALF) {
        float *kd = kc_in + head_base + (size_t)new_slot * HD;
        float *vd = vc_in + head_base + (size_t)new_slot * HD;
        kd[lane] = nky0;
        kd[lane + HALF] = nky1;
        vd[lane] = nv0;
        vd[lane + HALF] = nv1;
    }
    TL(9);
    TL_WRITE(g_tl_split, kTlWaves, (blockIdx.y * gridDim.x + blockIdx.x) * kWaves + wave, kTlStamps);
}

// Splits of more than kWaves blocks plus kWaves extra rows (3B at 32K: 256
// rows, four blocks per wave): decode_split_kernel's layouts and arithmetic
// with each wave's blocks in a loop that keeps the next block in a second
// register set, the extra rows and the new row as nine softmax states merged
// after the loop (wave 3 scores the new row besides its own extra row).
// Kept apart from the single-block kernel: the single rows as wave initial
// states and one row per wave measured 0.4-0.8 us slower here (a loop that
// streams at the read rate, and a different register allocation).
template <int HD, int NR>
__global__ __launch_bounds__(kThreads) void decode_multi_kernel(const float *__restrict__ q_in, float *kc_in,
                                                                float *vc_in, const float *__restrict__ k_in,
                                                                const float *__restrict__ v_in, int n_rows,
                                                                int rows_per_split, int new_slot, int slots,
                                                                DecodeArgs a, RopeRow rr) {
    constexpr int NT = HD / 16;    // K float4 per lane per block (MFMA k-steps / 4)
    constexpr int NJ = HD / 64;    // V float4 per lane per row
    constexpr int NMB = HD / 16;   // 16-dim output blocks
    constexpr int HALF = HD / 2;
    constexpr int NST = 2 * kWaves + 1;   // wave states, extra-row states, new row
    constexpr int CH = HD / 4;            // dims per lane of a K row (one k chunk)
    constexpr int NHG = NR > 4 ? 2 : 1;   // groups of 4 heads (score chains)
    constexpr int NEW_WAVE = kWaves - 1;  // the wave that takes the new row
    static_assert(NR >= 1 && NR <= 8, "at most 8 q-heads per workgroup");
    static_assert(HD == 64 || HD == 128, "head_dim 64 or 128");
    TL_DECL(kTlStamps);
    TL(0);

    constexpr int OST = HD + 4;    // LDS stride of a head's output (bank spread)
    __shared__ __align__(16) float s_o[kWaves * NR * OST];  // unnormalised wave outputs
    __shared__ __align__(16) float s_knew[HD];              // the new row: roped k
    __shared__ __align__(16) float s_vnew[HD];              // ... and v
    __shared__ __align__(16) float s_kx[kWaves * HD];       // the extra rows: k
    __shared__ __align__(16) float s_vx[kWaves * HD];       // ... and v
    __shared__ float s_m[NST * 8], s_l[NST * 8];
    __shared__ __align__(16) float s_p[kWaves * (8 * 16 + 8)];   // per wave: weights, rescale factors

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m16 = lane & 15, kq = lane >> 4;
    const int jq = lane & 3, bq = (lane >> 2) & 3, iq = lane >> 4;   // score layout: head, row group, row
    const int split = blockIdx.x, g = blockIdx.y;
    const int r0 = split * rows_per_split;
    const int r_end = min(r0 + rows_per_split, n_rows);
    const int n_own = max(r_end - r0, 0);
    // whole blocks, plus a last partial block of more than kWaves rows; a
    // remainder of at most kWaves rows is taken as extra rows, one per wave
    const int rem = n_own % kDecodeBlock;
    const int n_blk = n_own / kDecodeBlock + (rem > kWaves ? 1 : 0);
    const int n_extra = rem > kWaves ? 0 : rem;
    const int last_row = max(r_end - 1, 0);
    const int owner = n_rows == 0 ? 0 : min(new_slot, n_rows - 1) / rows_per_split;
    const bool is_owner = split == owner;
    const size_t head_base = (size_t)g * slots * HD;
    const float *kg = kc_in + head_base;
    const float *vg = vc_in + head_base;

    // ---- q of the NR heads of kv-head g, roped and pre-scaled by every wave
    // for itself and staged through the wave's own LDS rows, so no
    // workgroup barrier stands between a wave's loads and its first MFMA.
    // Pair p < NR * hd/8 of the wave is (q[h][4c..4c+3], q[h][hd/2 + 4c..])
    // with h = p / NC, c = p % NC; lane l takes pairs l and l + 64, which
    // share c = l % NC and so the four (cos, sin) pairs of dims 4c..4c+3.
    // The MFMA operand layout repeats every q value in 16/NR lanes and every
    // (cos, sin) pair in 16, so loading the operands directly would cost each
    // wave as much vector-memory traffic as its cache rows.
    constexpr int QS = HD + 4;                 // s_q row stride (bank spread)
    constexpr int NC = HALF / 4;               // float4 per half row
    constexpr int NP = (NR * NC + 63) / 64;    // pairs per lane
    static_assert(64 % NC == 0 && NP <= 2, "a lane's pairs share their (cos, sin) values");
    // per wave NR rows of roped q * 1/sqrt(hd) * log2(e), and one row that
    // takes the stores of lanes without a pair (so the stores need no branch)
    __shared__ __align__(16) float s_q[kWaves * (NR + 1) * QS];
    float *wq = s_q + wave * (NR + 1) * QS;
    const int sc = lane % NC;
    float4 sx0[NP], sx1[NP];
    const float4 scs01 = ld4(&rr.cs[8 * sc]), scs23 = ld4(&rr.cs[8 * sc + 4]);
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        const int sh = min((lane + 64 * i) / NC, NR - 1);
        const float *qh = q_in + (size_t)(g * NR + sh) * HD + 4 * sc;
        sx0[i] = ld4(qh);
        sx1[i] = ld4(qh + HALF);
    }
    TL(10);
    // the new k/v row and this wave's extra row, pair (i, i + hd/2) in lane
    // i: loaded by every lane of every wave (clamped rows), so that no load
    // is conditional, and ahead of the K rows, so that their scores are taken
    // while the cache rows stream in
    const int ni = min(lane, HALF - 1);
    const float nk0 = k_in[(size_t)g * HD + ni], nk1 = k_in[(size_t)g * HD + ni + HALF];
    const float nv0 = v_in[(size_t)g * HD + ni], nv1 = v_in[(size_t)g * HD + ni + HALF];
    const float2 ncs = *reinterpret_cast<const float2 *>(&rr.cs[2 * ni]);
    const int xrow = min(r0 + (n_own - n_extra) + wave, last_row);
    const float xk0 = kg[(size_t)xrow * HD + ni], xk1 = kg[(size_t)xrow * HD + ni + HALF];
    const float xv0 = vg[(size_t)xrow * HD + ni], xv1 = vg[(size_t)xrow * HD + ni + HALF];
    // the arguments the merge needs (read from the kernel-argument segment,
    // not preloaded)
    float *const out_p = a.out, *const part_o = a.part_o, *const part_ml = a.part_ml;
    const int n_split = a.n_split, n_rep = a.n_rep;

    float4 kA[NT], vA[4][NJ];
    float4 kB[NT], vB[4][NJ];
    auto load_k = [&](float4 *kf, int b) {
        const float *kr = kg + (size_t)min(r0 + 16 * b + m16, last_row) * HD + CH * kq;
#pragma unroll
        for (int t = 0; t < NT; ++t) kf[t] = ld4(kr + 4 * t);
    };
    auto load_v = [&](float4 (*vf)[NJ], int b) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const float *vr = vg + (size_t)min(r0 + 16 * b + 4 * s + kq, last_row) * HD + 4 * m16;
#pragma unroll
            for (int j = 0; j < NJ; ++j) vf[s][j] = ld4(vr + 64 * j);
        }
    };
    __builtin_amdgcn_sched_barrier(0);
    load_k(kA, wave);
    __builtin_amdgcn_sched_barrier(0);
    TL(1);
    // the merge arguments are waited for here, behind the K rows' requests: a
    // first read after the block loop would wait for a kernel-argument fetch
    // at the end of the kernel
    asm volatile("" ::"s"(out_p), "s"(part_o), "s"(part_ml), "s"(n_split), "s"(n_rep));

    // RoPE of the staged pairs into the wave's LDS rows, then the B operand:
    // lane l holds heads jq and jq + 4 (jq = l % 4) at dims CH kq + 4t + e
    // (heads past NR are zero); the dot products are widened to double and
    // scaled by kore's 1/sqrt(hd) and log2(e) there.
    const double qscale = (double)a.scale * 1.4426950408889634;
    float qb[NHG][NT][4];
    {
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int p = lane + 64 * i;
            const int row = p < NR * NC ? p / NC : NR;
            float y0[4], y1[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float4 c4 = e < 2 ? scs01 : scs23;
                const float2 cs = (e & 1) ? make_float2(c4.z, c4.w) : make_float2(c4.x, c4.y);
                rope_pair(comp(sx0[i], e), comp(sx1[i], e), cs, y0[e], y1[e]);
            }
            st4(&wq[row * QS + 4 * sc], make_float4(y0[0], y0[1], y0[2], y0[3]));
            st4(&wq[row * QS + HALF + 4 * sc], make_float4(y1[0], y1[1], y1[2], y1[3]));
        }
        __builtin_amdgcn_wave_barrier();
        // heads past NR read head NR - 1 and are zeroed by a bit mask: a
        // select of the loaded value became a read under a lane mask, each
        // waited for before the next
#pragma unroll
        for (int hg = 0; hg < NHG; ++hg) {
            const int h = jq + 4 * hg;
            const unsigned keep = h < NR ? 0xFFFFFFFFu : 0u;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const float4 qv = ld4(&wq[min(h, NR - 1) * QS + CH * kq + 4 * t]);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    qb[hg][t][e] = __builtin_bit_cast(float, __builtin_bit_cast(unsigned, comp(qv, e)) & keep);
            }
        }
    }
    TL(2);

    // dot of q (operand layout) with a k row staged in LDS, for heads jq + 4hg:
    // lane l sums its dims CH kq + 4t + e, then the four lanes of its chunk
    // row (l, l ^ 16, l ^ 32, l ^ 48) add up; every lane ends with the scores
    // (four independent partial sums per head group: a single chain of
    // dependent fp64 FMAs would take most of a microsecond)
    auto row_scores = [&](const float *kr, double (&out)[NHG]) {
        double sx[NHG][4];
#pragma unroll
        for (int hg = 0; hg < NHG; ++hg)
#pragma unroll
            for (int e = 0; e < 4; ++e) sx[hg][e] = 0.0;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float4 kx = ld4(&kr[CH * kq + 4 * t]);
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int hg = 0; hg < NHG; ++hg) sx[hg][e] = fma((double)qb[hg][t][e], (double)comp(kx, e), sx[hg][e]);
        }
#pragma unroll
        for (int hg = 0; hg < NHG; ++hg)
            out[hg] = sum4rows_d((sx[hg][0] + sx[hg][1]) + (sx[hg][2] + sx[hg][3])) * qscale;
    };
    // A single row as a softmax state: max = its score rounded to fp32, sum
    // = 2^(score - max) with the difference in fp64 (about 1), output = that
    // sum times the row (the merge applies the sum to the stored v row).
    // ---- the wave's extra row (state kWaves + wave; -inf and a zero row
    // when the wave has none) and, in NEW_WAVE, the new row (state 2 kWaves,
    // roped here; -inf and a zero row outside the owner workgroup).  Only
    // LDS and register work: no memory operation under these branches.  The
    // merge weighs each stored v row with the state's sum.
    {
        const bool x_on = wave < n_extra;
        if (lane < HALF) {
            s_kx[wave * HD + lane] = xk0;
            s_kx[wave * HD + lane + HALF] = xk1;
            s_vx[wave * HD + lane] = x_on ? xv0 : 0.f;
            s_vx[wave * HD + lane + HALF] = x_on ? xv1 : 0.f;
        }
        __builtin_amdgcn_wave_barrier();
        const bool on = x_on && xrow != new_slot;
        double sxs[NHG];
        row_scores(&s_kx[wave * HD], sxs);
#pragma unroll
        for (int hg = 0; hg < NHG; ++hg) {
            const double sx = sxs[hg];
            const int h = jq + 4 * hg;
            if (lane < 4 && h < NR) {
                const float mx = (float)sx;
                s_m[(kWaves + wave) * 8 + h] = on ? mx : -INFINITY;
                s_l[(kWaves + wave) * 8 + h] = on ? fast_exp2((float)(sx - (double)mx)) : 0.f;
            }
        }
    }
    float nky0, nky1;
    rope_pair(nk0, nk1, ncs, nky0, nky1);
    if (wave == NEW_WAVE) {
        if (lane < HALF) {
            s_knew[lane] = nky0;
            s_knew[lane + HALF] = nky1;
            s_vnew[lane] = is_owner ? nv0 : 0.f;
            s_vnew[lane + HALF] = is_owner ? nv1 : 0.f;
        }
        __builtin_amdgcn_wave_barrier();
        double sns[NHG];
        row_scores(s_knew, sns);
#pragma unroll
        for (int hg = 0; hg < NHG; ++hg) {
            const double sn = sns[hg];
            const int h = jq + 4 * hg;
            if (lane < 4 && h < NR) {
                const float mn = (float)sn;
                s_m[2 * kWaves * 8 + h] = is_owner ? mn : -INFINITY;
                s_l[2 * kWaves * 8 + h] = is_owner ? fast_exp2((float)(sn - (double)mn)) : 0.f;
            }
        }
    }
    TL(3);
    __builtin_amdgcn_sched_barrier(0);
    load_v(vA, wave);
    if (wave + kWaves < n_blk) {
        load_k(kB, wave + kWaves);
        load_v(vB, wave + kWaves);
    }
    __builtin_amdgcn_sched_barrier(0);
    TL(4);

    floatx4 o[NMB];
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) o[mb] = floatx4{0.f, 0.f, 0.f, 0.f};
    // softmax state of heads jq + 4hg (the same in every lane that holds them)
    float m_run[NHG], l_run[NHG];
#pragma unroll
    for (int hg = 0; hg < NHG; ++hg) {
        m_run[hg] = -INFINITY;
        l_run[hg] = 0.f;
    }
    float *wp = s_p + wave * (8 * 16 + 8);   // the wave's weights [head][k][s], then rescale factors [head]
    const int rD = 4 * bq + iq;              // this lane's row of the block in the score layout

    auto process = [&](const float4 *kf, const float4 (*vf)[NJ], int b, bool first) {
        const int rb = r0 + 16 * b;
        double acc[NHG];
#pragma unroll
        for (int hg = 0; hg < NHG; ++hg) acc[hg] = 0.0;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const double kv = (double)comp(kf[t], e);
#pragma unroll
                for (int hg = 0; hg < NHG; ++hg) acc[hg] = mfma4d(kv, (double)qb[hg][t][e], acc[hg]);
            }
        const int row = rb + rD;
        const bool ok = row < r_end && row != new_slot;
#pragma unroll
        for (int hg = 0; hg < NHG; ++hg) {
            const double sc = acc[hg] * qscale;
            float mt = ok ? (float)sc : -INFINITY;
            mt = fmaxf(mt, dpp<0x124>(mt));           // the four row groups of a 16-lane row
            mt = fmaxf(mt, dpp<0x128>(mt));
            const float m_new = fmaxf(m_run[hg], max4rows(mt));
            const float m_use = m_new == -INFINITY ? 0.f : m_new;   // a block with every row masked
            const float alpha = fast_exp2(m_run[hg] - m_use);
            const float p = ok ? fast_exp2((float)(sc - (double)m_use)) : 0.f;
            float ps = p + dpp<0x124>(p);
            ps += dpp<0x128>(ps);
            l_run[hg] = fmaf(l_run[hg], alpha, sum4rows(ps));
            m_run[hg] = m_new;
            const int h = jq + 4 * hg;
            wp[h * 16 + iq * 4 + bq] = p;
            if (lane < 4) wp[8 * 16 + h] = alpha;
        }
        __builtin_amdgcn_wave_barrier();
        // to the value layout: lane (m16, kq) takes rows 4s + kq of head m16
        const bool hv = m16 < 4 * NHG;
        const float4 pv = hv ? ld4(&wp[min(m16, 4 * NHG - 1) * 16 + kq * 4]) : zero4();
        if (!first) {
            const float al = hv ? wp[8 * 16 + min(m16, 4 * NHG - 1)] : 1.f;
#pragma unroll
            for (int mb = 0; mb < NMB; ++mb) o[mb] *= al;
        }
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
            for (int sk = 0; sk < 4; ++sk) o[mb] = mfma16(comp(vf[sk][mb / 4], mb % 4), comp(pv, sk), o[mb]);
        __builtin_amdgcn_wave_barrier();
    };
    for (int b = wave; b < n_blk;) {
        process(kA, vA, b, b == wave);
        b += kWaves;
        if (b >= n_blk) break;
        if (b + kWaves < n_blk) {
            load_k(kA, b + kWaves);
            load_v(vA, b + kWaves);
        }
        process(kB, vB, b, false);
        b += kWaves;
        if (b + kWaves < n_blk) {
            load_k(kB, b + kWaves);
            load_v(vB, b + kWaves);
        }
    }
    TL(5);
    // ---- the wave's state to LDS: o[mb][v] is head m16 at dim
    // 64(mb / 4) + 16kq + 4v + mb % 4; the max and sum of head jq + 4hg
    // come from lane jq
    if (m16 < NR) {
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v)
                st4(&s_o[(wave * NR + m16) * OST + 64 * j + 16 * kq + 4 * v],
                    make_float4(o[4 * j][v], o[4 * j + 1][v], o[4 * j + 2][v], o[4 * j + 3][v]));
    }
#pragma unroll
    for (int hg = 0; hg < NHG; ++hg) {
        const int h = jq + 4 * hg;
        if (lane < 4 && h < NR) {
            s_m[wave * 8 + h] = m_run[hg];
            s_l[wave * 8 + h] = l_run[hg];
        }
    }
    TL(6);
    __syncthreads();
    TL(7);

    // ---- merge of the wave states (and the new row's) per (head, float4):
    // thread (h, d4) for h < NR, d4 < hd/4 (NR * hd/4 <= kThreads)
    static_assert(8 * (HD / 4) <= kThreads, "one merge thread per output float4");
    if (tid < NR * (HD / 4)) {
        const int h = tid / (HD / 4), d4 = tid - h * (HD / 4);
        float mw[kWaves], lw[kWaves];
        float4 xw[kWaves];
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            mw[w] = s_m[w * 8 + h];
            lw[w] = s_l[w * 8 + h];
            xw[w] = ld4(&s_o[(w * NR + h) * OST + 4 * d4]);
        }
        float m = fmaxf(fmaxf(mw[0], mw[1]), fmaxf(mw[2], mw[3]));
        float l = 0.f;
        float4 acc = zero4();
        // the extra rows' and the new row's states, every one read (each is
        // written in every workgroup: the absent ones hold max -inf, sum 0 and
        // a zero row) and the absent ones masked, so that all the LDS reads
        // are issued together (reads under the per-state branches were each
        // waited for before the next)
        float ms[kWaves + 1], ls[kWaves + 1];
        float4 xs[kWaves + 1];
#pragma unroll
        for (int w = 0; w <= kWaves; ++w) {
            const int st = kWaves + w;
            ms[w] = s_m[st * 8 + h];
            ls[w] = s_l[st * 8 + h];
            xs[w] = ld4(w < kWaves ? &s_vx[w * HD + 4 * d4] : &s_vnew[4 * d4]);
        }
#pragma unroll
        for (int w = 0; w <= kWaves; ++w) {
            const bool on = w < kWaves ? w < n_extra : is_owner;
            ms[w] = on ? ms[w] : -INFINITY;
            ls[w] = on ? ls[w] : 0.f;
            xs[w] = on ? xs[w] : zero4();
            m = fmaxf(m, ms[w]);
        }
#pragma unroll
        for (int w = 0; w < 2 * kWaves + 1; ++w) {
            const bool on = w < kWaves ? true : (w < 2 * kWaves ? w - kWaves < n_extra : is_owner);
            if (!on) continue;
            const float mx = w < kWaves ? mw[w] : ms[w - kWaves];
            const float e0 = mx == -INFINITY ? 0.f : fast_exp2(mx - m);
            const float4 x = w < kWaves ? xw[w] : xs[w - kWaves];
            // a wave state holds its weighted output; a single row's state
            // holds the bare v row, weighed here with the state's sum
            const float e = w < kWaves ? e0 : e0 * ls[w - kWaves];
            l = w < kWaves ? fmaf(e, lw[w], l) : l + e;
            acc.x = fmaf(e, x.x, acc.x);
            acc.y = fmaf(e, x.y, acc.y);
            acc.z = fmaf(e, x.z, acc.z);
            acc.w = fmaf(e, x.w, acc.w);
        }
        const size_t hg = (size_t)g * n_rep + h;
        if (n_split == 1) {
            const float inv = 1.f / l;
            st4(out_p + hg * HD + 4 * d4, make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv));
        } else {
            st4(part_o + (hg * n_split + split) * HD + 4 * d4, acc);
            if (d4 == 0) {
                part_ml[(hg * n_split + split) * 2 + 0] = m;
                part_ml[(hg * n_split + split) * 2 + 1] = l;
            }
        }
    }
    TL(8);
    // ---- append of the new row (owner workgroup), last: no load waits
    // behind these stores
    if (is_owner && wave == NEW_WAVE && lane < HALF) {
        float *kd = kc_in + head_base + (size_t)new_slot * HD;
        float *vd = vc_in + head_base + (size_t)new_slot * HD;
        kd[lane] = nky0;
        kd[lane + HALF] = nky1;
        vd[lane] = nv0;
        vd[lane + HALF] = nv1;
    }
    TL(9);
    TL_WRITE(g_tl_split, kTlWaves, (blockIdx.y * gridDim.x + blockIdx.x) * kWaves + wave, kTlStamps);
}

// Block (q-head h, 32-dim chunk): out[h][chunk] = sum_s w_s o_s / sum_s w_s l_s
// with w_s = 2^(m_s - max_s m_s) (split maxima are in the log2 domain), the
// log-sum-exp merge of the splits.  Lane (sub, c) takes splits sub + 8 i
// (i < PER, so n_split <= 8 PER) and float4 c of the chunk, so a split's
// chunk is one whole 128-byte line; every load is issued before the first
// use (one memory round trip).
template <int HD, int PER>
__global__ __launch_bounds__(64) void decode_combine_kernel(const float *part_o, const float *part_ml, float *out,
                                                            int n_split) {
    TL_DECL(kTlCombStamps);
    TL(0);
    const int h = blockIdx.x, chunk = blockIdx.y, lane = threadIdx.x;
    const int S = n_split;
    const int sub = lane >> 3, c = lane & 7;
    const float2 *ml = reinterpret_cast<const float2 *>(part_ml) + (size_t)h * S;
    const float *po = part_o + (size_t)h * S * HD + chunk * 32 + c * 4;
    float4 x[PER];
    float2 st[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int s = min(sub + 8 * i, S - 1);
        x[i] = ld4(po + (size_t)s * HD);
        st[i] = ml[s];
    }
    __builtin_amdgcn_sched_barrier(0);   // keep every load ahead of the arithmetic
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER; ++i) m = fmaxf(m, st[i].x);
    m = max4rows(row16_max(m));
    TL(1);
    float4 acc = zero4();
    float den = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const float w = (sub + 8 * i < S && st[i].x != -INFINITY) ? fast_exp2(st[i].x - m) : 0.f;
        den = fmaf(w, st[i].y, den);
        acc.x = fmaf(w, x[i].x, acc.x);
        acc.y = fmaf(w, x[i].y, acc.y);
        acc.z = fmaf(w, x[i].z, acc.z);
        acc.w = fmaf(w, x[i].w, acc.w);
    }
    // sum over sub (lane bits 3..5): the two subs of a row by DPP (rotation
    // by 8 keeps c), the four rows by permlane swaps
    acc.x += dpp<0x128>(acc.x); acc.y += dpp<0x128>(acc.y); acc.z += dpp<0x128>(acc.z); acc.w += dpp<0x128>(acc.w);
    den += dpp<0x128>(den);
    acc.x = sum4rows(acc.x);
    acc.y = sum4rows(acc.y);
    acc.z = sum4rows(acc.z);
    acc.w = sum4rows(acc.w);
    den = sum4rows(den);
    if (sub == 0) {
        const float inv = 1.f / den;
        st4(out + (size_t)h * HD + chunk * 32 + c * 4,
            make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv));
    }
    TL(2);
    TL_WRITE(g_tl_comb, kTlComb, blockIdx.y * gridDim.x + blockIdx.x, kTlCombStamps);
}

// ------------------------------------------------------------------ append

// Block (token z, kv-head g): k row rotated at position pos0+z and stored,
// v row copied (kore.cpp:1536-1538).  Slot = position (a prefill never wraps).
__global__ void append_kernel(AppendArgs a, int hd) {
    const int z = blockIdx.x * blockDim.y + threadIdx.y, g = blockIdx.y, half = hd / 2;
    if (z >= a.n_tok) return;
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

// ------------------------------------------------------------ any geometry

// Block i < n_head: RoPE of q row i at the decode position into q_out; block
// n_head + g: RoPE of the new k row of kv-head g and the append of k and v at
// new_slot (kore.cpp:1424-1430).
__global__ void generic_decode_prep_kernel(const float *q, const float *k, const float *v, float *q_out,
                                           float *kc, float *vc, int n_head, int hd, int slots, int new_slot,
                                           RopeRow rr) {
    const int i = blockIdx.x, half = hd / 2;
    const bool is_q = i < n_head;
    const int g = i - n_head;
    const float *src = is_q ? q + (size_t)i * hd : k + (size_t)g * hd;
    float *dst = is_q ? q_out + (size_t)i * hd : kc + ((size_t)g * slots + new_slot) * hd;
    for (int d = threadIdx.x; d < half; d += blockDim.x) {
        float y0, y1;
        rope_pair(src[d], src[d + half], make_float2(rr.cs[2 * d], rr.cs[2 * d + 1]), y0, y1);
        dst[d] = y0;
        dst[d + half] = y1;
    }
    if (!is_q) {
        float *vd = vc + ((size_t)g * slots + new_slot) * hd;
        for (int d = threadIdx.x; d < hd; d += blockDim.x) vd[d] = v[(size_t)g * hd + d];
    }
}

__device__ __forceinline__ double wave_max_d(double x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x = fmax(x, __shfl_xor(x, o, 64));
    return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
    return x;
}

// Workgroup (key range, kv-head g x head chunk c): q-heads g * n_rep + c *
// chunk + i (i < nh) attend keys [r_begin, r_end) of kv-head g in LDS tiles
// of `tile` rows (rows past r_end read as zeros, never from memory).  Per
// tile: scores as fp64 dots of the fp32 roped q and k (each product exact in
// fp64), times kore's 1/sqrt(hd) and log2(e); one wave per head takes the
// tile's max and the weights 2^(score - max) with the difference in fp64;
// then every thread advances its outputs (head, dim) by the weighted V rows
// in fp32.  Prefill workgroups take row z = blockIdx.x with keys 0..pos0+z
// and rope their q rows from the table; decode workgroups take split
// blockIdx.x of the rows [0, n_rows) with q already roped.
__global__ __launch_bounds__(kThreads) void generic_attend_kernel(GenericArgs a) {
    extern __shared__ __align__(16) unsigned char g_lds[];
    const int hd = a.hd, T = a.tile, CH = a.chunk, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int g = blockIdx.y / a.n_chunks, c = blockIdx.y % a.n_chunks;
    const int h0 = c * CH, nh = min(CH, a.n_rep - h0);
    const int n_head = a.n_head_kv * a.n_rep, hq0 = g * a.n_rep + h0;
    const bool prefill = a.cs != nullptr;
    const int z = prefill ? (int)blockIdx.x : 0;
    const int r_begin = prefill ? 0 : (int)blockIdx.x * a.rows_per_split;
    const int r_end = prefill ? a.pos0 + z + 1 : min(r_begin + a.rows_per_split, a.n_rows);

    double *s_sc = reinterpret_cast<double *>(g_lds);   // [CH][T] scores
    float *s_p = reinterpret_cast<float *>(s_sc + CH * T);   // [CH][T] weights
    float *s_al = s_p + CH * T;                              // [CH] rescale of the tile
    float *s_m = s_al + CH, *s_l = s_m + CH;                 // [CH] running max, sum
    float *s_q = s_l + CH;                                   // [CH][hd]
    float *s_k = s_q + CH * hd;                              // [T][hd + 1]
    float *s_v = s_k + T * (hd + 1);                         // [T][hd]

    const float *qb = a.q + ((size_t)z * n_head + hq0) * hd;
    for (int e = tid; e < nh * hd; e += kThreads) {
        if (prefill) {
            const int i = e / hd, d = e % hd, half = hd / 2, d0 = d < half ? d : d - half;
            const float *qr = qb + (size_t)i * hd;
            float y0, y1;
            rope_pair(qr[d0], qr[d0 + half], a.cs[(size_t)(a.pos0 + z) * half + d0], y0, y1);
            s_q[e] = d < half ? y0 : y1;
        } else {
            s_q[e] = qb[e];
        }
    }
    if (tid < nh) {
        s_m[tid] = -INFINITY;
        s_l[tid] = 0.f;
    }
    const double sscale = (double)a.scale * 1.4426950408889634;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    const float *kg = a.kc + (size_t)g * a.slots * hd;
    const float *vg = a.vc + (size_t)g * a.slots * hd;
    for (int t0 = r_begin; t0 < r_end; t0 += T) {
        const int nr = min(T, r_end - t0);
        __syncthreads();   // the previous tile's readers are done (and s_q, s_m, s_l are set)
        const float *kt = kg + (size_t)t0 * hd, *vt = vg + (size_t)t0 * hd;
        for (int e = tid; e < T * hd; e += kThreads) {
            const int r = e / hd, d = e % hd;
            const bool ok = r < nr;
            s_k[r * (hd + 1) + d] = ok ? kt[e] : 0.f;
            s_v[e] = ok ? vt[e] : 0.f;
        }
        __syncthreads();
        for (int e = tid; e < nh * T; e += kThreads) {
            const int i = e / T, r = e % T;
            double s = -INFINITY;
            if (r < nr) {
                const float *qi = s_q + i * hd, *kr = s_k + r * (hd + 1);
                double d0 = 0.0, d1 = 0.0;
                for (int d = 0; d < hd; d += 2) {
                    d0 = fma((double)qi[d], (double)kr[d], d0);
                    d1 = fma((double)qi[d + 1], (double)kr[d + 1], d1);
                }
                s = (d0 + d1) * sscale;
            }
            s_sc[e] = s;
        }
        __syncthreads();
        for (int i = wave; i < nh; i += kWaves) {
            const double sv = lane < T ? s_sc[i * T + lane] : -INFINITY;
            const float m_old = s_m[i];
            const float m_new = fmaxf(m_old, (float)wave_max_d(sv));
            const float p = sv != -INFINITY ? fast_exp2((float)(sv - (double)m_new)) : 0.f;
            const float sum = wave_sum(p);
            if (lane < T) s_p[i * T + lane] = p;
            if (lane == 0) {
                const float al = m_old == -INFINITY ? 0.f : fast_exp2(m_old - m_new);
                s_al[i] = al;
                s_m[i] = m_new;
                s_l[i] = s_l[i] * al + sum;
            }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int o = tid + j * kThreads;
            if (o < nh * hd) {
                const int i = o / hd, d = o % hd;
                const float *pi = s_p + i * T;
                float x = acc[j] * s_al[i];
                for (int r = 0; r < nr; ++r) x = fmaf(pi[r], s_v[r * hd + d], x);
                acc[j] = x;
            }
        }
    }
    __syncthreads();
    if (prefill || a.n_split == 1) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int o = tid + j * kThreads;
            if (o < nh * hd) a.out[((size_t)z * n_head + hq0) * hd + o] = acc[j] / s_l[o / hd];
        }
    } else {
        const int sp = blockIdx.x;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int o = tid + j * kThreads;
            if (o < nh * hd) {
                const int i = o / hd, d = o % hd;
                a.part_o[((size_t)(hq0 + i) * a.n_split + sp) * hd + d] = acc[j];
            }
        }
        if (tid < nh)
            reinterpret_cast<float2 *>(a.part_ml)[(size_t)(hq0 + tid) * a.n_split + sp] =
                make_float2(s_m[tid], s_l[tid]);
    }
}

// Block h: log-sum-exp merge of q-head h's split partials (max and sum in
// the base-2 domain of generic_attend_kernel), one thread per dim.
__global__ void generic_combine_kernel(const float *part_o, const float *part_ml, float *out, int n_split, int hd) {
    const int h = blockIdx.x;
    const float2 *ml = reinterpret_cast<const float2 *>(part_ml) + (size_t)h * n_split;
    float m = -INFINITY;
    for (int s = 0; s < n_split; ++s) m = fmaxf(m, ml[s].x);
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float acc = 0.f, den = 0.f;
        for (int s = 0; s < n_split; ++s) {
            const float2 st = ml[s];
            const float w = fast_exp2(st.x - m);
            den = fmaf(w, st.y, den);
            acc = fmaf(w, part_o[((size_t)h * n_split + s) * hd + d], acc);
        }
        out[(size_t)h * hd + d] = acc / den;
    }
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
// The tiles go from HBM straight into LDS (global_load_lds_dwordx4: lane i of
// a load writes 16 bytes at the wave's base + 16 i), double-buffered, so tile
// t + 1 streams in while tile t is computed, with one barrier per tile and no
// staging registers.  V is kept row-major: output block tt of a wave holds
// dims NT i + tt (i < 32), so one 16-byte (hd 64: 8-byte) read of a V row
// feeds all NT blocks; K's float4 columns are XOR-swizzled by (row mod 16)
// so the 16-byte reads of 16 rows at one column fall in different banks.
// With key segments (a short chunk over a long cache has too few workgroups
// to fill the GPU) a workgroup covers one range of key tiles and writes its
// rows' unnormalised output with their max and sum instead.  The strips'
// causal work runs from 1 to n_tok / 32 tiles; two workgroups share a CU, and
// the grid is folded (PrefillArgs::fold) to pair long strips with short ones.
template <int HD>
__global__ __launch_bounds__(kThreads, 2) void prefill_kernel(PrefillArgs a) {
    constexpr int BK = 32;
    constexpr int NT = HD / 32;
    constexpr int HALF = HD / 2;
    constexpr int C4 = HD / 4;                 // float4 per cache row
    constexpr int NI = BK * C4 / 64 / kWaves;  // LDS loads per wave per tensor and tile
    static_assert(NI * 64 * kWaves == BK * C4, "whole 1 KB loads per tile");
    // one array per buffer: the compiler tracks LDS-direct loads per LDS
    // object, so reads of one buffer do not wait for loads into the other
    __shared__ __align__(16) float sK0[BK * HD], sK1[BK * HD];
    __shared__ __align__(16) float sV0[BK * HD], sV1[BK * HD];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nkv = a.n_head_kv;
    // work index: items run from the longest strips down; the second part
    // of the grid takes them from the short end, so that the two
    // workgroups of a CU (b and b + fold) add up to about the same work
    const int bx = blockIdx.x;
    const int wi = bx < a.fold ? bx : (int)gridDim.x - 1 - (bx - a.fold);
    const int g = wi % nkv;
    // split plan: unit = item << 2 | part (0 whole, 1 / 2 first / second half)
    const int unit = a.n_split > 0 ? (int)a.unit[wi / nkv] : 0;
    const int part = unit & 3;
    const int seg = a.n_split > 0 ? 0 : (wi / nkv) % a.n_kseg;
    const int item = a.n_split > 0 ? unit >> 2 : wi / nkv / a.n_kseg;
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

    // Q^T operand: qreg[4j+e] = roped q[qrow][8j + 4qg + e] * 1/sqrt(hd) * log2(e),
    // filled after the first key tile is requested (its loads then overlap q's)
    float qreg[HD / 2];
    auto load_q = [&] {
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
                qreg[4 * j + e2] = y0 * a.scale_log2;
                qreg[4 * (j + HD / 16) + e2] = y1 * a.scale_log2;
            }
        }
    };

    floatx16 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;

    // Tile t into (dK, dV): load i of wave w covers float4 slots
    // p = 64 (NI w + i) + lane, i.e. row p / C4 and position p % C4; V holds
    // column (p % C4) there, K column (p % C4) ^ (row & 15).  Keys past the
    // cache end are clamped to its last row (the causal mask excludes them:
    // every query position is below n_keys).
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    auto issue_tile = [&](float *dK, float *dV, int t) {
        if (t * BK + BK <= n_keys) {
            const size_t tb = ((size_t)g * a.slots + t * BK) * HD;
            const float *kb = a.kc + tb, *vb = a.vc + tb;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                // per-lane offsets inside a tile, the same for every tile
                const int chunk = NI * wave_u + i;
                const int p = 64 * chunk + lane;
                const int row = p / C4, pos = p % C4;
                const int koff = row * HD + 4 * (pos ^ (row & 15)), voff = row * HD + 4 * pos;
                __builtin_amdgcn_global_load_lds(kb + koff, (void __attribute__((address_space(3))) *)(dK + 256 * chunk), 16, 0, 0);
                __builtin_amdgcn_global_load_lds(vb + voff, (void __attribute__((address_space(3))) *)(dV + 256 * chunk), 16, 0, 0);
            }
        } else {
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int chunk = NI * wave_u + i;
                const int p = 64 * chunk + lane;
                const int row = p / C4, pos = p % C4;
                const size_t base = ((size_t)g * a.slots + min(t * BK + row, n_keys - 1)) * HD;
                __builtin_amdgcn_global_load_lds(a.kc + base + 4 * (pos ^ (row & 15)),
                                                 (void __attribute__((address_space(3))) *)(dK + 256 * chunk), 16, 0, 0);
                __builtin_amdgcn_global_load_lds(a.vc + base + 4 * pos,
                                                 (void __attribute__((address_space(3))) *)(dV + 256 * chunk), 16, 0, 0);
            }
        }
    };
    auto compute_tile = [&](const float *sK, const float *sV, int t) {
        const int k0 = t * BK;
        if (k0 > my_kmax) return;
        floatx16 s;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
        for (int j = 0; j < HD / 8; ++j) {
            const float4 a4 = ld4(&sK[qi * HD + 4 * ((2 * j + qg) ^ (qi & 15))]);
            s = mfma32(a4.x, qreg[4 * j + 0], s);
            s = mfma32(a4.y, qreg[4 * j + 1], s);
            s = mfma32(a4.z, qreg[4 * j + 2], s);
            s = mfma32(a4.w, qreg[4 * j + 3], s);
        }
        // s[r] = score(query qi, key k0 + 8(r/4) + 4qg + r%4), already in the
        // log2 domain; the causal mask only matters on tiles that reach past
        // the strip's first query position
        if (k0 + BK - 1 > a.pos0 + 32 * strip) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = k0 + 8 * (r / 4) + 4 * qg + (r % 4);
                if (key > qpos) s[r] = -INFINITY;
            }
        }
        float mt = s[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mt = fmaxf(mt, s[r]);
        {
            float lo, hi;
            pair32(mt, lo, hi);
            mt = fmaxf(lo, hi);
        }
        // Each query keeps a reference maximum and moves it only when the new
        // maximum exceeds it by more than 8 (log2 units): the exponentials
        // stay below 2^8 and the accumulator rescale is skipped for most
        // tiles (any reference gives the same normalised result).
        const float m_max = fmaxf(m_run, mt);
        const float m_new = (m_max > m_run + 8.f || m_run == -INFINITY) ? m_max : m_run;
        // a segment may start with a tile that is all masked for a row
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        const float alpha = fast_exp2(m_run - m_use);
        float psum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            s[r] = fast_exp2(s[r] - m_use);
            psum += s[r];
        }
        {
            float lo, hi;
            pair32(psum, lo, hi);
            psum = lo + hi;
        }
        l_run = fmaf(l_run, alpha, psum);
        m_run = m_new;
        // rescale only when some query's running max moved
        if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {
#pragma unroll
            for (int tt = 0; tt < NT; ++tt)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[tt][r] *= alpha;
        }
        // PV: k-step (sb, e) takes key 8sb + 4qg + e of the tile
#pragma unroll
        for (int sb = 0; sb < 4; ++sb)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float *vr = &sV[(8 * sb + 4 * qg + e) * HD + NT * qi];
                if constexpr (NT == 4) {
                    const float4 v4 = ld4(vr);
                    acc[0] = mfma32(v4.x, s[4 * sb + e], acc[0]);
                    acc[1] = mfma32(v4.y, s[4 * sb + e], acc[1]);
                    acc[2] = mfma32(v4.z, s[4 * sb + e], acc[2]);
                    acc[3] = mfma32(v4.w, s[4 * sb + e], acc[3]);
                } else {
                    const float2 v2 = *reinterpret_cast<const float2 *>(vr);
                    acc[0] = mfma32(v2.x, s[4 * sb + e], acc[0]);
                    acc[1] = mfma32(v2.y, s[4 * sb + e], acc[1]);
                }
            }
    };

    // key tiles of this workgroup: a key segment, a half of a split item
    // (the plan splits only items of at least two tiles), or all of them
    const int t_half = n_tiles / 2;
    const int t_begin = part == 2 ? t_half : seg * a.seg_tiles;
    const int t_end = part == 1 ? t_half : (a.n_kseg == 1 ? n_tiles : min(n_tiles, t_begin + a.seg_tiles));
    if (t_begin < t_end) issue_tile(sK0, sV0, t_begin);
    load_q();
    for (int t = t_begin; t < t_end; t += 2) {
        // this wave's loads of tile t have landed; after the barrier every
        // wave's have, and every wave is done with the other buffer
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (t + 1 < t_end) issue_tile(sK1, sV1, t + 1);
        compute_tile(sK0, sV0, t);
        if (t + 1 >= t_end) break;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (t + 2 < t_end) issue_tile(sK0, sV0, t + 2);
        compute_tile(sK1, sV1, t + 1);
    }

    // output: lane (qi, qg) register r of block tt is dim NT i + tt with
    // i = 8 (r / 4) + 4 qg + r % 4, so the NT blocks give NT consecutive dims
    auto store_row = [&](float *dst, float sc) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int i = 8 * (r / 4) + 4 * qg + (r % 4);
            if constexpr (NT == 4)
                st4(dst + 4 * i, make_float4(acc[0][r] * sc, acc[1][r] * sc, acc[2][r] * sc, acc[3][r] * sc));
            else
                *reinterpret_cast<float2 *>(dst + 2 * i) = make_float2(acc[0][r] * sc, acc[1][r] * sc);
        }
    };
    if (a.n_kseg > 1 || part != 0) {
        if (!active) return;
        const size_t pe = part != 0 ? (((size_t)g * a.n_split + item) * 4 + wave) * 2 + (part - 1)
                                    : ((size_t)g * total + ee) * a.n_kseg + seg;
        store_row(a.part_o + (pe * 32 + qi) * HD, 1.f);
        if (qg == 0) {
            a.part_ml[(pe * 32 + qi) * 2 + 0] = m_run;
            a.part_ml[(pe * 32 + qi) * 2 + 1] = l_run;
        }
        return;
    }
    if (qvalid) store_row(a.out + ((size_t)qrow * n_head + h) * HD, 1.f / l_run);
}

// Block = one (kv-head, strip, q-head) entry of the prefill: the log-sum-exp
// merge of its key segments (or of the two halves of a split item) for 32
// query rows; thread (row r, chunk c) owns HD / 8 dims of one row.
template <int HD>
__global__ __launch_bounds__(256) void prefill_combine_kernel(PrefillArgs a) {
    constexpr int CH = HD / 8;                          // dims per thread
    const int total = a.n_rep * a.n_strips;
    int g, e, S;
    size_t base;
    if (a.n_split > 0) {
        // block = (kv-head, split item, wave) of the split plan
        const int id = blockIdx.x, gi = id >> 2;
        g = gi / a.n_split;
        e = (gi - g * a.n_split) * 4 + (id & 3);
        if (e >= total) return;
        S = 2;
        base = (size_t)id * 2;
    } else {
        const int entry = blockIdx.x;
        g = entry / total;
        e = entry - g * total;
        S = a.n_kseg;
        base = (size_t)entry * S;
    }
    const int strip = a.n_strips - 1 - e / a.n_rep;
    const int h = g * a.n_rep + e % a.n_rep;
    const int r = threadIdx.x >> 3, c = threadIdx.x & 7;
    const int qrow = 32 * strip + r;
    if (qrow >= a.n_tok) return;
    // segments in batches of four, every load of a batch issued before its
    // arithmetic (one memory round trip per batch); the sums in segment order
    constexpr int kSeg = 4;
    const float2 *ml = reinterpret_cast<const float2 *>(a.part_ml);
    float m = -INFINITY;
    for (int s0 = 0; s0 < S; s0 += 2 * kSeg) {
        float mv[2 * kSeg];
#pragma unroll
        for (int u = 0; u < 2 * kSeg; ++u) mv[u] = s0 + u < S ? ml[(base + s0 + u) * 32 + r].x : -INFINITY;
#pragma unroll
        for (int u = 0; u < 2 * kSeg; ++u) m = fmaxf(m, mv[u]);
    }
    float den = 0.f;
    float4 acc[CH / 4];
#pragma unroll
    for (int j = 0; j < CH / 4; ++j) acc[j] = zero4();
    for (int s0 = 0; s0 < S; s0 += kSeg) {
        float2 st[kSeg];
        float4 x[kSeg][CH / 4];
#pragma unroll
        for (int u = 0; u < kSeg; ++u)
            if (s0 + u < S) {
                st[u] = ml[(base + s0 + u) * 32 + r];
                const float *po = a.part_o + ((base + s0 + u) * 32 + r) * HD + c * CH;
#pragma unroll
                for (int j = 0; j < CH / 4; ++j) x[u][j] = ld4(po + 4 * j);
            }
#pragma unroll
        for (int u = 0; u < kSeg; ++u)
            if (s0 + u < S) {
                const float w = st[u].x == -INFINITY ? 0.f : exp2f(st[u].x - m);
                den = fmaf(w, st[u].y, den);
#pragma unroll
                for (int j = 0; j < CH / 4; ++j) {
                    acc[j].x = fmaf(w, x[u][j].x, acc[j].x);
                    acc[j].y = fmaf(w, x[u][j].y, acc[j].y);
                    acc[j].z = fmaf(w, x[u][j].z, acc[j].z);
                    acc[j].w = fmaf(w, x[u][j].w, acc[j].w);
                }
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

// ------------------------------------------------------- fixed scratch

// Split partials of kore_attn_decode_noalloc_dev: every GPU holds its own copy
// of this array for the life of the process, and every call on that GPU
// shares it.  Host code never passes the array's name to a kernel (on the
// host it names a stand-in, not device memory); it passes the address that
// hipGetSymbolAddress gives for the current device.
static __device__ __align__(256) float scratch[kStaticScratchFloats];

// --------------------------------------------------------------- dispatch

// Dynamic LDS that brings a kernel's static LDS up to `total` bytes (0 if it
// is there already or the attributes cannot be read).
unsigned dyn_lds_above(const void *kernel, size_t total) {
    hipFuncAttributes fa{};
    if (hipFuncGetAttributes(&fa, kernel) != hipSuccess) return 0u;
    return fa.sharedSizeBytes < total ? (unsigned)(total - fa.sharedSizeBytes) : 0u;
}

template <int HD, int NR>
hipError_t launch_decode_nr(const DecodeArgs &a, const RopeRow &rr, hipStream_t s) {
    // The leading scalar arguments (everything before the first aggregate:
    // the pointers and sizes the first loads need, the new row's included)
    // are preloaded into SGPRs at wave launch (gfx950 kernel-argument
    // preload, at most 16 dwords), so no load is issued behind a
    // kernel-argument fetch.
    // Splits of at most kWaves blocks plus kWaves extra rows give every wave
    // one block at most: that kernel has no prefetch registers or branches.
    // With at most as many workgroups as CUs, the single-block kernel asks
    // for enough (unused) dynamic LDS that a CU holds one (it fits two by
    // registers, and two on a CU would leave another idle); with twice as
    // many (wg_per_cu 2) every CU holds two.
    const dim3 grid(a.n_split, a.n_head_kv);
    if (a.rows_per_split > kWaves * kDecodeBlock + kWaves) {
        // one per CU; the head_dim-64 instances would fit two by registers
        static const unsigned pad_m =
            dyn_lds_above(reinterpret_cast<const void *>(&decode_multi_kernel<HD, NR>), kLdsPerCu / 2 + 256);
        hipLaunchKernelGGL((decode_multi_kernel<HD, NR>), grid, dim3(kThreads), pad_m, s, a.q, a.kc, a.vc, a.k, a.v,
                           a.n_rows, a.rows_per_split, a.new_slot, a.slots, a, rr);
    } else {
        // enough (unused) dynamic LDS that a CU holds exactly the workgroups
        // the grid plans for it: more than half the CU's LDS for one, more
        // than a third for two (the instances with few registers, head_dim 64
        // or 3 q-heads per kv-head, would otherwise fit three or more, and a
        // CU holding three leaves another with one)
        static const unsigned pad[2] = {[] {
            return dyn_lds_above(reinterpret_cast<const void *>(&decode_split_kernel<HD, NR>), kLdsPerCu / 2 + 256);
        }(), [] {
            return dyn_lds_above(reinterpret_cast<const void *>(&decode_split_kernel<HD, NR>), kLdsPerCu / 3 + 256);
        }()};
        hipLaunchKernelGGL((decode_split_kernel<HD, NR>), grid, dim3(kThreads), pad[a.wg_per_cu == 2 ? 1 : 0], s,
                           a.q, a.kc, a.vc, a.k, a.v, a.n_rows, a.rows_per_split, a.new_slot, a.slots, a, rr);
    }
    static_assert(kMaxDecodeSplits <= 8 * 32, "the combine takes at most 32 splits per lane");
    const dim3 cgrid(a.n_head_kv * a.n_rep, HD / 32);
    const float *po = a.part_o, *pml = a.part_ml;
    if (a.n_split > 128) hipLaunchKernelGGL((decode_combine_kernel<HD, 32>), cgrid, dim3(64), 0, s, po, pml, a.out, a.n_split);
    else if (a.n_split > 64) hipLaunchKernelGGL((decode_combine_kernel<HD, 16>), cgrid, dim3(64), 0, s, po, pml, a.out, a.n_split);
    else if (a.n_split > 32) hipLaunchKernelGGL((decode_combine_kernel<HD, 8>), cgrid, dim3(64), 0, s, po, pml, a.out, a.n_split);
    else if (a.n_split > 16) hipLaunchKernelGGL((decode_combine_kernel<HD, 4>), cgrid, dim3(64), 0, s, po, pml, a.out, a.n_split);
    else if (a.n_split > 1) hipLaunchKernelGGL((decode_combine_kernel<HD, 2>), cgrid, dim3(64), 0, s, po, pml, a.out, a.n_split);
    return hipGetLastError();
}

template <int HD>
hipError_t launch_decode_hd(const DecodeArgs &a, const RopeRow &rr, hipStream_t s) {
    switch (a.n_rep) {
        case 1: return launch_decode_nr<HD, 1>(a, rr, s);
        case 2: return launch_decode_nr<HD, 2>(a, rr, s);
        case 3: return launch_decode_nr<HD, 3>(a, rr, s);
        case 4: return launch_decode_nr<HD, 4>(a, rr, s);
        case 5: return launch_decode_nr<HD, 5>(a, rr, s);
        case 6: return launch_decode_nr<HD, 6>(a, rr, s);
        case 7: return launch_decode_nr<HD, 7>(a, rr, s);
        case 8: return launch_decode_nr<HD, 8>(a, rr, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

#ifdef KORE_DECODE_TIMELINE
// Timing build only: the stamps of the latest decode_split_kernel launch
// ([workgroup * 4 + wave][kTlStamps]) and decode_combine_kernel launch
// ([workgroup][kTlCombStamps]), after a device synchronisation.
extern "C" __attribute__((visibility("default"))) int kore_attn_tl_read(unsigned long long *split, size_t split_words,
                                                                        unsigned long long *comb, size_t comb_words) {
    if (split_words > sizeof(g_tl_split) / 8 || comb_words > sizeof(g_tl_comb) / 8) return -1;
    if (hipDeviceSynchronize() != hipSuccess) return -4;
    if (split_words && hipMemcpyFromSymbol(split, HIP_SYMBOL(g_tl_split), split_words * 8) != hipSuccess) return -4;
    if (comb_words && hipMemcpyFromSymbol(comb, HIP_SYMBOL(g_tl_comb), comb_words * 8) != hipSuccess) return -4;
    return 0;
}
#endif

hipError_t static_scratch(int device, float **ptr) {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static float *addr[kMaxDevices] = {};
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        addr[device] = static_cast<float *>(p);
    }
    *ptr = addr[device];
    return hipSuccess;
}

bool decode_supported(int head_dim, int n_rep) {
    return (head_dim == 64 || head_dim == 128) && n_rep >= 1 && n_rep <= 8;
}

bool prefill_supported(int head_dim, int n_rep) {
    return (head_dim == 64 || head_dim == 128) && n_rep >= 1;
}

int decode_rows_per_split(int head_dim, int n_rows, int n_head_kv, int num_cu) {
    // S = num_cu / n_head_kv splits per kv-head (one workgroup per CU; at
    // most kMaxDecodeSplits, and at least kDecodeBlock rows per split) of
    // ceil(n_rows / S) rows.  A split is processed as whole blocks of
    // kDecodeBlock rows (MFMA) plus up to kWaves extra rows (VALU, one per
    // wave), so a row count a little over a multiple of the blocks does not
    // cost a wave a second block; a larger remainder is rounded up to a
    // whole block while that stays within one block per wave (fewer splits,
    // the same blocks per wave).  Past that a wave takes a second block
    // whether the last one is whole or not, and rounding up would leave CUs
    // idle (4420 rows of a 4-kv-head model: 56 splits of 80 instead of 64
    // of 70).  When one workgroup per CU would need a second block per wave
    // (the multi-block kernel), twice the splits are taken if that brings
    // every split back to one block per wave: the single-block kernel then
    // runs two workgroups per CU (7B at 8191 rows: 11.7 against 13.7 us per
    // layer; 3B at 16383: 12.3 against 13.6).  At the same row count one
    // workgroup per CU is faster (the second wave on each SIMD stages its q
    // and scores its single row on the same SIMD; 7B at 4095 rows: 10.7
    // against 8.2 us).  The
    // multi-block kernel at two per CU (one register set, q read from LDS per
    // block, no spills) won only where every wave got the same two or three
    // blocks (3B at 32767: 19.1 against 19.6 us) and lost elsewhere (3B at
    // 24575: 17.4 against 16.1), so longer splits stay at one per CU.
    (void)head_dim;
    auto rows_for = [&](int cus) {
        const int S = std::max(1, std::min({cus / std::max(n_head_kv, 1), kMaxDecodeSplits, n_rows / kDecodeBlock}));
        int rps = std::max(1, (n_rows + S - 1) / S);
        const int up = (rps + kDecodeBlock - 1) / kDecodeBlock * kDecodeBlock;
        if (rps % kDecodeBlock > kWaves && up <= kWaves * kDecodeBlock) rps = up;
        return rps;
    };
    const int single = kWaves * kDecodeBlock + kWaves;
    const int r1 = rows_for(num_cu);
    if (r1 <= single) return r1;
    const int r2 = rows_for(2 * num_cu);
    return r2 <= single ? r2 : r1;
}

hipError_t launch_decode(const DecodeArgs &a, const RopeRow &rr, int head_dim, hipStream_t s) {
    if (head_dim == 128) return launch_decode_hd<128>(a, rr, s);
    if (head_dim == 64) return launch_decode_hd<64>(a, rr, s);
    return hipErrorInvalidValue;
}

hipError_t launch_append(const AppendArgs &a, int head_dim, hipStream_t s) {
    // four tokens per workgroup (threadIdx.y), a kv-head per blockIdx.y
    constexpr int kTok = 4;
    const dim3 grid((a.n_tok + kTok - 1) / kTok, a.n_head_kv);
    const int threads = head_dim / 2 >= 64 ? 64 : (head_dim / 2 > 0 ? head_dim / 2 : 1);
    hipLaunchKernelGGL(append_kernel, grid, dim3(threads, kTok), 0, s, a, head_dim);
    return hipGetLastError();
}

int prefill_key_segments(int n_tok, int pos0, int n_head_kv, int n_rep, int num_cu, int *seg_tiles) {
    // Split the key range when the workgroups of a chunk do not fill every
    // CU (two fit per CU): as many segments as keep all of them in one wave
    // of two per CU, each of at least 2 key tiles.  A 64-row chunk has 16
    // workgroups (7B): unsplit, each walks all its key tiles alone.
    const int n_strips = (n_tok + 31) / 32;
    const int n_wg = (n_rep * n_strips + 3) / 4 * n_head_kv;
    const int n_tiles = (pos0 + n_tok - 1) / 32 + 1;
    int n_kseg = 1;
    if (n_wg < num_cu)
        n_kseg = std::max(1, std::min(2 * num_cu / n_wg, n_tiles / 2));
    *seg_tiles = (n_tiles + n_kseg - 1) / n_kseg;
    return n_kseg;
}

void prefill_split_plan(PrefillArgs &a, int num_cu) {
    // Two workgroups fit per CU and the grid is folded so that each CU's pair
    // adds up to about the mean work; with between one and two workgroups per
    // CU some CUs hold one item only, while the pairs' sums run up to about
    // the longest item plus the shortest.  Splitting the longest items into
    // two halves of their key tiles fills the grid to two per CU and lets the
    // pairs (r-th longest unit with the r-th shortest) even out.
    a.n_split = 0;
    a.n_units = 0;
    const int items = (a.n_rep * a.n_strips + 3) / 4;
    const int n_wg = items * a.n_head_kv;
    if (a.n_kseg != 1 || n_wg < num_cu || n_wg >= 2 * num_cu) return;
    const int n_keys = a.pos0 + a.n_tok;
    auto tiles = [&](int i) {   // key tiles of item i (its first entry's strip)
        const int strip0 = a.n_strips - 1 - (4 * i) / a.n_rep;
        return std::min(a.pos0 + 32 * strip0 + 31, n_keys - 1) / 32 + 1;
    };
    int split = std::min(items, (2 * num_cu - n_wg) / a.n_head_kv);
    while (split > 0 && tiles(split - 1) < 4) --split;   // halves of at least two tiles
    if (split == 0 || items + split > kMaxPrefillUnits) return;
    struct Unit { int tiles, code; };
    std::vector<Unit> u;
    u.reserve(items + split);
    for (int i = 0; i < items; ++i) {
        const int t = tiles(i);
        if (i < split) {
            u.push_back({t / 2, i << 2 | 1});
            u.push_back({t - t / 2, i << 2 | 2});
        } else {
            u.push_back({t, i << 2});
        }
    }
    std::stable_sort(u.begin(), u.end(), [](const Unit &x, const Unit &y) { return x.tiles > y.tiles; });
    for (size_t r = 0; r < u.size(); ++r) a.unit[r] = (uint16_t)u[r].code;
    a.n_split = split;
    a.n_units = (int)u.size();
}

hipError_t launch_prefill(const PrefillArgs &a, int head_dim, hipStream_t s) {
    const int items = (a.n_rep * a.n_strips + 3) / 4;
    const dim3 grid(a.n_split > 0 ? a.n_units * a.n_head_kv : items * a.n_head_kv * a.n_kseg);
    if (head_dim == 128) hipLaunchKernelGGL(prefill_kernel<128>, grid, dim3(kThreads), 0, s, a);
    else if (head_dim == 64) hipLaunchKernelGGL(prefill_kernel<64>, grid, dim3(kThreads), 0, s, a);
    else return hipErrorInvalidValue;
    if (a.n_split > 0) {
        const dim3 cgrid(a.n_head_kv * a.n_split * 4);
        if (head_dim == 128) hipLaunchKernelGGL(prefill_combine_kernel<128>, cgrid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL(prefill_combine_kernel<64>, cgrid, dim3(256), 0, s, a);
    } else if (a.n_kseg > 1) {
        const dim3 cgrid(a.n_head_kv * a.n_rep * a.n_strips);
        if (head_dim == 128) hipLaunchKernelGGL(prefill_combine_kernel<128>, cgrid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL(prefill_combine_kernel<64>, cgrid, dim3(256), 0, s, a);
    }
    return hipGetLastError();
}

bool generic_supported(int head_dim) {
    return head_dim >= 2 && head_dim <= kMaxGenericHeadDim && head_dim % 2 == 0;
}

void generic_shape(int head_dim, int n_rep, int *tile, int *chunk, int *n_chunks) {
    // K and V tiles within 40 KB; a tile's rows fit one wave (softmax); at
    // most 1024 (head, dim) outputs (4 per thread) and 1024 (head, row) scores.
    int T = 64;
    while (T > 8 && (size_t)T * (2 * head_dim + 1) * sizeof(float) > 40 * 1024) T /= 2;
    const int ch = std::max(1, std::min({n_rep, 1024 / head_dim, 1024 / T}));
    *tile = T;
    *chunk = ch;
    *n_chunks = (n_rep + ch - 1) / ch;
}

size_t generic_lds_bytes(int head_dim, int tile, int chunk) {
    const size_t T = tile, C = chunk, hd = head_dim;
    return C * T * sizeof(double) + (C * T + 3 * C + C * hd + T * (hd + 1) + T * hd) * sizeof(float);
}

int generic_max_split(int head_dim, int n_rep, int n_head_kv, int num_cu) {
    int T, ch, nc;
    generic_shape(head_dim, n_rep, &T, &ch, &nc);
    return std::max(1, std::min(kMaxGenericSplits, num_cu / std::max(1, n_head_kv * nc)));
}

int generic_rows_per_split(int head_dim, int n_rep, int n_rows, int n_head_kv, int num_cu) {
    // at most generic_max_split splits, each whole tiles (the last one shorter)
    int T, ch, nc;
    generic_shape(head_dim, n_rep, &T, &ch, &nc);
    const int S = std::max(1, std::min(generic_max_split(head_dim, n_rep, n_head_kv, num_cu), (n_rows + T - 1) / T));
    const int rps = std::max(1, (n_rows + S - 1) / S);
    return (rps + T - 1) / T * T;
}

hipError_t launch_generic_decode(const GenericArgs &a, const float *q, const float *k, const float *v,
                                 float *q_out, float *kc, float *vc, int n_head, int new_slot, const RopeRow &rr,
                                 hipStream_t s) {
    hipLaunchKernelGGL(generic_decode_prep_kernel, dim3(n_head + a.n_head_kv), dim3(64), 0, s, q, k, v, q_out, kc,
                       vc, n_head, a.hd, a.slots, new_slot, rr);
    const size_t lds = generic_lds_bytes(a.hd, a.tile, a.chunk);
    hipLaunchKernelGGL(generic_attend_kernel, dim3(a.n_split, a.n_head_kv * a.n_chunks), dim3(kThreads), lds, s, a);
    if (a.n_split > 1)
        hipLaunchKernelGGL(generic_combine_kernel, dim3(n_head), dim3(std::min(256, (a.hd + 63) / 64 * 64)), 0, s,
                           a.part_o, a.part_ml, a.out, a.n_split, a.hd);
    return hipGetLastError();
}

hipError_t launch_generic_prefill(const GenericArgs &a, int n_tok, hipStream_t s) {
    const size_t lds = generic_lds_bytes(a.hd, a.tile, a.chunk);
    hipLaunchKernelGGL(generic_attend_kernel, dim3(n_tok, a.n_head_kv * a.n_chunks), dim3(kThreads), lds, s, a);
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
