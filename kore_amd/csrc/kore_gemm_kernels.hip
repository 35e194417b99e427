// kore_gemm_kernels.hip - gfx950 kernels of kore's batched prefill matmul
// (matmul_batch_float, kore.cpp:783-845): out[b][r] = row r of the
// dequantised Q4_K / Q6_K weights . x[b] for B <= 64 activations at once, for
// up to four matrices that share x in one launch.  Two paths:
//
// fp16 (the default; described with its kernels below): the weights enter
// v_mfma_f32_32x32x16_f16 as exact small integers and the activations as fp16
// hi + lo parts, with kore's block scales applied per block in fp32.
//
// fp32 (KORE_GEMM=fp32, kept for comparisons): v_mfma_f32_16x16x4f32 on
// weights dequantised in registers: a wave owns 16 rows of a 64-row tile and
// up to 64 activations (NB blocks of 16); lane l supplies row l % 16 and, of
// every 256-column block, the 64 columns of group l / 16 (the order of the K
// sum inside a block is permuted so that each lane dequantises contiguous
// bytes; the sum is the same up to fp32 rounding).  The activations of a
// block are staged in LDS, each of them a 260-float row so the 16-byte reads
// of 16 consecutive activations hit different banks.  The next block's
// activations and weights are loaded into registers while the current
// block's MFMAs run.
//
// Work split (both paths): stream-K.  The iteration space (tile, block) of all
// matrices is cut into `workers` contiguous runs of equal length, one per
// workgroup, so every CU gets the same number of block iterations whatever
// the shapes.  A tile split between workers leaves one partial sum per worker
// in a slot of the workspace (slot 2p for worker p's first tile, 2p + 1 for
// its last), and a second launch adds each split tile's slots in worker order.
// (Finishing split tiles inside the first launch would need device-scope
// fences, which write back and invalidate the XCD's L2 each time and cost far
// more than the second launch.)
//
// kore sums each output in one fused multiply-add chain over the columns; both
// paths sum in MFMA blocks, so results agree with kore's to rounding (kore's
// own tolerance, max|d| <= 1e-4 max|ref| + 1e-6, kore_kernels.cpp:742), not
// bit for bit.  For one device, shape and B the result is deterministic.
#include "kore_qmv_kernels.h"
#include "kore_g16_split.h"
#include "kore_swiglu.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <mutex>

namespace kore_qmv_gpu {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kXStride = 260;           // floats per staged activation row

__device__ __forceinline__ float f16f(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

__device__ __forceinline__ uint32_t word(const uint4 &a, const uint4 &b, int k) {   // word k of 8
    const uint4 &v = k < 4 ? a : b;
    const int m = k & 3;
    return m == 0 ? v.x : m == 1 ? v.y : m == 2 ? v.z : v.w;
}

__device__ __forceinline__ int q4s(const uint4 &h, int j) {   // 6-bit scale of sub-block j
    const int s = 8 * (j & 3);
    return j < 4 ? (int)((h.y >> s) & 63) : (int)(((h.w >> s) & 0x0F) | (((h.y >> (s + 6)) & 3) << 4));
}
__device__ __forceinline__ int q4m(const uint4 &h, int j) {   // 6-bit min of sub-block j
    const int s = 8 * (j & 3);
    return j < 4 ? (int)((h.z >> s) & 63) : (int)(((h.w >> (s + 4)) & 0x0F) | (((h.z >> (s + 6)) & 3) << 4));
}

// One lane's weights of one block.  Q4_K (group kk: 32 nibble bytes + header):
// v[0] header, v[1..2] bytes 16 + 32 kk ...  Q6_K (lane kk = 2 h + j): v[0..1]
// the 32 ql bytes 64 h + 32 j ..., whose low and high nibbles are the low bits
// of values 128 h + 32 j + l and 128 h + 32 (j + 2) + l; v[2..3] the 32 qh bytes
// of half h (2 high bits of each of those values); sc the 8 scale bytes of half
// h; d the f16 scale.
template <bool Q6>
struct WRaw {
    uint4 v[Q6 ? 4 : 3];
    uint32_t sc[Q6 ? 2 : 1], d;
};

template <bool Q6>
__device__ __forceinline__ void load_w(WRaw<Q6> &g, const GemmMat &m, int row, int blk, int nblk, int kk) {
    if (!Q6 || m.type == kQ4K) {
        const uint8_t *b = m.w + ((int64_t)row * nblk + blk) * kQ4Bytes;
        g.v[0] = *(const uint4 *)b;
        g.v[1] = *(const uint4 *)(b + 16 + 32 * kk);
        g.v[2] = *(const uint4 *)(b + 32 + 32 * kk);
    } else if constexpr (Q6) {
        const uint8_t *b = m.w + ((int64_t)row * nblk + blk) * kQ6Body;
        const int h = kk >> 1, j = kk & 1;
        g.v[0] = *(const uint4 *)(b + 64 * h + 32 * j);
        g.v[1] = *(const uint4 *)(b + 64 * h + 32 * j + 16);
        g.v[2] = *(const uint4 *)(b + 128 + 32 * h);
        g.v[3] = *(const uint4 *)(b + 128 + 32 * h + 16);
        const uint2 sc = *(const uint2 *)(b + 192 + 8 * h);
        g.sc[0] = sc.x;
        g.sc[1] = sc.y;
        g.d = m.wd[(int64_t)row * nblk + blk];
    }
}

// One block: acc[nb] += W(16 rows x 256) . X(256 x 16 activations of block nb).
// Step t4 covers columns 64 kk + 4 t4 .. + 3 of the lane: its activations are
// read from LDS one step ahead (bx double buffer) and its four weights
// dequantised before its 4 NB MFMAs, so neither LDS latency nor the
// dequantisation chain sits in front of an MFMA.
template <int NB>
__device__ __forceinline__ void read_bx(floatx4 *bx, const float *xs, int i, int col) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) bx[nb] = *(const floatx4 *)&xs[(16 * nb + i) * kXStride + col];
}

template <int NB>
__device__ __forceinline__ void mfma_step(const float *av, const floatx4 *bx, floatx4 *acc) {
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[tt], bx[nb][tt], acc[nb], 0, 0, 0);
}

template <int NB, bool Q6>
__device__ __forceinline__ void block_q4(const WRaw<Q6> &g, const float *xs, int i, int kk, floatx4 *acc) {
    // kore's dequant_block_q4_K (kore.cpp:337-353): d1 = d*sc, m1 = dmin*min, value = d1*q - m1
    const uint4 &hdr = g.v[0];
    const float d = f16f(hdr.x & 0xFFFFu), dmin = f16f(hdr.x >> 16);
    const float d1 = d * (float)q4s(hdr, 2 * kk), m1 = dmin * (float)q4m(hdr, 2 * kk);
    const float d2 = d * (float)q4s(hdr, 2 * kk + 1), m2 = dmin * (float)q4m(hdr, 2 * kk + 1);
    floatx4 bx[2][NB];
    read_bx<NB>(bx[0], xs, i, 64 * kk);
#pragma unroll
    for (int t4 = 0; t4 < 16; ++t4) {
        // the next step's reads go out first, a whole step before their use
        __builtin_amdgcn_sched_barrier(0);
        if (t4 + 1 < 16) read_bx<NB>(bx[(t4 + 1) & 1], xs, i, 64 * kk + 4 * (t4 + 1));
        __builtin_amdgcn_sched_barrier(0);
        float av[4];
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
            const int tk = 4 * t4 + tt;              // column 64 kk + tk of the block
            const int byte = tk & 31;
            const uint32_t w = word(g.v[1], g.v[2], byte >> 2);
            const uint32_t q = (w >> (8 * (byte & 3) + (tk >= 32 ? 4 : 0))) & 15u;
            av[tt] = tk < 32 ? d1 * (float)q - m1 : d2 * (float)q - m2;
        }
        mfma_step<NB>(av, bx[t4 & 1], acc);
    }
}

template <int NB>
__device__ __forceinline__ void block_q6(const WRaw<true> &g, const float *xs, int i, int kk, floatx4 *acc) {
    // kore's dequant_block_q6_K (kore.cpp:359-381): value = (d * sc) * (q6 - 32).  Lane
    // kk = 2 h + j takes values tk = 0..63 at column 128 h + 32 (j + 2 a) + l, a = tk / 32,
    // l = tk % 32: low bits from nibble a of ql byte l, high bits 2 (j + 2 a) of qh byte l,
    // scale byte 2 (j + 2 a) + l / 16 of the half's eight
    const int h = kk >> 1, j = kk & 1;
    const float d = f16f(g.d);
    float ds[4];                                      // [2 a + l / 16]
#pragma unroll
    for (int e = 0; e < 4; ++e) ds[e] = d * (float)(int)(int8_t)((g.sc[e >> 1] >> (8 * (2 * j + (e & 1)))) & 0xFF);
    const int col0 = 128 * h + 32 * j;
    floatx4 bx[2][NB];
    read_bx<NB>(bx[0], xs, i, col0);
#pragma unroll
    for (int t4 = 0; t4 < 16; ++t4) {
        __builtin_amdgcn_sched_barrier(0);
        if (t4 + 1 < 16) read_bx<NB>(bx[(t4 + 1) & 1], xs, i, col0 + 64 * ((t4 + 1) >> 3) + 4 * ((t4 + 1) & 7));
        __builtin_amdgcn_sched_barrier(0);
        float av[4];
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
            const int tk = 4 * t4 + tt, a = tk >> 5, l = tk & 31;
            const uint32_t lw = word(g.v[0], g.v[1], l >> 2);
            const uint32_t hw = word(g.v[2], g.v[3], l >> 2);
            const uint32_t nib = (lw >> (8 * (l & 3) + 4 * a)) & 15u;
            const uint32_t hb = (hw >> (8 * (l & 3) + 2 * (j + 2 * a))) & 3u;
            av[tt] = ds[2 * a + (l >> 4)] * (float)((int)(nib | (hb << 4)) - 32);
        }
        mfma_step<NB>(av, bx[t4 & 1], acc);
    }
}

__device__ __forceinline__ int mat_of_tile(const GemmArgs &a, int tile) {
    int m = 0;
#pragma unroll
    for (int k = 1; k < kMaxGroup; ++k)
        if (k < a.n_mat && tile >= a.m[k].tile0) m = k;
    return m;
}

// First iteration of worker p's run, and the worker whose run holds iteration
// `it` (the largest p with run_first(p) <= it; runs are never empty because
// the host keeps workers <= iterations).
__device__ __forceinline__ int64_t run_first(int64_t T, int P, int p) { return T * p / P; }
__device__ __forceinline__ int run_of(int64_t T, int P, int64_t it) { return (int)(((it + 1) * P - 1) / T); }

// D block of an MFMA: lane l holds rows 4 (l / 16) + v, activation l % 16 of
// each 16-block; rows past the matrix and activations past B are dropped.
// When every 4-row group is whole and 16-byte aligned (rows % 4 == 0, out
// aligned) a lane stores its four rows of an activation as one vector.
template <int NB>
__device__ __forceinline__ void store_tile(const GemmArgs &a, const GemmMat &mt, int tile, int wave, int i, int kk,
                                           const floatx4 *acc) {
    const int r0 = (tile - mt.tile0) * kGemmRowsPerTile + 16 * wave + 4 * kk;
    const bool vec = (mt.rows & 3) == 0 && ((uintptr_t)mt.out & 15) == 0 && ((uintptr_t)mt.bias & 15) == 0;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const int b = 16 * nb + i;
        if (b >= a.B) continue;
        float *o = mt.out + (int64_t)b * mt.rows + r0;
        // kore's q += bq (kore.cpp:1530-1532) and x += o (kore.cpp:1567-1570, 1586-1589)
        floatx4 val = acc[nb];
        if (vec) {
            if (r0 < mt.rows) {
                if (mt.bias) val = val + *(const floatx4 *)(mt.bias + r0);
                if (mt.accumulate) val = *(const floatx4 *)o + val;
                *(floatx4 *)o = val;
            }
        } else {
#pragma unroll
            for (int v = 0; v < 4; ++v)
                if (r0 + v < mt.rows) {
                    float f = val[v];
                    if (mt.bias) f = f + mt.bias[r0 + v];
                    o[v] = mt.accumulate ? o[v] + f : f;
                }
        }
    }
}

// Fix-up launch: workgroup t finishes tile t if the main launch split it, adding
// the partial sums of its workers in worker order.
template <int NB>
__global__ __launch_bounds__(kThreads) void gemm_fixup_kernel(GemmArgs a) {
    const int tile = blockIdx.x, nblk = a.nblk, P = a.workers;
    const int64_t T = (int64_t)a.tiles * nblk, tfirst = (int64_t)tile * nblk;
    const int pf = run_of(T, P, tfirst), pl = run_of(T, P, tfirst + nblk - 1);
    if (pf == pl) return;                        // one worker ran the whole tile and stored it
    const int t = threadIdx.x, l = t & 63, wave = t >> 6, i = l & 15, kk = l >> 4;
    // contributions in worker order, the loads of up to eight contributors in flight at once
    constexpr int kBatch = 8;
    floatx4 acc[NB];
    for (int q0 = pf; q0 <= pl; q0 += kBatch) {
        floatx4 v[kBatch][NB];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int q = min(q0 + u, pl);
            const int slot = 2 * q + (run_first(T, P, q) / nblk == tile ? 0 : 1);
            const floatx4 *src = (const floatx4 *)a.partials + (int64_t)slot * (kGemmSlotFloats / 4);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) v[u][nb] = src[(wave * 4 + nb) * 64 + l];
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                if (q0 + u <= pl) acc[nb] = q0 + u == pf ? v[u][nb] : acc[nb] + v[u][nb];
    }
    store_tile<NB>(a, a.m[mat_of_tile(a, tile)], tile, wave, i, kk, acc);
}

// Q6: the launch holds a Q6_K matrix (the Q4_K-only kernel keeps smaller
// weight records in registers).
template <int NB, bool Q6>
__global__ __launch_bounds__(kThreads, 2) void gemm_kernel(GemmArgs a) {   // two workgroups per CU
    extern __shared__ __align__(16) float xs[];      // [16 NB][kXStride]
    const int t = threadIdx.x, l = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);   // uniform: addresses built from it stay scalar
    const int i = l & 15, kk = l >> 4;
    const int nblk = a.nblk, P = a.workers;
    const int64_t T = (int64_t)a.tiles * nblk;
    // consecutive runs on one XCD (workgroups are dealt to the 8 XCDs in turn),
    // so the workers that share a split tile share an L2
    const int p = (P % 8 == 0) ? (int)(blockIdx.x % 8) * (P / 8) + (int)(blockIdx.x / 8) : (int)blockIdx.x;
    const int64_t it0 = run_first(T, P, p), it1 = run_first(T, P, p + 1);
    if (it0 >= it1) return;
    const int64_t cols = (int64_t)nblk * 256;

    // activation staging: thread t moves float4 t + 256 j of the block, i.e.
    // quad l of activation wave + 4 j (a wave-uniform row: its base address is
    // scalar); activations past B repeat the last one (their MFMA columns are
    // never stored)
    const float *xrow[4 * NB];
#pragma unroll
    for (int j = 0; j < 4 * NB; ++j) xrow[j] = a.x + (int64_t)min(wave + 4 * j, a.B - 1) * cols;
    floatx4 xr[4 * NB];       // native vectors: HIP's float4 is a struct whose copies stay in memory
    auto row_of = [&](int tile, int m) {
        return min((tile - a.m[m].tile0) * kGemmRowsPerTile + 16 * wave + i, a.m[m].rows - 1);
    };

    int tile = (int)(it0 / nblk), blk = (int)(it0 % nblk), seg0 = blk;
    int m = mat_of_tile(a, tile);
    WRaw<Q6> g;
    load_w<Q6>(g, a.m[m], row_of(tile, m), blk, nblk, kk);
#pragma unroll
    for (int j = 0; j < 4 * NB; ++j) xr[j] = *(const floatx4 *)(xrow[j] + 256 * blk + 4 * l);

    floatx4 acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = floatx4{0.f, 0.f, 0.f, 0.f};

    for (int64_t it = it0; it < it1; ++it) {
        __syncthreads();                                 // every wave is done with the previous block
#pragma unroll
        for (int j = 0; j < 4 * NB; ++j) *(floatx4 *)&xs[(wave + 4 * j) * kXStride + 4 * l] = xr[j];
        __syncthreads();
        const WRaw<Q6> gc = g;
        const int cm = m;
        int ntile = tile, nblk_i = blk + 1;
        if (nblk_i == nblk) { nblk_i = 0; ++ntile; }
        if (it + 1 < it1) {                              // the next block, while this one runs
            m = ntile == tile ? m : mat_of_tile(a, ntile);
            load_w<Q6>(g, a.m[m], row_of(ntile, m), nblk_i, nblk, kk);
#pragma unroll
            for (int j = 0; j < 4 * NB; ++j) xr[j] = *(const floatx4 *)(xrow[j] + 256 * nblk_i + 4 * l);
        }
        if constexpr (Q6) {
            if (a.m[cm].type == kQ4K) block_q4<NB, Q6>(gc, xs, i, kk, acc);
            else block_q6<NB>(gc, xs, i, kk, acc);
        } else {
            block_q4<NB, Q6>(gc, xs, i, kk, acc);
        }

        if (it + 1 == it1 || nblk_i == 0) {              // end of this worker's part of the tile
            if (seg0 != 0 || blk + 1 != nblk) {          // split tile: partial sums for the fix-up launch
                const int slot = 2 * p + (it0 / nblk == tile ? 0 : 1);
                floatx4 *mine = (floatx4 *)a.partials + (int64_t)slot * (kGemmSlotFloats / 4);
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) mine[(wave * 4 + nb) * 64 + l] = acc[nb];
            } else {
                store_tile<NB>(a, a.m[cm], tile, wave, i, kk, acc);
            }
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) acc[nb] = floatx4{0.f, 0.f, 0.f, 0.f};
            seg0 = 0;
        }
        tile = ntile;
        blk = nblk_i;
    }
}

// ------------------------------------------------------------- fp16 path
//
// out[b][r] = sum over blocks of d_r * P[b][r] - dmin_r * M[b][r], with
//   P = sum_c A_c x_c, A_c = sc_j q_c (Q4_K, an integer <= 945, exact in fp16)
//   or sc_j (q_c - 32) (Q6_K, |A| <= 4096: an fp16 high part and an exact
//   integer low part), and M = sum_j m_j Sx_j (Q4_K minimums times the
//   activations' sub-block sums): kore's value d*sc*q - dmin*m regrouped, so
//   the results agree with kore's to rounding (kore's tolerance), not bit for
//   bit.  Each activation block is scaled by a power of two s (max |x s| <
//   2^10) and split into fp16 hi + lo (|x s - hi - lo| <= 2^-22 |x s|); the
//   products of an integer weight and an fp16 part are exact in the MFMA's
//   fp32 accumulator, and 1 / s is applied with d.
//
// MFMA v_mfma_f32_32x32x16_f16 (lane layout checked on the GPU): A = the
// activations (32 of them x 16 k), lane l holds activation l % 32 at k 8 (l /
// 32) + e; B = the weights (16 k x 32 rows), lane l holds row l % 32 at the
// same k; D lane l register r = activation 8 (r / 4) + 4 (l / 32) + r % 4 of
// row l % 32.  Within a block, k-step s (16 columns) and half h take the
// nibble dword q = 16 h + s of a Q4_K row (group g = q / 8, dword t = q % 8):
// slots e < 4 are columns 64 g + 4 t + e (low nibbles), e >= 4 columns 64 g +
// 32 + 4 t + e - 4 (high nibbles); the split activations are stored in that
// order, as chunk c = 2 s + h of 8 fp16 per activation, chunk position c ^ (b
// & 15) so that the 16-byte reads of 16 activations hit different banks.  The
// same order gives a Q6_K lane contiguous bytes too (its half h of ql, qh and
// the scales).

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

// One workgroup of 1024 threads per activation row b: the split of x[min(b,
// B - 1)] with one power-of-two scale s for the whole row (max |x s| < 2^10),
// so that 1 / s is applied once per tile instead of once per block; the
// blocks' 1 / s slots all hold it.  The row (up to 32768 values) is read once
// into registers: thread t holds float4 groups t + 1024 j, lane t % 64 of block
// 16 j + t / 64, for the row maximum and then the split (g16_split_group).
constexpr int kPrepThreads = 1024, kPrepPer = 8;
static_assert(kPrepThreads * kPrepPer * 4 >= 32768, "rows of up to 32768 values (kore's 128 blocks)");
__global__ __launch_bounds__(kPrepThreads) void gemm16_prep_kernel(const float *__restrict__ x,
                                                                    uint8_t *__restrict__ x16, int B, int nblk) {
    __shared__ float red[kPrepThreads / 64];
    const int b = blockIdx.x, t = threadIdx.x, lane = t & 63;
    const float4 *row = (const float4 *)(x + (int64_t)min(b, B - 1) * nblk * 256);
    const int n4 = nblk * 64;
    float4 v[kPrepPer];
#pragma unroll
    for (int j = 0; j < kPrepPer; ++j) v[j] = row[min(t + j * kPrepThreads, n4 - 1)];
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < kPrepPer; ++j)
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
    amax = g16_wave_max(amax);
    if (lane == 0) red[t >> 6] = amax;
    __syncthreads();
    amax = red[0];
#pragma unroll
    for (int k = 1; k < kPrepThreads / 64; ++k) amax = fmaxf(amax, red[k]);
    float s1, s2, inv;
    g16_split_scale(amax, s1, s2, inv);
#pragma unroll
    for (int j = 0; j < kPrepPer; ++j) {
        if (t + j * kPrepThreads >= n4) break;         // whole waves: n4 is a multiple of 64
        const float ys[4] = {(v[j].x * s1) * s2, (v[j].y * s1) * s2, (v[j].z * s1) * s2, (v[j].w * s1) * s2};
        g16_split_group(x16, b, (t + j * kPrepThreads) >> 6, lane, ys, inv);
    }
}

// One lane's weights of one block: Q4_K the header and nibble bytes 64 h ..
// 64 h + 63; Q6_K ql bytes 64 h .., qh bytes 32 h .., the half's 8 scales, d.
template <bool Q6>
struct W16 {
    uint4 v[Q6 ? 6 : 5];
    uint2 sc;
    uint32_t d;
};

// Weight loads, non-temporal when nothing reads the same weights again (one
// unit per tile): the streamed weights then leave the split activations in L2.
typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 ld_w4(const uint8_t *p, bool nt) {
    const u32x4v v = nt ? __builtin_nontemporal_load((const u32x4v *)p) : *(const u32x4v *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld_w2(const uint8_t *p, bool nt) {
    const u32x2v v = nt ? __builtin_nontemporal_load((const u32x2v *)p) : *(const u32x2v *)p;
    return make_uint2(v.x, v.y);
}

template <bool Q6>
__device__ __forceinline__ void load_w16(W16<Q6> &g, const GemmMat &m, int row, int blk, int nblk, int h, bool nt) {
    if (!Q6 || m.type == kQ4K) {
        const uint8_t *b = m.w + ((int64_t)row * nblk + blk) * kQ4Bytes;
        g.v[0] = ld_w4(b, nt);
#pragma unroll
        for (int k = 0; k < 4; ++k) g.v[1 + k] = ld_w4(b + 16 + 64 * h + 16 * k, nt);
    } else if constexpr (Q6) {
        const uint8_t *b = m.w + ((int64_t)row * nblk + blk) * kQ6Body;
#pragma unroll
        for (int k = 0; k < 4; ++k) g.v[k] = ld_w4(b + 64 * h + 16 * k, nt);
        g.v[4] = ld_w4(b + 128 + 32 * h, nt);
        g.v[5] = ld_w4(b + 128 + 32 * h + 16, nt);
        g.sc = ld_w2(b + 192 + 8 * h, nt);
        g.d = m.wd[(int64_t)row * nblk + blk];
    }
}

__device__ __forceinline__ uint32_t dword_of(const uint4 *v, int k) {   // dword k of v[0..]
    const uint4 &u = v[k >> 2];
    const int m = k & 3;
    return m == 0 ? u.x : m == 1 ? u.y : m == 2 ? u.z : u.w;
}

// (1024 + byte i, 1024 + byte j) of u as fp16 (0x64 high bytes)
__device__ __forceinline__ half2v magic2(uint32_t u, uint32_t sel) {
    return __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, u, sel));
}

// The activations' A operand of k-step s for tile tt, hi and lo parts.
__device__ __forceinline__ void read_a(const uint8_t *ls, int m, int c, half8 &ahi, half8 &alo) {
    const int off = m * 512 + ((c ^ (m & 15)) * 16);
    ahi = *(const half8 *)(ls + off);
    alo = *(const half8 *)(ls + kG16Lo + off);
}

__device__ __forceinline__ floatx16 mfma16(half8 a, half8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// The A operands (hi, lo) of k-step s for the NT tiles of activations from
// activation am on (am = 32 for the second half of a halves-mode unit).
template <int NT>
__device__ __forceinline__ void read_step(const uint8_t *ls, int l, int s, int am, half8 (*A)[2]) {
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) read_a(ls, am + 32 * tt + (l & 31), 2 * s + (l >> 5), A[tt][0], A[tt][1]);
}

// One Q4_K block: P[tt] = sum_k A x (hi and lo parts); the tiles' MFMA
// chains alternate.
template <int NT, bool Q6>
__device__ __forceinline__ void block16_q4(const W16<Q6> &g, const uint8_t *ls, int l, int am, floatx16 *P) {
    const int h = l >> 5;
    const uint4 &hdr = g.v[0];
    // scales of sub-blocks 4h .. 4h + 3 as fp16 pairs (sc, sc) and (-1024 sc, -1024 sc)
    half2v scp[4], scn[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const _Float16 sc = (_Float16)(float)q4s(hdr, 4 * h + k);
        scp[k] = half2v{sc, sc};
        scn[k] = half2v{(_Float16)(-1024.f) * sc, (_Float16)(-1024.f) * sc};
    }
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) P[tt] = floatx16{};
#pragma unroll
    for (int s = 0; s < 16; ++s) {
        half8 A[NT][2];
        read_step<NT>(ls, l, s, am, A);
        const uint32_t D = dword_of(&g.v[1], s);
        const uint32_t L = D & 0x0F0F0F0Fu, H = (D >> 4) & 0x0F0F0F0Fu;
        const int a = s >> 3;                                   // sub-blocks 4h + 2a (low), + 1 (high)
        half2v w0 = __builtin_elementwise_fma(magic2(L, 0x04010400u), scp[2 * a], scn[2 * a]);
        half2v w1 = __builtin_elementwise_fma(magic2(L, 0x04030402u), scp[2 * a], scn[2 * a]);
        half2v w2 = __builtin_elementwise_fma(magic2(H, 0x04010400u), scp[2 * a + 1], scn[2 * a + 1]);
        half2v w3 = __builtin_elementwise_fma(magic2(H, 0x04030402u), scp[2 * a + 1], scn[2 * a + 1]);
        const half8 bw = {w0[0], w0[1], w1[0], w1[1], w2[0], w2[1], w3[0], w3[1]};
#pragma unroll
        for (int pp = 0; pp < 2; ++pp)
#pragma unroll
            for (int tt = 0; tt < NT; ++tt) P[tt] = mfma16(A[tt][pp], bw, P[tt]);
    }
}

// Q4_K minimums of one block: M[tt] = sum_j m_j Sx_j, k 0..7 the hi parts of
// Sx_0..7 times m_0..7, k 8..15 the lo parts times the same.
template <int NT, bool Q6>
__device__ __forceinline__ void block16_q4_mins(const W16<Q6> &g, const uint8_t *ls, int l, int am, floatx16 *M) {
    const uint4 &hdr = g.v[0];
    half8 bm;
#pragma unroll
    for (int j = 0; j < 8; ++j) bm[j] = (_Float16)(float)q4m(hdr, j);
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
        const half8 sx = *(const half8 *)(ls + kG16Sx + (am + 32 * tt + (l & 31)) * 32 + 16 * (l >> 5));
        M[tt] = mfma16(sx, bm, floatx16{});
    }
}

// One Q6_K block: P[tt] = sum_k (A_hi + A_lo) (x_hi + x_lo) without the lo x lo term.
template <int NT>
__device__ __forceinline__ void block16_q6(const W16<true> &g, const uint8_t *ls, int l, int am, floatx16 *P) {
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) P[tt] = floatx16{};
#pragma unroll
    for (int s = 0; s < 16; ++s) {
        half8 A[NT][2];
        read_step<NT>(ls, l, s, am, A);
        const int a = s >> 3, t = s & 7, sh = 4 * a;
        const uint32_t D1 = dword_of(g.v, t), D2 = dword_of(g.v, 8 + t), Q = dword_of(&g.v[4], t);
        const uint32_t q1 = ((D1 >> sh) & 0x0F0F0F0Fu) | (((Q >> sh) & 0x03030303u) << 4);
        const uint32_t q2 = ((D2 >> sh) & 0x0F0F0F0Fu) | (((Q >> (sh + 2)) & 0x03030303u) << 4);
        // scales of the four values of each half: bytes 4a + (t >= 4) and 4a + 2 + (t >= 4)
        const int si1 = 4 * a + (t >> 2), si2 = si1 + 2;
        const uint32_t scw1 = si1 < 4 ? g.sc.x : g.sc.y, scw2 = si2 < 4 ? g.sc.x : g.sc.y;
        const _Float16 s1 = (_Float16)(float)(int)(int8_t)(scw1 >> (8 * (si1 & 3)));
        const _Float16 s2 = (_Float16)(float)(int)(int8_t)(scw2 >> (8 * (si2 & 3)));
        const half2v m1056 = {(_Float16)(-1056.f), (_Float16)(-1056.f)};
        const half2v v0 = magic2(q1, 0x04010400u) + m1056, v1 = magic2(q1, 0x04030402u) + m1056;
        const half2v v2 = magic2(q2, 0x04010400u) + m1056, v3 = magic2(q2, 0x04030402u) + m1056;
        const half2v c1 = {s1, s1}, c2 = {s2, s2};
        const half2v h0 = v0 * c1, h1 = v1 * c1, h2 = v2 * c2, h3 = v3 * c2;        // fp16(A)
        const half2v l0 = __builtin_elementwise_fma(v0, c1, -h0), l1 = __builtin_elementwise_fma(v1, c1, -h1);
        const half2v l2 = __builtin_elementwise_fma(v2, c2, -h2), l3 = __builtin_elementwise_fma(v3, c2, -h3);
        const half8 bh = {h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
        const half8 bl = {l0[0], l0[1], l1[0], l1[1], l2[0], l2[1], l3[0], l3[1]};
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) P[tt] = mfma16(A[tt][0], bh, P[tt]);
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) P[tt] = mfma16(A[tt][1], bh, P[tt]);
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) P[tt] = mfma16(A[tt][0], bl, P[tt]);
    }
}

// D lane l register r of tile tt: activation am + 32 tt + 8 (r / 4) + 4 (l / 32) + r % 4, row l % 32
template <int NT>
__device__ __forceinline__ void store16(const GemmArgs &a, const GemmMat &mt, int tile, int wave, int l, int am,
                                        const floatx16 *acc) {
    const int row = (tile - mt.tile0) * kG16Rows + 32 * wave + (l & 31);
    if (row >= mt.rows) return;
    const float bias = mt.bias ? mt.bias[row] : 0.f;
#pragma unroll
    for (int tt = 0; tt < NT; ++tt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int b = am + 32 * tt + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
            if (b >= a.B) continue;
            float *o = mt.out + (int64_t)b * mt.rows + row;
            // kore's q += bq (kore.cpp:1530-1532) and x += o (kore.cpp:1567-1570, 1586-1589)
            float f = acc[tt][r];
            if (mt.bias) f = f + bias;
            *o = mt.accumulate ? *o + f : f;
        }
}

// One workgroup of 8 waves per CU (tiles of 256 rows: each activation block's
// split is staged once for 256 rows), two LDS buffers: the next block's split
// activations are copied in (global_load_lds, a linear copy) while the
// current block's MFMAs run.  The two buffers are separate LDS objects and the
// loop is unrolled by two, so the compiler sees that reading one does not
// depend on the copy into the other.  Work units are the tiles, or with
// a.halves = 2 (NT = 1) each tile's two halves of 32 activations (unit 2 tile
// + half): twice the units for launches with few tiles, each staging and
// multiplying half the activations.
constexpr int kG16Threads = 512;

template <int NT, bool Q6>
__global__ __launch_bounds__(kG16Threads, 1) void gemm16_kernel(GemmArgs a) {
    __shared__ __align__(16) uint8_t ls0[kG16BlockBytes];
    __shared__ __align__(16) uint8_t ls1[kG16BlockBytes];
    const int t = threadIdx.x, l = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int h = l >> 5;
    const int nblk = a.nblk, P = a.workers, hv = a.halves;
    const int64_t T = (int64_t)a.tiles * hv * nblk;
    const int p = (P % 8 == 0) ? (int)(blockIdx.x % 8) * (P / 8) + (int)(blockIdx.x / 8) : (int)blockIdx.x;
    const int64_t it0 = run_first(T, P, p), it1 = run_first(T, P, p + 1);
    if (it0 >= it1) return;
    auto row_of = [&](int tile, int m) {
        return min((tile - a.m[m].tile0) * kG16Rows + 32 * wave + (l & 31), a.m[m].rows - 1);
    };
    // a block's split activations: 4240 chunks of 16 bytes, copied linearly:
    // eight rounds of 64 chunks per wave, then the last 144 by waves 0..2
    constexpr int kChunks = kG16BlockBytes / 16;
    constexpr int kRounds = kChunks / (8 * 64);
    static_assert(kG16BlockBytes % 16 == 0 && kChunks - 8 * 64 * kRounds <= 8 * 64, "whole chunks");
    auto stage = [&](uint8_t *dst, int blk) {
        const uint8_t *src = a.x16 + (int64_t)blk * kG16BlockBytes + 16 * l;
#pragma unroll
        for (int k = 0; k < kRounds; ++k) {
            const int c0 = (k * 8 + wave) * 64;
            __builtin_amdgcn_global_load_lds(src + 16 * c0, (void __attribute__((address_space(3))) *)(dst + 16 * c0), 16, 0, 0);
        }
        const int c0 = (kRounds * 8 + wave) * 64;
        if (c0 < kChunks && c0 + l < kChunks)
            __builtin_amdgcn_global_load_lds(src + 16 * c0, (void __attribute__((address_space(3))) *)(dst + 16 * c0), 16, 0, 0);
    };
    // the 32 activations am .. am + 31 of a block (halves mode), at their own
    // offsets: hi and lo (1024 chunks each, four rounds of 64 per wave), the
    // sub-block sums (64 chunks, wave 0) and 1 / s (8 chunks, wave 1)
    auto stage_half = [&](uint8_t *dst, int blk, int am) {
        const uint8_t *src = a.x16 + (int64_t)blk * kG16BlockBytes + 16 * l;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int c0 = (r < 2 ? 0 : kG16Lo / 16) + am * 32 + 64 * (wave + 8 * (r & 1));
            __builtin_amdgcn_global_load_lds(src + 16 * c0, (void __attribute__((address_space(3))) *)(dst + 16 * c0), 16, 0, 0);
        }
        const int cs = kG16Sx / 16 + am * 2, ci = kG16Inv / 16 + am / 4;
        if (wave == 0)
            __builtin_amdgcn_global_load_lds(src + 16 * cs, (void __attribute__((address_space(3))) *)(dst + 16 * cs), 16, 0, 0);
        if (wave == 1 && l < 8)
            __builtin_amdgcn_global_load_lds(src + 16 * ci, (void __attribute__((address_space(3))) *)(dst + 16 * ci), 16, 0, 0);
    };
    auto stage_unit = [&](uint8_t *dst, int blk, int am) {
        if (hv == 1) stage(dst, blk);
        else stage_half(dst, blk, am);
    };
    // acc += d P - dmin M per block, in the rows' scaled units; times 1 / s of
    // each activation when the tile is stored or left as a partial
    floatx16 acc[NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) acc[tt] = floatx16{};
    auto unscale = [&](const uint8_t *ls, int am) {
#pragma unroll
        for (int tt = 0; tt < NT; ++tt)
#pragma unroll
            for (int qd = 0; qd < 4; ++qd) {
                const float4 f = *(const float4 *)(ls + kG16Inv + 4 * (am + 32 * tt + 8 * qd + 4 * h));
                acc[tt][4 * qd + 0] *= f.x;
                acc[tt][4 * qd + 1] *= f.y;
                acc[tt][4 * qd + 2] *= f.z;
                acc[tt][4 * qd + 3] *= f.w;
            }
    };
    auto compute = [&](const uint8_t *ls, const W16<Q6> &gc, int cm, int am) {
        if (Q6 && a.m[cm].type == kQ6K) {
            floatx16 Pb[NT];
            if constexpr (Q6) block16_q6<NT>(gc, ls, l, am, Pb);
            const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)gc.d);
#pragma unroll
            for (int tt = 0; tt < NT; ++tt)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[tt][r] = fmaf(d, Pb[tt][r], acc[tt][r]);
        } else {
            // d P first, then the minimums in the same registers
            floatx16 Pb[NT];
            block16_q4<NT, Q6>(gc, ls, l, am, Pb);
            const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(gc.v[0].x & 0xFFFFu));
            const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(gc.v[0].x >> 16));
#pragma unroll
            for (int tt = 0; tt < NT; ++tt)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[tt][r] = fmaf(d, Pb[tt][r], acc[tt][r]);
            block16_q4_mins<NT, Q6>(gc, ls, l, am, Pb);
#pragma unroll
            for (int tt = 0; tt < NT; ++tt)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[tt][r] = fmaf(-dmin, Pb[tt][r], acc[tt][r]);
        }
    };

    int unit = (int)(it0 / nblk), blk = (int)(it0 % nblk), seg0 = blk;
    int tile = unit / hv, am = (unit % hv) * 32;
    int m = mat_of_tile(a, tile);
    W16<Q6> g;
    load_w16<Q6>(g, a.m[m], row_of(tile, m), blk, nblk, h, hv == 1);
    stage_unit(ls0, blk, am);
    __builtin_amdgcn_s_waitcnt(0x0F70);                // vmcnt(0)
    __syncthreads();

    // one iteration: block `blk` of `unit` from `cur`, the next block's split into `nxt`
    auto step = [&](int64_t it, const uint8_t *cur, uint8_t *nxt) {
        int nunit = unit, nb = blk + 1;
        if (nb == nblk) { nb = 0; ++nunit; }
        const int ntile = nunit / hv, nam = (nunit % hv) * 32;
        const W16<Q6> gc = g;
        const int cm = m;
        if (it + 1 < it1) {                            // the next block's activations and weights
            stage_unit(nxt, nb, nam);
            m = ntile == tile ? m : mat_of_tile(a, ntile);
            load_w16<Q6>(g, a.m[m], row_of(ntile, m), nb, nblk, h, hv == 1);
        }
        compute(cur, gc, cm, am);
        if (it + 1 == it1 || nb == 0) {                // end of this worker's part of the unit
            unscale(cur, am);
            if (seg0 != 0 || blk + 1 != nblk) {        // split unit: partial sums for the fix-up launch
                const int slot = 2 * p + (it0 / nblk == unit ? 0 : 1);
                float *mine = a.partials + (int64_t)slot * kG16SlotFloats;
#pragma unroll
                for (int tt = 0; tt < NT; ++tt)
#pragma unroll
                    for (int r = 0; r < 16; ++r) mine[((wave * 2 + tt) * 16 + r) * 64 + l] = acc[tt][r];
            } else {
                store16<NT>(a, a.m[cm], tile, wave, l, am, acc);
            }
#pragma unroll
            for (int tt = 0; tt < NT; ++tt) acc[tt] = floatx16{};
            seg0 = 0;
        }
        unit = nunit;
        tile = ntile;
        am = nam;
        blk = nb;
        __builtin_amdgcn_s_waitcnt(0x0F70);            // vmcnt(0): the next block's copies have landed
        __syncthreads();                               // ... for every wave, and `cur` is free
    };
    for (int64_t it = it0; it < it1; it += 2) {
        step(it, ls0, ls1);
        if (it + 1 >= it1) break;
        step(it + 1, ls1, ls0);
    }
}

// Fix-up of the fp16 path: blockIdx.x = unit (tile, or tile and half),
// blockIdx.y = a slice of 1024 of its kG16SlotFloats partial floats (slot
// float ((wave 2 + tt) 16 + r) 64 + l is register r of activation tile tt of
// lane l of wave `wave`, 8 waves; a halves-mode unit has tile 0 only); thread
// t adds float4 t of the slice over the unit's workers in worker order, eight
// workers' loads in flight at a time, and stores four consecutive rows of one
// activation.
__global__ __launch_bounds__(kThreads) void gemm16_fixup_kernel(GemmArgs a) {
    const int unit = blockIdx.x, nblk = a.nblk, P = a.workers, hv = a.halves;
    const int tile = unit / hv, am = (unit % hv) * 32;
    const int64_t T = (int64_t)a.tiles * hv * nblk, tfirst = (int64_t)unit * nblk;
    const int pf = run_of(T, P, tfirst), pl = run_of(T, P, tfirst + nblk - 1);
    if (pf == pl) return;                        // one worker ran the whole unit and stored it
    const int f = blockIdx.y * 1024 + 4 * threadIdx.x;   // first of the thread's four floats
    const int l = f & 63, r = (f >> 6) & 15, tt = (f >> 10) & 1, wave = f >> 11;
    if (hv == 2 && tt) return;
    const int b = am + 32 * tt + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
    if (b >= a.B) return;
    // up to eight contributors' loads in flight, only those the unit has
    // (pf and pl are the same for the whole workgroup: uniform branches)
    constexpr int kBatch = 8;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int q0 = pf; q0 <= pl; q0 += kBatch) {
        float4 v[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
            if (q0 + u <= pl) {
                const int q = q0 + u;
                const int slot = 2 * q + (run_first(T, P, q) / nblk == unit ? 0 : 1);
                v[u] = *(const float4 *)(a.partials + (int64_t)slot * kG16SlotFloats + f);
            }
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
            if (q0 + u <= pl) {
                if (q0 + u == pf) acc = v[u];
                else {
                    acc.x += v[u].x;
                    acc.y += v[u].y;
                    acc.z += v[u].z;
                    acc.w += v[u].w;
                }
            }
    }
    const GemmMat &mt = a.m[mat_of_tile(a, tile)];
    const int row0 = (tile - mt.tile0) * kG16Rows + 32 * wave + (l & 31);
    float *o = mt.out + (int64_t)b * mt.rows + row0;
    // kore's q += bq (kore.cpp:1530-1532) and x += o (kore.cpp:1567-1570, 1586-1589)
    if (row0 + 3 < mt.rows && !(((uintptr_t)o | (uintptr_t)(mt.bias ? mt.bias + row0 : nullptr)) & 15)) {
        float4 v = acc;                                // four whole rows, 16-byte aligned
        if (mt.bias) {
            const float4 bb = *(const float4 *)(mt.bias + row0);
            v = make_float4(v.x + bb.x, v.y + bb.y, v.z + bb.z, v.w + bb.w);
        }
        if (mt.accumulate) {
            const float4 ov = *(const float4 *)o;
            v = make_float4(ov.x + v.x, ov.y + v.y, ov.z + v.z, ov.w + v.w);
        }
        *(float4 *)o = v;
        return;
    }
    const float vals[4] = {acc.x, acc.y, acc.z, acc.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int row = row0 + k;
        if (row >= mt.rows) break;
        float v = vals[k];
        if (mt.bias) v = v + mt.bias[row];
        o[k] = mt.accumulate ? o[k] + v : v;
    }
}


// Fix-up of a gate/up pair (GemmArgs::glu): blockIdx.x = gate unit u (tile, or
// tile and half), whose rows and activations up unit u + m[1].tile0 x halves
// shares; blockIdx.y and the thread's float4 as in gemm16_fixup_kernel.  Each
// of the two values comes from its unit's partial sums (added in worker order,
// as the fix-up adds them) when the unit was split, else from the output the
// main kernel stored; m[0].out receives kore's SwiGLU of the pair
// (kore.cpp:1577-1581), bit for bit what the plain fix-up followed by the
// SwiGLU kernel gives.
__global__ __launch_bounds__(kThreads) void gemm16_glu_fixup_kernel(GemmArgs a) {
    const int ug = blockIdx.x, nblk = a.nblk, P = a.workers, hv = a.halves;
    const int tile = ug / hv, am = (ug % hv) * 32;
    const int64_t T = (int64_t)a.tiles * hv * nblk;
    const int f = blockIdx.y * 1024 + 4 * threadIdx.x;   // first of the thread's four floats
    const int l = f & 63, r = (f >> 6) & 15, tt = (f >> 10) & 1, wave = f >> 11;
    if (hv == 2 && tt) return;
    const int b = am + 32 * tt + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
    const int rows = a.m[0].rows, row0 = tile * kG16Rows + 32 * wave + (l & 31);
    if (b >= a.B || row0 >= rows) return;
    const bool whole = row0 + 3 < rows;
    // both units' loads of a batch issued before either is summed (a unit
    // stored whole is read from its output instead); sums in worker order
    constexpr int kBatch = 8;
    auto range = [&](int unit, int &pf, int &pl) {
        pf = run_of(T, P, (int64_t)unit * nblk);
        pl = run_of(T, P, (int64_t)unit * nblk + nblk - 1);
    };
    auto issue = [&](int unit, int pf, int pl, int q0, const float *out, float4 *v) {
        if (pf == pl) {
            const float *o = out + (int64_t)b * rows + row0;
            if (whole && !((uintptr_t)o & 15)) {
                v[0] = *(const float4 *)o;
            } else {
                v[0] = make_float4(o[0], 0.f, 0.f, 0.f);
                if (row0 + 1 < rows) v[0].y = o[1];
                if (row0 + 2 < rows) v[0].z = o[2];
                if (row0 + 3 < rows) v[0].w = o[3];
            }
            return;
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
            if (q0 + u <= pl) {
                const int q = q0 + u;
                const int slot = 2 * q + (run_first(T, P, q) / nblk == unit ? 0 : 1);
                v[u] = *(const float4 *)(a.partials + (int64_t)slot * kG16SlotFloats + f);
            }
    };
    auto add = [&](int pf, int pl, int q0, const float4 *v, float4 &acc) {
        if (pf == pl) {
            acc = v[0];
            return;
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
            if (q0 + u <= pl) {
                if (q0 + u == pf) acc = v[u];
                else {
                    acc.x += v[u].x;
                    acc.y += v[u].y;
                    acc.z += v[u].z;
                    acc.w += v[u].w;
                }
            }
    };
    const int uu = ug + a.m[1].tile0 * hv;
    int pfg, plg, pfu, plu;
    range(ug, pfg, plg);
    range(uu, pfu, plu);
    float4 vg[kBatch], vu[kBatch], g, u;
    issue(ug, pfg, plg, pfg, a.m[0].out, vg);
    issue(uu, pfu, plu, pfu, a.m[1].out, vu);
    add(pfg, plg, pfg, vg, g);
    add(pfu, plu, pfu, vu, u);
    if (pfg != plg)
        for (int q0 = pfg + kBatch; q0 <= plg; q0 += kBatch) {
            issue(ug, pfg, plg, q0, a.m[0].out, vg);
            add(pfg, plg, q0, vg, g);
        }
    if (pfu != plu)
        for (int q0 = pfu + kBatch; q0 <= plu; q0 += kBatch) {
            issue(uu, pfu, plu, q0, a.m[1].out, vu);
            add(pfu, plu, q0, vu, u);
        }
    float *o = a.m[0].out + (int64_t)b * rows + row0;
    const float4 y = make_float4(kore_swiglu(g.x, u.x), kore_swiglu(g.y, u.y), kore_swiglu(g.z, u.z),
                                 kore_swiglu(g.w, u.w));
    if (whole && !((uintptr_t)o & 15)) {
        *(float4 *)o = y;
        return;
    }
    const float ys[4] = {y.x, y.y, y.z, y.w};
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (row0 + k < rows) o[k] = ys[k];
}

constexpr size_t lds_bytes(int nbk) { return (size_t)16 * nbk * kXStride * sizeof(float); }

// Dynamic LDS above 64 KiB (64 activations: 66,560 bytes) needs the kernel's
// limit raised once; gfx950 has 160 KiB per CU.  The same call records how many
// workgroups of the kernel fit on a CU (LDS and registers).
template <int NB, bool Q6>
hipError_t prepare_nb(int *per_cu) {
    static std::once_flag once;
    static hipError_t err = hipSuccess;
    static int occ = 1;
    std::call_once(once, [&] {
        err = hipFuncSetAttribute((const void *)gemm_kernel<NB, Q6>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)lds_bytes(NB));
        if (err == hipSuccess)
            err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, gemm_kernel<NB, Q6>, kThreads, lds_bytes(NB));
        occ = std::max(1, std::min(4, occ));
    });
    *per_cu = occ;
    return err;
}

template <bool Q6>
hipError_t prepare_t(int B, int *per_cu) {
    switch ((B + 15) / 16) {
        case 1: return prepare_nb<1, Q6>(per_cu);
        case 2: return prepare_nb<2, Q6>(per_cu);
        case 3: return prepare_nb<3, Q6>(per_cu);
        default: return prepare_nb<4, Q6>(per_cu);
    }
}

template <int NB, bool Q6>
hipError_t launch_nb(const GemmArgs &a, hipStream_t s) {
    int occ = 0;
    if (hipError_t e = prepare_nb<NB, Q6>(&occ)) return e;
    hipLaunchKernelGGL((gemm_kernel<NB, Q6>), dim3(a.workers), dim3(kThreads), lds_bytes(NB), s, a);
    if (hipError_t e = hipGetLastError()) return e;
    // every run a whole number of tiles: nothing split
    const int64_t T = (int64_t)a.tiles * a.nblk;
    if (T % a.workers == 0 && (T / a.workers) % a.nblk == 0) return hipSuccess;
    hipLaunchKernelGGL((gemm_fixup_kernel<NB>), dim3(a.tiles), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

template <bool Q6>
hipError_t launch_t(const GemmArgs &a, hipStream_t s) {
    switch ((a.B + 15) / 16) {
        case 1: return launch_nb<1, Q6>(a, s);
        case 2: return launch_nb<2, Q6>(a, s);
        case 3: return launch_nb<3, Q6>(a, s);
        default: return launch_nb<4, Q6>(a, s);
    }
}

}  // namespace

int gemm_max_workers(int num_cu) { return 4 * num_cu; }

bool gemm_fp16() {
    static const bool fp16 = [] {
        const char *e = std::getenv("KORE_GEMM");
        return !(e && std::strcmp(e, "fp32") == 0);
    }();
    return fp16;
}

int gemm_rows_per_tile() { return gemm_fp16() ? kG16Rows : kGemmRowsPerTile; }

int gemm_halves(int tiles, int nblk, int B, int num_cu) {
    return gemm_fp16() && B > 32 && (int64_t)tiles * nblk < 2LL * std::max(num_cu, 1) ? 2 : 1;
}

int gemm_workers(int tiles, int nblk, int B, bool has_q6k, int num_cu) {
    int occ = 1;                               // fp16 path: one workgroup per CU (LDS)
    if (!gemm_fp16() && (has_q6k ? prepare_t<true>(B, &occ) : prepare_t<false>(B, &occ)) != hipSuccess) occ = 1;
    const int64_t T = (int64_t)tiles * nblk;
    int64_t p = std::min<int64_t>((int64_t)occ * num_cu, std::max<int64_t>(1, T / 2));
    if (p >= 8) p -= p % 8;
    return (int)p;
}

namespace {

template <int NT, bool Q6>
hipError_t launch16_nt(const GemmArgs &a, hipStream_t s) {
    if (!a.presplit) {
        // every activation the units read: 32 per tile of activations, both halves in halves mode
        hipLaunchKernelGGL(gemm16_prep_kernel, dim3(32 * NT * a.halves), dim3(kPrepThreads), 0, s, a.x, a.x16, a.B,
                           a.nblk);
        if (hipError_t e = hipGetLastError()) return e;
    }
    hipLaunchKernelGGL((gemm16_kernel<NT, Q6>), dim3(a.workers), dim3(kG16Threads), 0, s, a);
    if (hipError_t e = hipGetLastError()) return e;
    if (a.glu) {   // every gate tile: its SwiGLU is written by the pair's fix-up
        hipLaunchKernelGGL(gemm16_glu_fixup_kernel, dim3(a.m[1].tile0 * a.halves, kG16SlotFloats / 1024),
                           dim3(kThreads), 0, s, a);
        return hipGetLastError();
    }
    const int64_t T = (int64_t)a.tiles * a.halves * a.nblk;
    if (T % a.workers == 0 && (T / a.workers) % a.nblk == 0) return hipSuccess;
    // 16 slices of 1024 partial floats (the slices of a second tile of
    // activations return at once when NT = 1)
    hipLaunchKernelGGL(gemm16_fixup_kernel, dim3(a.tiles * a.halves, kG16SlotFloats / 1024), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

template <bool Q6>
hipError_t launch16(const GemmArgs &a, hipStream_t s) {
    return a.B > 32 && a.halves == 1 ? launch16_nt<2, Q6>(a, s) : launch16_nt<1, Q6>(a, s);
}

}  // namespace

hipError_t launch_gemm(GemmArgs a, hipStream_t s) {
    if (a.n_mat < 1 || a.n_mat > kMaxGroup || a.nblk <= 0 || a.B <= 0 || a.B > kGemmMaxB) return hipErrorInvalidValue;
    if (a.workers < 1 || !a.partials) return hipErrorInvalidValue;
    const bool fp16 = gemm_fp16();
    if (fp16 && (!a.x16 || a.nblk > kMaxBlocks)) return hipErrorInvalidValue;   // the pre-pass holds 128 blocks
    if (a.presplit && !fp16) return hipErrorInvalidValue;
    const int rpt = gemm_rows_per_tile();
    int tiles = 0;
    for (int k = 0; k < a.n_mat; ++k) {
        const GemmMat &m = a.m[k];
        if (m.rows <= 0 || !m.w || !m.out || (m.type != kQ4K && m.type != kQ6K) || (m.type == kQ6K && !m.wd))
            return hipErrorInvalidValue;
        a.m[k].tile0 = tiles;
        tiles += (m.rows + rpt - 1) / rpt;
    }
    if (a.halves != 1 && !(a.halves == 2 && fp16)) return hipErrorInvalidValue;
    if (a.glu && (!fp16 || a.n_mat != 2 || a.m[0].rows != a.m[1].rows || a.m[0].bias ||
                  a.m[1].bias || a.m[0].accumulate || a.m[1].accumulate))
        return hipErrorInvalidValue;
    if (tiles != a.tiles || (int64_t)tiles * a.halves * a.nblk < a.workers) return hipErrorInvalidValue;
    bool q6 = false;
    for (int k = 0; k < a.n_mat; ++k) q6 |= a.m[k].type == kQ6K;
    if (fp16) return q6 ? launch16<true>(a, s) : launch16<false>(a, s);
    return q6 ? launch_t<true>(a, s) : launch_t<false>(a, s);
}

}  // namespace kore_qmv_gpu
