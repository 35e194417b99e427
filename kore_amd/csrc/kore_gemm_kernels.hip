// kore_gemm_kernels.hip - gfx950 kernel of kore's batched prefill matmul
// (matmul_batch_float, kore.cpp:783-845): out[b][r] = row r of the
// dequantised Q4_K / Q6_K weights . x[b] for B <= 64 activations at once, for
// up to four matrices that share x in one launch.
//
// fp32 MFMA (v_mfma_f32_16x16x4f32) on weights dequantised in registers: a
// wave owns 16 rows of a 64-row tile and up to 64 activations (NB blocks of
// 16); lane l supplies row l % 16 and, of every 256-column block, the 64
// columns of group l / 16 (the order of the K sum inside a block is permuted
// so that each lane dequantises contiguous bytes; the sum is the same up to
// fp32 rounding).  The activations of a block are staged in LDS, each of them
// a 260-float row so the 16-byte reads of 16 consecutive activations hit
// different banks.  The next block's activations and weights are loaded into
// registers while the current block's MFMAs run.
//
// Work split: stream-K.  The iteration space (tile, block) of all matrices is
// cut into `workers` contiguous runs of equal length, one per workgroup, so
// every CU gets the same number of block iterations whatever the shapes.  A
// tile split between workers leaves one partial sum per worker in a slot of
// the workspace (slot 2p for worker p's first tile, 2p + 1 for its last), and
// a second launch adds each split tile's slots in worker order.  (Finishing
// split tiles inside the first launch would need device-scope fences, which
// write back and invalidate the XCD's L2 each time and cost far more than the
// second launch.)
//
// kore sums each output in one fused multiply-add chain over the columns; this
// sums in MFMA blocks, so results agree with kore's to fp32 rounding (kore's
// own tolerance, max|d| <= 1e-4 max|ref| + 1e-6, kore_kernels.cpp:742), not
// bit for bit.  For one device, shape and B the result is deterministic.
#include "kore_qmv_kernels.h"

#include <algorithm>
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

int gemm_workers(int tiles, int nblk, int B, bool has_q6k, int num_cu) {
    int occ = 1;
    if ((has_q6k ? prepare_t<true>(B, &occ) : prepare_t<false>(B, &occ)) != hipSuccess) occ = 1;
    const int64_t T = (int64_t)tiles * nblk;
    int64_t p = std::min<int64_t>((int64_t)occ * num_cu, std::max<int64_t>(1, T / 2));
    if (p >= 8) p -= p % 8;
    return (int)p;
}

hipError_t launch_gemm(GemmArgs a, hipStream_t s) {
    if (a.n_mat < 1 || a.n_mat > kMaxGroup || a.nblk <= 0 || a.B <= 0 || a.B > kGemmMaxB) return hipErrorInvalidValue;
    if (a.workers < 1 || !a.partials) return hipErrorInvalidValue;
    int tiles = 0;
    for (int k = 0; k < a.n_mat; ++k) {
        const GemmMat &m = a.m[k];
        if (m.rows <= 0 || !m.w || !m.out || (m.type != kQ4K && m.type != kQ6K) || (m.type == kQ6K && !m.wd))
            return hipErrorInvalidValue;
        a.m[k].tile0 = tiles;
        tiles += (m.rows + kGemmRowsPerTile - 1) / kGemmRowsPerTile;
    }
    if (tiles != a.tiles || (int64_t)tiles * a.nblk < a.workers) return hipErrorInvalidValue;
    bool q6 = false;
    for (int k = 0; k < a.n_mat; ++k) q6 |= a.m[k].type == kQ6K;
    return q6 ? launch_t<true>(a, s) : launch_t<false>(a, s);
}

}  // namespace kore_qmv_gpu
