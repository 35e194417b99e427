// kore_gemm_kernels.hip - gfx950 kernels of kore's batched prefill matmul
// (matmul_batch_float, kore.cpp:783-845): out[b][r] = row r of the
// dequantised Q4_K / Q6_K weights . x[b] for B <= 64 activations at once.
//
// fp32 MFMA (v_mfma_f32_16x16x4f32) on weights dequantised in registers: a
// wave owns 16 rows and up to 64 activations (NB blocks of 16); lane l
// supplies row l % 16 and, of every 256-column block, the 64 columns of group
// l / 16 (the order of the K sum inside a block is permuted so that each lane
// dequantises contiguous bytes; the sum is the same up to fp32 rounding).  The
// activations of a block are staged in LDS, each of them a 260-float row so
// the 16-byte reads of 16 consecutive activations hit different banks.  Row-
// poor matrices split their blocks over several workgroups (split-K) and a
// second kernel adds the partial sums in split order.  kore sums each output
// in one fused multiply-add chain over the columns; this sums in MFMA blocks,
// so results agree with kore's to fp32 rounding (kore's own tolerance,
// max|d| <= 1e-4 max|ref| + 1e-6, kore_kernels.cpp:742), not bit for bit.
#include "kore_qmv_kernels.h"

#include <mutex>

namespace kore_qmv_gpu {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kRowsPerWg = 64;          // 16 per wave
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

// One lane's weights of one block: Q4_K group kk (32 nibble bytes + header);
// Q6_K values 64 kk .. 64 kk + 63 (64 ql bytes of half kk / 2, 32 qh bytes,
// the four scales of the lane, d).
struct Q4G { uint4 hdr, qa, qb; };
struct Q6G { uint4 l0, l1, l2, l3, h0, h1; uint32_t sc, d; };

__device__ __forceinline__ Q4G load4(const uint8_t *b, int kk) {
    Q4G g;
    g.hdr = *(const uint4 *)b;
    g.qa = *(const uint4 *)(b + 16 + 32 * kk);
    g.qb = *(const uint4 *)(b + 32 + 32 * kk);
    return g;
}

__device__ __forceinline__ Q6G load6(const uint8_t *b, const uint16_t *dp, int kk) {
    const int h = kk >> 1;
    Q6G g;
    g.l0 = *(const uint4 *)(b + 64 * h);
    g.l1 = *(const uint4 *)(b + 64 * h + 16);
    g.l2 = *(const uint4 *)(b + 64 * h + 32);
    g.l3 = *(const uint4 *)(b + 64 * h + 48);
    g.h0 = *(const uint4 *)(b + 128 + 32 * h);
    g.h1 = *(const uint4 *)(b + 128 + 32 * h + 16);
    g.sc = *(const uint32_t *)(b + 192 + 4 * kk);   // sc[8h + 4(kk&1) + 0..3]
    g.d = *dp;
    return g;
}

template <int TYPE>
using Group = std::conditional_t<TYPE == kQ4K, Q4G, Q6G>;

template <int TYPE, int NB>
__global__ __launch_bounds__(kThreads) void gemm_kernel(GemmArgs a) {
    extern __shared__ __align__(16) float xs[];      // [16 NB][kXStride]
    constexpr int BB = TYPE == kQ4K ? kQ4Bytes : kQ6Body;
    const int t = threadIdx.x, wave = t >> 6, l = t & 63;
    const int i = l & 15, kk = l >> 4;
    const int tile = blockIdx.x / a.splits, split = blockIdx.x % a.splits;
    const int kb0 = (int)((int64_t)a.nblk * split / a.splits);
    const int kb1 = (int)((int64_t)a.nblk * (split + 1) / a.splits);
    const int row = min(tile * kRowsPerWg + 16 * wave + i, a.rows - 1);
    const int64_t cols = (int64_t)a.nblk * 256;
    const uint8_t *wrow = a.w + (int64_t)row * a.nblk * BB;
    const uint16_t *drow = TYPE == kQ6K ? a.wd + (int64_t)row * a.nblk : nullptr;

    auto load = [&](int blk) -> Group<TYPE> {
        if constexpr (TYPE == kQ4K) return load4(wrow + (int64_t)blk * BB, kk);
        else return load6(wrow + (int64_t)blk * BB, drow + blk, kk);
    };

    floatx4 acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = floatx4{0.f, 0.f, 0.f, 0.f};

    Group<TYPE> cur = load(min(kb0, a.nblk - 1));
    for (int blk = kb0; blk < kb1; ++blk) {
        __syncthreads();                                 // the previous block's reads of xs are done
        for (int c = t; c < 16 * NB * 64; c += kThreads) {
            const int b = c >> 6, q = c & 63;
            if (b < a.B)
                *(float4 *)&xs[b * kXStride + 4 * q] = *(const float4 *)(a.x + b * cols + 256 * (int64_t)blk + 4 * q);
        }
        const Group<TYPE> g = cur;
        cur = load(min(blk + 1, kb1 - 1));               // the next block's weights, while this one runs
        __syncthreads();

        if constexpr (TYPE == kQ4K) {
            // kore's dequant_block_q4_K (kore.cpp:337-353): d1 = d*sc, m1 = dmin*min, value = d1*q - m1
            const float d = f16f(g.hdr.x & 0xFFFFu), dmin = f16f(g.hdr.x >> 16);
            const float d1 = d * (float)q4s(g.hdr, 2 * kk), m1 = dmin * (float)q4m(g.hdr, 2 * kk);
            const float d2 = d * (float)q4s(g.hdr, 2 * kk + 1), m2 = dmin * (float)q4m(g.hdr, 2 * kk + 1);
#pragma unroll
            for (int t4 = 0; t4 < 16; ++t4) {
                float4 bx[NB];
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) bx[nb] = *(const float4 *)&xs[(16 * nb + i) * kXStride + 64 * kk + 4 * t4];
#pragma unroll
                for (int tt = 0; tt < 4; ++tt) {
                    const int tk = 4 * t4 + tt;              // column 64 kk + tk of the block
                    const int byte = tk & 31;
                    const uint32_t w = word(g.qa, g.qb, byte >> 2);
                    const uint32_t q = (w >> (8 * (byte & 3) + (tk >= 32 ? 4 : 0))) & 15u;
                    const float av = tk < 32 ? d1 * (float)q - m1 : d2 * (float)q - m2;
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb) {
                        const float bv = tt == 0 ? bx[nb].x : tt == 1 ? bx[nb].y : tt == 2 ? bx[nb].z : bx[nb].w;
                        acc[nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[nb], 0, 0, 0);
                    }
                }
            }
        } else {
            // kore's dequant_block_q6_K (kore.cpp:359-381): value = (d * sc) * (q6 - 32);
            // lane kk: h = kk / 2, groups k = 2 (kk % 2) + tk / 32, low or high nibble by kk % 2
            const float d = f16f(g.d);
            const int kh = kk & 1;
            float ds[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) ds[e] = d * (float)(int)(int8_t)((g.sc >> (8 * e)) & 0xFF);
#pragma unroll
            for (int t4 = 0; t4 < 16; ++t4) {
                float4 bx[NB];
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) bx[nb] = *(const float4 *)&xs[(16 * nb + i) * kXStride + 64 * kk + 4 * t4];
#pragma unroll
                for (int tt = 0; tt < 4; ++tt) {
                    const int tk = 4 * t4 + tt, l32 = tk & 31, kt = tk >> 5;
                    const uint4 &lv = tk < 16 ? g.l0 : tk < 32 ? g.l1 : tk < 48 ? g.l2 : g.l3;
                    const int m = (tk >> 2) & 3;
                    const uint32_t lw = m == 0 ? lv.x : m == 1 ? lv.y : m == 2 ? lv.z : lv.w;
                    const uint32_t hw = word(g.h0, g.h1, l32 >> 2);
                    const uint32_t nib = (lw >> (8 * (tk & 3) + 4 * kh)) & 15u;
                    const uint32_t hb = (hw >> (8 * (l32 & 3) + 4 * kh + 2 * kt)) & 3u;
                    const float av = ds[2 * kt + (l32 >> 4)] * (float)((int)(nib | (hb << 4)) - 32);
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb) {
                        const float bv = tt == 0 ? bx[nb].x : tt == 1 ? bx[nb].y : tt == 2 ? bx[nb].z : bx[nb].w;
                        acc[nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[nb], 0, 0, 0);
                    }
                }
            }
        }
    }

    // D block: lane l holds rows 4 (l / 16) + v, activation l % 16 of each 16-block
    float *out = a.out + (int64_t)split * a.B * a.rows;
    const int r0 = tile * kRowsPerWg + 16 * wave + 4 * kk;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const int b = 16 * nb + i;
        if (b >= a.B) continue;
#pragma unroll
        for (int v = 0; v < 4; ++v)
            if (r0 + v < a.rows) out[(int64_t)b * a.rows + r0 + v] = acc[nb][v];
    }
}

// out[e] = sum over s of part[s][e], s in order.
__global__ __launch_bounds__(kThreads) void gemm_reduce_kernel(const float *__restrict__ part, int splits,
                                                               int64_t n, float *__restrict__ out) {
    const int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (e >= n) return;
    float s = part[e];
    for (int k = 1; k < splits; ++k) s += part[(int64_t)k * n + e];
    out[e] = s;
}

// Dynamic LDS above 64 KiB (64 activations: 66,560 bytes) needs the kernel's
// limit raised once; gfx950 has 160 KiB per CU.
template <int TYPE, int NB>
hipError_t launch_nb(const GemmArgs &a, int grid, hipStream_t s) {
    const size_t lds = (size_t)16 * NB * kXStride * sizeof(float);
    static std::once_flag once;
    static hipError_t attr = hipSuccess;
    std::call_once(once, [&] {
        attr = hipFuncSetAttribute((const void *)gemm_kernel<TYPE, NB>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                   (int)lds);
    });
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((gemm_kernel<TYPE, NB>), dim3(grid), dim3(kThreads), lds, s, a);
    return hipGetLastError();
}

template <int TYPE>
hipError_t launch_t(const GemmArgs &a, int grid, hipStream_t s) {
    switch ((a.B + 15) / 16) {
        case 1: return launch_nb<TYPE, 1>(a, grid, s);
        case 2: return launch_nb<TYPE, 2>(a, grid, s);
        case 3: return launch_nb<TYPE, 3>(a, grid, s);
        default: return launch_nb<TYPE, 4>(a, grid, s);
    }
}

}  // namespace

int gemm_splits(int rows, int nblk, int num_cu) {
    const int tiles = (rows + kRowsPerWg - 1) / kRowsPerWg;
    int s = 1;
    // two workgroups per CU, each split at least two blocks long
    while (tiles * s * 2 < 2 * num_cu && nblk / (2 * s) >= 2) s *= 2;
    return s;
}

hipError_t launch_gemm(GemmArgs a, float *out, float *partials, hipStream_t s) {
    if (a.rows <= 0 || a.nblk <= 0 || a.B <= 0 || a.B > kGemmMaxB || a.splits <= 0) return hipErrorInvalidValue;
    if (a.type != kQ4K && a.type != kQ6K) return hipErrorInvalidValue;
    if (a.splits > 1 && !partials) return hipErrorInvalidValue;
    const int tiles = (a.rows + kRowsPerWg - 1) / kRowsPerWg;
    const int64_t grid = (int64_t)tiles * a.splits;
    if (grid > INT32_MAX) return hipErrorInvalidValue;
    a.out = a.splits > 1 ? partials : out;
    hipError_t e = a.type == kQ4K ? launch_t<kQ4K>(a, (int)grid, s) : launch_t<kQ6K>(a, (int)grid, s);
    if (e != hipSuccess || a.splits == 1) return e;
    const int64_t n = (int64_t)a.B * a.rows;
    hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)((n + kThreads - 1) / kThreads)), dim3(kThreads), 0, s,
                       (const float *)partials, a.splits, n, out);
    return hipGetLastError();
}

}  // namespace kore_qmv_gpu
