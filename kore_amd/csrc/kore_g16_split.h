// kore_g16_split.h - writing the fp16 batched matmul's split activations
// (device code shared by gemm16_prep_kernel and the rmsnorm that writes the
// split itself).  Internal to libkore_qmv.so.
//
// Per 256-column block the split of up to 64 activations takes kG16BlockBytes:
// hi [64][32 chunks of 8 fp16] (chunk c of activation b at position c ^ (b &
// 15), so that 16 activations' 16-byte reads hit different banks), lo (same
// layout), the eight sub-block sums (hi, lo fp16) and 1 / s per activation.
// Column 4 i .. 4 i + 3 of a block (float4 group i) is in chunk c = 2 (q & 15)
// + (q >> 4), q = 8 (i / 16) + i % 8, its first (i % 16 < 8) or second half:
// the MFMA's k order over the Q4_K nibble dwords.
#pragma once

#include "kore_qmv_kernels.h"

namespace kore_qmv_gpu {

// x of another lane of the same 16-lane row: lane i ^ 1 (0xB1), i ^ 2 (0x4E),
// 7 - i within its 8 lanes (0x141, row_half_mirror), (i - 4) / (i - 8) mod 16
// (0x124 / 0x128, row rotations).
template <int CTRL>
__device__ __forceinline__ float g16_dppf(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// The maximum of x over the wave, in every lane: the 16-lane rows by DPP, then
// the four rows by lane swaps (v_permlane16_swap / v_permlane32_swap with x as
// both operands return the two rows of each pair, the two halves, in their
// results).
__device__ __forceinline__ float g16_wave_max(float x) {
    x = fmaxf(x, g16_dppf<0xB1>(x));
    x = fmaxf(x, g16_dppf<0x4E>(x));
    x = fmaxf(x, g16_dppf<0x124>(x));
    x = fmaxf(x, g16_dppf<0x128>(x));
    const uint32_t u = __float_as_uint(x);
    const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const uint32_t a0 = a[0], a1 = a[1];
    x = fmaxf(__uint_as_float(a0), __uint_as_float(a1));
    const uint32_t w = __float_as_uint(x);
    const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
    const uint32_t b0 = b[0], b1 = b[1];
    return fmaxf(__uint_as_float(b0), __uint_as_float(b1));
}

// The row's power of two s = s1 * s2 (max |y s| < 2^10 for amax = max |y|;
// callers scale as (y * s1) * s2, both factors powers of two, so the product is
// exact) and 1 / s.  s reaches 2^149 for rows whose maximum is a subnormal
// float (s1 alone would overflow above 2^127; s2 is 1 for every row whose
// maximum is at least 2^-117); 1 / s stays a float down to 2^-149.  A row with
// an infinite or NaN value takes s = 2^10: its products are non-finite anyway.
__device__ __forceinline__ void g16_split_scale(float amax, float &s1, float &s2, float &inv) {
    int e = 0;
    if (amax <= 3.40282347e38f) (void)frexpf(amax, &e);   // amax < 2^e (0 for amax = 0)
    e = max(e, -139);
    const int sh = 10 - e, sh1 = min(sh, 127);
    s1 = ldexpf(1.f, sh1);
    s2 = ldexpf(1.f, sh - sh1);
    inv = ldexpf(1.f, e - 10);
}

// Float4 group `lane` of block `blk` of activation b: ys = its four values
// times s.  The hi and lo fp16 parts in one 8-byte store each, the sub-block
// sum (the four values, then lanes ^1, ^2, ^4: 32 columns) and 1 / s.  Every
// lane of the wave takes part (lane sums); lane = the wave's lane index.
__device__ __forceinline__ void g16_split_group(uint8_t *__restrict__ x16, int b, int blk, int lane,
                                                const float ys[4], float inv) {
    typedef _Float16 half4v __attribute__((ext_vector_type(4)));
    const int iw = lane & 15, low = iw < 8, tq = low ? iw : iw - 8;
    const int q = 8 * (lane >> 4) + tq, c = 2 * (q & 15) + (q >> 4);
    const int off = b * 512 + ((c ^ (b & 15)) * 16) + (low ? 0 : 8);
    half4v h, l;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        h[k] = (_Float16)ys[k];
        l[k] = (_Float16)(ys[k] - (float)h[k]);
    }
    uint8_t *blkp = x16 + (int64_t)blk * kG16BlockBytes;
    *(uint2 *)(blkp + off) = __builtin_bit_cast(uint2, h);
    *(uint2 *)(blkp + kG16Lo + off) = __builtin_bit_cast(uint2, l);
    // lanes ^ 1, ^ 2, then the other quad of the 8 (every lane of a quad holds
    // the same sum after the first two steps, so the mirror lane's is its quad's)
    float S = (ys[0] + ys[1]) + (ys[2] + ys[3]);
    S += g16_dppf<0xB1>(S);
    S += g16_dppf<0x4E>(S);
    S += g16_dppf<0x141>(S);
    if ((lane & 7) == 0) {
        const _Float16 sh = (_Float16)S, sl = (_Float16)(S - (float)sh);
        _Float16 *sx = (_Float16 *)(blkp + kG16Sx + b * 32);
        sx[lane >> 3] = sh;
        sx[8 + (lane >> 3)] = sl;
    }
    if (lane == 0) *(float *)(blkp + kG16Inv + b * 4) = inv;
}

}  // namespace kore_qmv_gpu
