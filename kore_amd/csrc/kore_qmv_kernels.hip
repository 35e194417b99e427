// kore_qmv_kernels.hip - gfx950 kernels of kore's quantised matrix-vector
// product: Q8_K activation quantisation and Q4_K / Q6_K x Q8_K row dot
// products (kore.cpp:422-682), bit-identical to kore's scalar and AVX2 code.
//
// The matvec is HBM-bound: every weight byte is read once, the activations
// (at most 128 x 292 bytes) are staged in LDS by every workgroup.  A row's
// work is cut into units (row, 256-value block) and each unit into four
// parts handled by four adjacent lanes.  A part computes exact integer sums
// (v_dot4_i32_i8 over 4 bytes at a time; every partial kore forms in an
// int32 lane is reproduced exactly).  kore's float arithmetic - one fused
// multiply-add per AVX2 lane and block, in block order, then its horizontal
// sums - is a sequential chain per row; the integer results of a step's
// units go through LDS to one wave that advances the chains, so blocks can
// be spread over all lanes without changing a single rounding.
#include "kore_qmv_kernels.h"
#include "kore_g16_split.h"
#include "kore_swiglu.h"

#include <algorithm>
#include <climits>
#include <cstdlib>
#include <type_traits>

namespace kore_qmv_gpu {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float f16_bits(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, 0, false);
}

// Products of a 6- or 8-bit scale and a sum of at most 2^16 in magnitude:
// both fit the 24-bit multiplier (full rate, unlike v_mul_lo_u32).
__device__ __forceinline__ int mul24(int a, int b) { return __mul24(a, b); }

__device__ __forceinline__ int quad_xor1(int v) { return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true); }
__device__ __forceinline__ int quad_xor2(int v) { return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true); }
__device__ __forceinline__ float quad_xor1f(float v) { return __int_as_float(quad_xor1(__float_as_int(v))); }
__device__ __forceinline__ float quad_xor2f(float v) { return __int_as_float(quad_xor2(__float_as_int(v))); }

// ------------------------------------------------------------------ Q8_K

// Row-of-16 DPP moves: lane i of each 16-lane row reads lane i ^ 1, i ^ 2
// (quad permutations) or lane (i - 4) / (i - 8) mod 16 (row rotations).
template <int CTRL>
__device__ __forceinline__ int dpp(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false); }

// What lane m of a 16-lane DPP row holds of a quantised block: its 16 int8
// values (16m .. 16m+15), their sum (bsums[m]) and the block's d.
struct Q8Lane {
    uint4 qs;
    int bsum;
    float d;
};

// ------------------------------------------------------------------ pre-ops

// kore's rmsnorm scale from the sum of squares ss (kore.cpp:1370):
// 1.0f / std::sqrt((float)(ss / n) + eps).  sqrt and the reciprocal are taken
// in double and rounded once to float, which is the correctly rounded float
// result (53 >= 2 * 24 + 2 bits) whatever the compiler does with float sqrt
// and division.
__device__ __forceinline__ float kore_rms_scale(double ss, int n, float eps) {
    const float a = (float)(ss / (double)n) + eps;
    const float r = (float)sqrt((double)a);
    return (float)(1.0 / (double)r);
}

__device__ __forceinline__ void two_sum(double a, double b, double &s, double &e) {
    s = a + b;
    const double bb = s - a;
    e = (a - (s - bb)) + (b - bb);
}

// kore's rmsnorm scale of x[0..n) for a whole workgroup (every thread gets it).
// kore sums (double)x[i] * x[i] in index order in double (kore.cpp:1368-1369);
// here a double-double sum in parallel gives the exact sum S to ~2^-100, and
// every order's double sum of n nonnegative terms lies within gamma(n-1) * S of
// it.  When the float scale is the same at both ends of that interval it is
// kore's (the scale is monotone in ss); otherwise one thread runs kore's loop.
// red: 2 * kThreads / 64 doubles of LDS (at least one).
// The reduction and certification of block_rms_scale from each thread's
// double-double partial sum (hi, lo) of x[t], x[t + kThreads], ...
__device__ float block_rms_scale_from(double hi, double lo, const float *x, int n, float eps, double *red) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    // wave, then the four waves in order: one barrier
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const double ohi = __shfl_xor(hi, off), olo = __shfl_xor(lo, off);
        double s, e;
        two_sum(hi, ohi, s, e);
        hi = s;
        lo = (lo + olo) + e;
    }
    if (lane == 0) {
        red[2 * wave] = hi;
        red[2 * wave + 1] = lo;
    }
    __syncthreads();
    hi = red[0];
    lo = red[1];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) {
        double s, e;
        two_sum(hi, red[2 * w], s, e);
        hi = s;
        lo = (lo + red[2 * w + 1]) + e;
    }
    const double S = hi + lo;
    const double g = (double)(n - 1) * 0x1p-53 / (1.0 - (double)(n - 1) * 0x1p-53);
    const double m = 2.0 * g + 0x1p-50;   // + the double-double and final roundings
    const float lo_s = kore_rms_scale(S * (1.0 - m), n, eps), hi_s = kore_rms_scale(S * (1.0 + m), n, eps);
    __syncthreads();                       // red is reused below and by the caller
    if (__float_as_uint(lo_s) == __float_as_uint(hi_s)) return lo_s;
    if (t == 0) {                          // kore's own loop
        double ss = 0.0;
        for (int i = 0; i < n; ++i) ss += (double)x[i] * x[i];
        red[0] = ss;
    }
    __syncthreads();
    const float sc = kore_rms_scale(red[0], n, eps);
    __syncthreads();
    return sc;
}

// The same scale from each thread's plain double sum ss of its squares (each
// (double)x * x is exact): sums in registers and across the wave by DPP and
// lane swaps, the four waves' sums through LDS in a fixed order, so every
// thread holds the same S.  Any order's double sum of n nonnegative exact
// terms lies within gamma(n-1) * S of the exact sum, this one and kore's
// alike, so kore's sum lies within 2 gamma(n-1) / (1 - gamma(n-1)) of S_gpu;
// the float scale is certified at both ends of twice that interval, and
// otherwise one thread runs kore's loop.  red: kThreads / 64 doubles.
__device__ __forceinline__ double dpp_d(double x, int which) {
    const unsigned long long u = __builtin_bit_cast(unsigned long long, x);
    int lo = (int)(unsigned)u, hi = (int)(unsigned)(u >> 32);
    switch (which) {
        case 0: lo = dpp<0xB1>(lo); hi = dpp<0xB1>(hi); break;     // lane ^ 1
        case 1: lo = dpp<0x4E>(lo); hi = dpp<0x4E>(hi); break;     // lane ^ 2
        case 2: lo = dpp<0x124>(lo); hi = dpp<0x124>(hi); break;   // rotate the 16-lane row by 4
        default: lo = dpp<0x128>(lo); hi = dpp<0x128>(hi); break;  // ... by 8
    }
    return __builtin_bit_cast(double, ((unsigned long long)(unsigned)hi << 32) | (unsigned)lo);
}
__device__ float block_rms_scale_sum(double ss, const float *x, int n, float eps, double *red) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
#pragma unroll
    for (int k = 0; k < 4; ++k) ss += dpp_d(ss, k);
    // the four 16-lane rows: lane l and l ^ 16, then l and l ^ 32
#pragma unroll
    for (int p32 = 0; p32 < 2; ++p32) {
        const unsigned long long u = __builtin_bit_cast(unsigned long long, ss);
        const unsigned lo = (unsigned)u, hi = (unsigned)(u >> 32);
        const auto rl = p32 ? __builtin_amdgcn_permlane32_swap(lo, lo, false, false)
                            : __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
        const auto rh = p32 ? __builtin_amdgcn_permlane32_swap(hi, hi, false, false)
                            : __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
        const unsigned l0 = rl[0], l1 = rl[1], h0 = rh[0], h1 = rh[1];
        ss = __builtin_bit_cast(double, ((unsigned long long)h0 << 32) | l0) +
             __builtin_bit_cast(double, ((unsigned long long)h1 << 32) | l1);
    }
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    double S = red[0];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) S += red[w];
    const double g = (double)(n - 1) * 0x1p-53 / (1.0 - (double)(n - 1) * 0x1p-53);
    const double m = 4.0 * g + 0x1p-50;
    const float lo_s = kore_rms_scale(S * (1.0 - m), n, eps), hi_s = kore_rms_scale(S * (1.0 + m), n, eps);
    // every thread holds the same S, so the branch is uniform; its caller
    // (the fused matvec prologue) writes red again only after its own barrier
    if (__float_as_uint(lo_s) == __float_as_uint(hi_s)) return lo_s;
    __syncthreads();                       // every thread has read red before it is rewritten
    if (t == 0) {                          // kore's own loop
        double sk = 0.0;
        for (int i = 0; i < n; ++i) sk += (double)x[i] * x[i];
        red[0] = sk;
    }
    __syncthreads();
    const float sc = kore_rms_scale(red[0], n, eps);
    __syncthreads();
    return sc;
}

__device__ float block_rms_scale(const float *x, int n, float eps, double *red) {
    // 8 loads at a time issued ahead of the dependent sum chain (clamped
    // indexes: no load waits on a branch); a slot past n adds 0.0, which leaves
    // hi and lo unchanged, so the order is that of one value at a time
    constexpr int kPer = 8;
    double hi = 0.0, lo = 0.0;
    for (int i0 = threadIdx.x; i0 < n; i0 += kPer * kThreads) {
        float v[kPer];
#pragma unroll
        for (int j = 0; j < kPer; ++j) v[j] = x[min(i0 + j * kThreads, n - 1)];
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const float xv = i0 + j * kThreads < n ? v[j] : 0.0f;
            double s, e;
            two_sum(hi, (double)xv * (double)xv, s, e);
            hi = s;
            lo += e;
        }
    }
    return block_rms_scale_from(hi, lo, x, n, eps, red);
}

__device__ __forceinline__ Q8Lane quantize16(const float (&v)[16], int m);

// kore's quantisation of one 256-value block (kore.cpp:422-446) by the 16
// lanes of a DPP row: lane m owns values 16m .. 16m+15 (x 16-byte aligned),
// after the pre-op (rmsnorm with `scale`, or SwiGLU) of the values at xb[i] =
// x[base + i].
__device__ __forceinline__ Q8Lane quantize_lane(const float *xb, int m, const PreOp &pre = PreOp{nullptr, 0.f, nullptr},
                                                float scale = 1.f, int64_t base = 0) {
    float v[16];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float4 f = *(const float4 *)(xb + 16 * m + 4 * k);
        v[4 * k] = f.x;
        v[4 * k + 1] = f.y;
        v[4 * k + 2] = f.z;
        v[4 * k + 3] = f.w;
    }
    if (pre.norm_w) {                      // kore.cpp:1371: x[i] * scale * w[i]
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float4 w = *(const float4 *)(pre.norm_w + base + 16 * m + 4 * k);
            v[4 * k] = (v[4 * k] * scale) * w.x;
            v[4 * k + 1] = (v[4 * k + 1] * scale) * w.y;
            v[4 * k + 2] = (v[4 * k + 2] * scale) * w.z;
            v[4 * k + 3] = (v[4 * k + 3] * scale) * w.w;
        }
    } else if (pre.up) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float4 u = *(const float4 *)(pre.up + base + 16 * m + 4 * k);
            v[4 * k] = kore_swiglu(v[4 * k], u.x);
            v[4 * k + 1] = kore_swiglu(v[4 * k + 1], u.y);
            v[4 * k + 2] = kore_swiglu(v[4 * k + 2], u.z);
            v[4 * k + 3] = kore_swiglu(v[4 * k + 3], u.w);
        }
    }
    return quantize16(v, m);
}

// v_cvt_i32_f32: a NaN converts to 0 (the instruction's own rule; C's
// conversion leaves it undefined)
__device__ __forceinline__ int cvt_i32(float f) {
    int r;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(f));
    return r;
}

// The quantisation proper of quantize_lane: lane m of a DPP row holds values
// 16m .. 16m+15 of the block (after any pre-op) in v.
__device__ __forceinline__ Q8Lane quantize16(const float (&v)[16], int m) {
    // kore keeps the first value of largest magnitude, starting from amax = 0
    // with a strict comparison (kore.cpp:424-428): the largest |x| wins, ties
    // go to the lowest index, NaN and zeros are never chosen.  Here: the
    // largest magnitude over the row (fmaxf passes over a NaN), then each
    // lane's first value of that magnitude as the key 2 index + sign bit,
    // whose minimum over the row names kore's value (its magnitude is amax).
    float amax = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) amax = fmaxf(amax, fabsf(v[e]));
    amax = fmaxf(amax, __int_as_float(dpp<0xB1>(__float_as_int(amax))));
    amax = fmaxf(amax, __int_as_float(dpp<0x4E>(__float_as_int(amax))));
    amax = fmaxf(amax, __int_as_float(dpp<0x124>(__float_as_int(amax))));
    amax = fmaxf(amax, __int_as_float(dpp<0x128>(__float_as_int(amax))));
    int idx = 16;
    float sv = 0.f;
#pragma unroll
    for (int e = 15; e >= 0; --e) {
        const bool hit = fabsf(v[e]) == amax;
        idx = hit ? e : idx;
        sv = hit ? v[e] : sv;
    }
    int key = idx < 16 ? (int)((uint32_t)(32 * m + 2 * idx) | (__float_as_uint(sv) >> 31)) : INT_MAX;
    key = min(key, dpp<0xB1>(key));
    key = min(key, dpp<0x4E>(key));
    key = min(key, dpp<0x124>(key));
    key = min(key, dpp<0x128>(key));
    uint32_t packed[4] = {0, 0, 0, 0};
    int bsum = 0;
    float d = 0.f;
    if (amax != 0.f) {
        const float bval = (key & 1) ? -amax : amax;
        const float iscale = -127.0f / bval;
        if (fabsf(iscale) < INFINITY) {
            // |iscale x| <= 127 (1 + 2^-24)^2 for every |x| <= amax, so the
            // round-half-even integer lies in [-127, 127] (kore's clamp at 127
            // never acts) and its low byte is kore's int8; a NaN x gives 0,
            // as kore's x86 conversion gives INT_MIN, whose low byte is 0
            int q[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) q[e] = cvt_i32(rintf(iscale * v[e]));
#pragma unroll
            for (int k = 0; k < 4; ++k)
                packed[k] = __builtin_amdgcn_perm(__builtin_amdgcn_perm((uint32_t)q[4 * k + 3], (uint32_t)q[4 * k + 2], 0x0c0c0400u),
                                                  __builtin_amdgcn_perm((uint32_t)q[4 * k + 1], (uint32_t)q[4 * k], 0x0c0c0400u),
                                                  0x05040100u);
#pragma unroll
            for (int k = 0; k < 4; ++k) bsum = __builtin_amdgcn_sdot4((int)packed[k], 0x01010101, bsum, false);
        }
        // else iscale is infinite (amax < 127 / FLT_MAX): every product is
        // infinite or NaN, kore's conversion gives INT_MIN and the int8 0
        d = 1.0f / iscale;
    }
    return Q8Lane{make_uint4(packed[0], packed[1], packed[2], packed[3]), bsum, d};
}

// Activations in LDS, laid out for 16-byte reads: the 256 int8 values of
// block i at i * 272 (a 16-byte pad between blocks spreads them over the
// banks), bsums at nblk * 272 + 32 i, d at nblk * 304 + 4 i.
constexpr int kXsQs = 272;
__host__ __device__ constexpr size_t xs_bytes(int nblk) { return (size_t)nblk * 308; }

struct Q8View {
    const uint8_t *p;
    int nblk;
    __device__ uint4 qs16(int i, int byte) const { return *(const uint4 *)(p + i * kXsQs + byte); }
    __device__ int bsum(int i, int j) const { return *(const int16_t *)(p + nblk * kXsQs + 32 * i + 2 * j); }
    __device__ float d(int i) const { return *(const float *)(p + nblk * 304 + 4 * i); }
};

__device__ __forceinline__ void xs_store(uint8_t *xs, int nblk, int i, int m, const Q8Lane &q) {
    *(uint4 *)(xs + i * kXsQs + 16 * m) = q.qs;
    *(int16_t *)(xs + nblk * kXsQs + 32 * i + 2 * m) = (int16_t)q.bsum;
    if (m == 0) *(float *)(xs + nblk * 304 + 4 * i) = q.d;
}

// Sixteen blocks per workgroup, one per 16-lane row, written as kore's records
// or (IMAGE) in the matvec's LDS layout, which workgroups then copy verbatim.
template <bool IMAGE>
__global__ __launch_bounds__(kThreads) void quantize_q8k_kernel(const float *__restrict__ x,
                                                                uint8_t *__restrict__ xq, int64_t nblocks,
                                                                PreOp pre) {
    __shared__ double red[2 * kThreads];
    // rmsnorm needs the whole vector's scale: every workgroup computes it
    const float scale = pre.norm_w ? block_rms_scale(x, (int)(nblocks * 256), pre.norm_eps, red) : 1.f;
    const int64_t blk = (int64_t)blockIdx.x * (kThreads / 16) + (threadIdx.x >> 4);
    if (blk >= nblocks) return;
    const int m = threadIdx.x & 15;
    const Q8Lane q = quantize_lane(x + blk * 256, m, pre, scale, blk * 256);
    if constexpr (IMAGE) {
        xs_store(xq, (int)nblocks, (int)blk, m, q);
        return;
    }
    uint8_t *rec = xq + blk * kQ8Bytes;
    uint32_t *qw = (uint32_t *)(rec + 4 + 16 * m);
    qw[0] = q.qs.x;
    qw[1] = q.qs.y;
    qw[2] = q.qs.z;
    qw[3] = q.qs.w;
    *(int16_t *)(rec + 260 + 2 * m) = (int16_t)q.bsum;
    if (m == 0) *(float *)rec = q.d;
}

// kore's SwiGLU (kore.cpp:1465-1468) then quantize_row_q8_K of the product:
// one block per workgroup, one value per thread (its exp and division in
// double are the long part, so they are spread over 256 lanes), then the 16
// lanes of the first DPP row quantise the block from LDS.  Bit-identical to
// quantize_q8k_kernel with the SwiGLU pre-op.
template <bool IMAGE>
__global__ __launch_bounds__(kThreads) void swiglu_quantize_kernel(const float *__restrict__ g,
                                                                   const float *__restrict__ u,
                                                                   uint8_t *__restrict__ xq, int64_t nblocks) {
    __shared__ __align__(16) float sv[256];
    const int64_t blk = blockIdx.x;
    const int t = threadIdx.x;
    sv[t] = kore_swiglu(g[blk * 256 + t], u[blk * 256 + t]);
    __syncthreads();
    if (t >= 16) return;
    float v[16];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float4 f = *(const float4 *)&sv[16 * t + 4 * k];
        v[4 * k] = f.x;
        v[4 * k + 1] = f.y;
        v[4 * k + 2] = f.z;
        v[4 * k + 3] = f.w;
    }
    const Q8Lane q = quantize16(v, t);
    if constexpr (IMAGE) {
        xs_store(xq, (int)nblocks, (int)blk, t, q);
        return;
    }
    uint8_t *rec = xq + blk * kQ8Bytes;
    uint32_t *qw = (uint32_t *)(rec + 4 + 16 * t);
    qw[0] = q.qs.x;
    qw[1] = q.qs.y;
    qw[2] = q.qs.z;
    qw[3] = q.qs.w;
    *(int16_t *)(rec + 260 + 2 * t) = (int16_t)q.bsum;
    if (t == 0) *(float *)rec = q.d;
}

// ------------------------------------------------------------------ units

// Raw bytes of one unit part: whole 16-byte chunks.
//   Q4_K part j: the header (d, dmin, 12 scale bytes) and nibble chunks j and
//   j + 4 of the block, i.e. groups c = j/2 and 2 + j/2 (32 bytes each), half
//   j % 2 of each: the bytes of kore's AVX2 lanes 4(j%2) .. 4(j%2)+3.
//   Q6_K part j (g = j % 2, kp = j / 2): the ql chunks of groups (h, kp) for
//   h = 0, 1, lanes 4g .. 4g+3 (their high nibbles are groups (h, kp+2)), the
//   matching qh chunks, the 16 scales and the block's f16 d.
struct Q4Raw { uint4 hdr, a, b; };
struct Q6Raw { uint4 a0, a1, h0, h1, sc; uint32_t d; };

__device__ __forceinline__ Q4Raw load_q4(const uint8_t *b, int j) {
    Q4Raw r;
    r.hdr = *(const uint4 *)b;
    r.a = *(const uint4 *)(b + 16 + 16 * j);
    r.b = *(const uint4 *)(b + 80 + 16 * j);
    return r;
}

__device__ __forceinline__ Q6Raw load_q6(const uint8_t *b, const uint16_t *dp, int j) {
    const int q = 16 * (2 * (j >> 1) + (j & 1)), qh = 16 * (j & 1);
    Q6Raw r;
    r.a0 = *(const uint4 *)(b + q);
    r.a1 = *(const uint4 *)(b + 64 + q);
    r.h0 = *(const uint4 *)(b + 128 + qh);
    r.h1 = *(const uint4 *)(b + 160 + qh);
    r.sc = *(const uint4 *)(b + 192);
    r.d = *dp;
    return r;
}

// Per-part record handed to the chain lanes (16 bytes).
//   AVX2 Q4_K: s[k0], s[k0+1] (the part's two AVX2 lanes), min product of
//              lane j, then d (j even) or dmin (j odd)
//   AVX2 Q6_K: s[k0], s[k0+1], the block's bias sum, d
//   scalar:    isum, imin (Q4_K), dmin bits, d, the same in all four parts
struct Rec { int a, b, c; float x; };

// Q4_K block (kore.cpp:324-326): 6-bit scale / min of sub-block j from the
// 12 packed bytes (kore.cpp:327-335); j may differ between lanes: both forms,
// then a select (no branch).
__device__ __forceinline__ int q4_scale(const uint4 &h, int j) {
    const int s = 8 * (j & 3);
    const int lo = (h.y >> s) & 63;
    const int hi = ((h.w >> s) & 0x0F) | (((h.y >> (s + 6)) & 3) << 4);
    return j < 4 ? lo : hi;
}
__device__ __forceinline__ int q4_min(const uint4 &h, int j) {
    const int s = 8 * (j & 3);
    const int lo = (h.z >> s) & 63;
    const int hi = ((h.w >> (s + 4)) & 0x0F) | (((h.z >> (s + 6)) & 3) << 4);
    return j < 4 ? lo : hi;
}

__device__ __forceinline__ uint32_t w4(const uint4 &v, int k) {
    return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w;
}

// The two AVX2 lanes part j keeps: its four lane sums S cover the groups it
// loaded, part j ^ 2 holds the other groups of the same four lanes; one DPP
// exchange gives part j lanes 2 sel, 2 sel + 1 of its four (sel = j / 2).
__device__ __forceinline__ void own_lanes(const int S[4], int sel, int &s0, int &s1) {
    const int give0 = sel ? S[0] : S[2], give1 = sel ? S[1] : S[3];
    const int keep0 = sel ? S[2] : S[0], keep1 = sel ? S[3] : S[1];
    s0 = keep0 + quad_xor2(give0);
    s1 = keep1 + quad_xor2(give1);
}

// Part j of a Q4_K unit (kore.cpp:535-587): lanes k = 4(j%2) .. +3 over
// groups c = j/2 and 2 + j/2; kept: lanes 4(j%2) + 2(j/2) + {0, 1}.  The
// 4-lane minimum sum: lane j = sub-blocks 2j, 2j+1 (kore.cpp:556-560).
template <bool AVX2>
__device__ __forceinline__ Rec part_q4(const Q4Raw &r, const Q8View &x, int i, int j) {
    const int hh = j & 1, c1 = j >> 1, c2 = c1 + 2;
    const int sl1 = q4_scale(r.hdr, 2 * c1), sh1 = q4_scale(r.hdr, 2 * c1 + 1);
    const int sl2 = q4_scale(r.hdr, 2 * c2), sh2 = q4_scale(r.hdr, 2 * c2 + 1);
    const uint4 lo1 = x.qs16(i, 64 * c1 + 16 * hh), hi1 = x.qs16(i, 64 * c1 + 32 + 16 * hh);
    const uint4 lo2 = x.qs16(i, 64 * c2 + 16 * hh), hi2 = x.qs16(i, 64 * c2 + 32 + 16 * hh);
    int S[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t a = w4(r.a, k), b = w4(r.b, k);
        S[k] = mul24(sl1, dot4(a & 0x0F0F0F0Fu, w4(lo1, k))) + mul24(sh1, dot4((a >> 4) & 0x0F0F0F0Fu, w4(hi1, k))) +
               mul24(sl2, dot4(b & 0x0F0F0F0Fu, w4(lo2, k))) + mul24(sh2, dot4((b >> 4) & 0x0F0F0F0Fu, w4(hi2, k)));
    }
    const int prod = mul24(q4_min(r.hdr, 2 * j), x.bsum(i, 4 * j) + x.bsum(i, 4 * j + 1)) +
                     mul24(q4_min(r.hdr, 2 * j + 1), x.bsum(i, 4 * j + 2) + x.bsum(i, 4 * j + 3));
    const float yd = x.d(i);
    const float d = f16_bits(r.hdr.x & 0xFFFFu) * yd;
    const float dmin = f16_bits(r.hdr.x >> 16) * yd;
    if constexpr (AVX2) {
        int s0, s1;
        own_lanes(S, c1, s0, s1);
        return Rec{s0, s1, prod, (j & 1) ? dmin : d};
    }
    int isum = (S[0] + S[1]) + (S[2] + S[3]), imin = prod;
    isum += quad_xor1(isum);
    isum += quad_xor2(isum);
    imin += quad_xor1(imin);
    imin += quad_xor2(imin);
    return Rec{isum, imin, __float_as_int(dmin), d};
}

// Part j of a Q6_K unit (kore.cpp:591-632): lanes m = 4g .. 4g+3 of groups
// (h, kp) and (h, kp + 2), h = 0, 1 (g = j % 2, kp = j / 2), scale
// sc[8h + 2k + g]; kept: lanes 4g + 2kp + {0, 1}.
template <bool AVX2>
__device__ __forceinline__ Rec part_q6(const Q6Raw &r, const Q8View &x, int i, int j) {
    const int g = j & 1, kp = j >> 1;
    const int sb = 8 * (2 * kp + g);
    // scales of groups (h, k) = (0, kp), (0, kp+2), (1, kp), (1, kp+2)
    const int s0 = (int)(int8_t)((r.sc.x >> sb) & 0xFF), s1 = (int)(int8_t)((r.sc.y >> sb) & 0xFF);
    const int s2 = (int)(int8_t)((r.sc.z >> sb) & 0xFF), s3 = (int)(int8_t)((r.sc.w >> sb) & 0xFF);
    const uint4 q0l = x.qs16(i, 32 * kp + 16 * g), q0h = x.qs16(i, 32 * (kp + 2) + 16 * g);
    const uint4 q1l = x.qs16(i, 128 + 32 * kp + 16 * g), q1h = x.qs16(i, 128 + 32 * (kp + 2) + 16 * g);
    const int shq = 2 * kp;
    int S[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        // two high bits of group k at bit 2k of qh: shifted once, bits 4-5 of
        // (q >> 2kp) << 4 are group kp's, bits 4-5 of q >> 2kp group kp+2's
        const uint32_t a0 = w4(r.a0, k), a1 = w4(r.a1, k);
        const uint32_t qq0 = w4(r.h0, k) >> shq, qq1 = w4(r.h1, k) >> shq;
        const uint32_t u0l = (a0 & 0x0F0F0F0Fu) | ((qq0 << 4) & 0x30303030u);
        const uint32_t u0h = ((a0 >> 4) & 0x0F0F0F0Fu) | (qq0 & 0x30303030u);
        const uint32_t u1l = (a1 & 0x0F0F0F0Fu) | ((qq1 << 4) & 0x30303030u);
        const uint32_t u1h = ((a1 >> 4) & 0x0F0F0F0Fu) | (qq1 & 0x30303030u);
        S[k] = mul24(s0, dot4(u0l, w4(q0l, k))) + mul24(s1, dot4(u0h, w4(q0h, k))) +
               mul24(s2, dot4(u1l, w4(q1l, k))) + mul24(s3, dot4(u1h, w4(q1h, k)));
    }
    // bias sum over the 16 sub-blocks (kore.cpp:605): part j takes 4j .. 4j+3,
    // the scale word j chosen by two selects (a select tree on the lane's j
    // was compiled as branches, each waiting for the loads)
    const uint32_t scw = (j & 2) ? ((j & 1) ? r.sc.w : r.sc.z) : ((j & 1) ? r.sc.y : r.sc.x);
    int ibias = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) ibias += mul24((int)(int8_t)((scw >> (8 * e)) & 0xFF), x.bsum(i, 4 * j + e));
    ibias += quad_xor1(ibias);
    ibias += quad_xor2(ibias);
    const float d = f16_bits(r.d) * x.d(i);
    if constexpr (AVX2) {
        int s0, s1;
        own_lanes(S, kp, s0, s1);
        return Rec{s0, s1, ibias, d};
    }
    // kore's scalar reference sums (q6 - 32) * q8 (kore.cpp:480-506): the same
    // integer as sum(sc * q6 * q8) - 32 * sum(sc * bsums)
    int isum = (S[0] + S[1]) + (S[2] + S[3]);
    isum += quad_xor1(isum);
    isum += quad_xor2(isum);
    return Rec{isum - 32 * ibias, 0, 0, d};
}

// ------------------------------------------------------------------ matvec

// Wave layout: RW rows of one matrix, P = 16 / RW blocks per step, four parts
// per unit.  Lane l: part j = l % 4, row (l / 4) % RW, block phase l / (4 RW).
// A workgroup's four waves take consecutive row groups of a tile (4 RW rows)
// and share only the staged activations; each wave walks its rows' blocks in
// order on its own.  With P = 1 a lane's part feeds its own chain directly;
// with P > 1 the parts of a step go through the wave's LDS records to the
// lanes of phase 0, which advance the chains block by block.  The weight
// loads of the next D steps are in flight while a step is computed, across
// the tiles of the workgroup's run [tile_begin, tile_end).
template <int TYPE, bool AVX2, int RW, bool FUSED, int D, int PIPE>
__device__ __forceinline__ void matvec_body(const MatDesc &md, int tile_begin, int tile_end, const GroupArgs &a,
                                            uint8_t *smem) {
    constexpr int P = 16 / RW;
    constexpr int BB = TYPE == kQ4K ? kQ4Bytes : kQ6Body;
    const int t = threadIdx.x, wave = t >> 6, l = t & 63;
    const int j = l & 3, rho = (l >> 2) % RW, ph = l / (4 * RW);
    Rec *recs = (Rec *)smem + wave * 128;                   // [2][64] per wave
    uint8_t *xs = smem + 2 * kThreads * sizeof(Rec);        // nblk BlockQ8K records

    const int nblk = a.nblk;
    const int nsteps = (nblk + P - 1) / P;
    const int total = (tile_end - tile_begin) * nsteps;
    const int rows = md.rows;
    auto row_of = [&](int tile) { return min((tile * 4 + wave) * RW + rho, rows - 1); };

    using Raw = std::conditional_t<TYPE == kQ4K, Q4Raw, Q6Raw>;
    // load cursor: saturates at the last step, so every load is unconditional
    int lk = 0, lt = tile_begin, ls = 0;
    const uint8_t *lrow = md.w + (int64_t)row_of(lt) * nblk * BB;
    const uint16_t *ldrow = TYPE == kQ6K ? md.wd + (int64_t)row_of(lt) * nblk : nullptr;
    auto load_next = [&]() -> Raw {
        const int i = min(ls * P + ph, nblk - 1);
        Raw r;
        if constexpr (TYPE == kQ4K) r = load_q4(lrow + i * kQ4Bytes, j);
        else r = load_q6(lrow + i * kQ6Body, ldrow + i, j);
        if (lk + 1 < total) {
            ++lk;
            if (++ls == nsteps) {
                ls = 0;
                ++lt;
                lrow = md.w + (int64_t)row_of(lt) * nblk * BB;
                if constexpr (TYPE == kQ6K) ldrow = md.wd + (int64_t)row_of(lt) * nblk;
            }
        }
        return r;
    };

    // the activations; the first D steps' weights are requested as soon as
    // the activations' own loads are issued, so their latency runs under the
    // quantisation (loads complete in order: requested earlier, the
    // activations are waited for without waiting for the weights)
    Raw buf[D];
    if (FUSED && nblk > kThreads / 16) {
        // more blocks than one pass of 16-lane quantisers covers (the host
        // fuses such inputs only when asked to): the scale over the whole
        // vector first, then pass after pass, then the weights
        const PreOp pre{a.norm_w, a.norm_eps, a.up};
        const float scale = a.norm_w ? block_rms_scale(a.x, nblk * 256, a.norm_eps, (double *)smem) : 1.f;
        for (int b = t >> 4; b < nblk; b += kThreads / 16)
            xs_store(xs, nblk, b, t & 15, quantize_lane(a.x + (int64_t)b * 256, t & 15, pre, scale, (int64_t)b * 256));
#pragma unroll
        for (int d = 0; d < D; ++d) buf[d] = load_next();
    } else if constexpr (FUSED) {
        // one pass: thread t quantises values
        // 16 m .. 16 m + 15 of block b as lane m of a DPP row, from one round
        // of loads of x and of the pre-op's operand (rmsnorm weights or up;
        // x again when there is none); threads past the last block take a
        // clamped copy, add nothing to the sum of squares and store nothing
        const int b = t >> 4, m = t & 15;
        const bool on = b < nblk;
        const int64_t off = (int64_t)min(b, nblk - 1) * 256 + 16 * m;
        const float *opnd = a.norm_w ? a.norm_w : a.up ? a.up : a.x;
        float v[16], w[16];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float4 f = *(const float4 *)(a.x + off + 4 * k);
            v[4 * k] = f.x; v[4 * k + 1] = f.y; v[4 * k + 2] = f.z; v[4 * k + 3] = f.w;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float4 f = *(const float4 *)(opnd + off + 4 * k);
            w[4 * k] = f.x; w[4 * k + 1] = f.y; w[4 * k + 2] = f.z; w[4 * k + 3] = f.w;
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int d = 0; d < D; ++d) buf[d] = load_next();
        __builtin_amdgcn_sched_barrier(0);
        if (a.norm_w) {
            // kore's rmsnorm (kore.cpp:1367-1372): the certified scale of
            // block_rms_scale_sum from this thread's sum of squares (four
            // chains), then x * scale * w with kore's roundings; the records
            // area is free until the blocks start
            double sq[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
            for (int e = 0; e < 16; ++e) sq[e & 3] += on ? (double)v[e] * (double)v[e] : 0.0;
            const float scale = block_rms_scale_sum((sq[0] + sq[1]) + (sq[2] + sq[3]), a.x, nblk * 256, a.norm_eps,
                                                    (double *)smem);
#pragma unroll
            for (int e = 0; e < 16; ++e) v[e] = (v[e] * scale) * w[e];
        } else if (a.up) {
#pragma unroll
            for (int e = 0; e < 16; ++e) v[e] = kore_swiglu(v[e], w[e]);
        }
        const Q8Lane q = quantize16(v, m);
        if (on) xs_store(xs, nblk, b, m, q);
    } else if (a.xq_image) {
        // already in the LDS layout (xs_bytes(nblk) is a multiple of 4 bytes)
        const int n16 = (int)(xs_bytes(nblk) >> 4);
        for (int c = t; c < n16; c += kThreads) ((uint4 *)xs)[c] = ((const uint4 *)a.xq)[c];
        for (int c = 4 * n16 + t; c < (int)(xs_bytes(nblk) >> 2); c += kThreads)
            ((uint32_t *)xs)[c] = ((const uint32_t *)a.xq)[c];
    } else {
        // kore's records (dword-aligned) into the LDS layout: per block, the
        // 64 qs dwords by 64 lanes, then the 8 bsums dwords and d
        const int w = t >> 6, l = t & 63;
        for (int b = w; b < nblk; b += kThreads / 64) {
            const uint32_t *src = (const uint32_t *)(a.xq + b * kQ8Bytes);
            *(uint32_t *)(xs + b * kXsQs + 4 * l) = src[1 + l];
            if (l < 8) *(uint32_t *)(xs + nblk * kXsQs + 32 * b + 4 * l) = src[65 + l];
            else if (l == 8) *(float *)(xs + nblk * 304 + 4 * b) = __uint_as_float(src[0]);
        }
    }
    if constexpr (!FUSED) {
#pragma unroll
        for (int d = 0; d < D; ++d) buf[d] = load_next();
    }
    __syncthreads();
    const Q8View x{xs, nblk};

    float acc0 = 0.f, acc1 = 0.f, accm = 0.f;               // chain state of the phase-0 lanes
    const bool chain = ph == 0;
    int ct = tile_begin, cs = 0;                            // compute cursor

    auto advance = [&](const Rec &q, const Rec &q0, const Rec &q1) {
        // one block of kore's per-lane float arithmetic; q is this lane's
        // part, q0 / q1 parts 0 / 1 of the same unit
        if constexpr (AVX2) {
            if constexpr (TYPE == kQ4K) {
                acc0 = fmaf(q0.x, (float)q.a, acc0);
                acc1 = fmaf(q0.x, (float)q.b, acc1);
                accm = fmaf(-q1.x, (float)q.c, accm);
            } else {
                acc0 = fmaf(q.x, (float)q.a, acc0);
                acc1 = fmaf(q.x, (float)q.b, acc1);
                accm = fmaf(-(q.x * 32.0f), (float)q.c, accm);   // summ (kore.cpp:606)
            }
        } else {
            if constexpr (TYPE == kQ4K) {
                const float t1 = q0.x * (float)q0.a;
                const float t2 = __int_as_float(q0.c) * (float)q0.b;
                acc0 = acc0 + (t1 - t2);
            } else {
                acc0 = acc0 + q0.x * (float)q0.a;
            }
        }
    };

    // one step k of the compute cursor over the loaded parts `raw`
    auto step = [&](const Raw &raw, int k) {
        const int i = min(cs * P + ph, nblk - 1);
        Rec r;
        if constexpr (TYPE == kQ4K) r = part_q4<AVX2>(raw, x, i, j);
        else r = part_q6<AVX2>(raw, x, i, j);
        if (k < total) {
            if constexpr (P == 1) {
                // the unit's four parts are this lane's quad: d / dmin from parts 0 / 1
                Rec q0 = r, q1 = r;
                if constexpr (TYPE == kQ4K && AVX2) {
                    // part j holds d (j even) or dmin (j odd): take both from the quad
                    const float other = quad_xor1f(r.x);
                    q0.x = (j & 1) ? other : r.x;
                    q1.x = (j & 1) ? r.x : other;
                }
                advance(r, q0, q1);
            } else {
                Rec *rb = recs + (k & 1) * 64;
                rb[l] = r;
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                if (chain) {
                    // the records of four blocks at a time are read before
                    // their chain steps, so the LDS latency is paid per group
                    const int nb = min(P, nblk - cs * P);
#pragma unroll
                    for (int b0 = 0; b0 < P; b0 += 4) {
                        if (b0 >= nb) break;
                        constexpr int G = P < 4 ? P : 4;
                        Rec qs[G], q0s[G], q1s[G];
#pragma unroll
                        for (int u = 0; u < G; ++u) {
                            const int base = ((b0 + u) * RW + rho) * 4;
                            qs[u] = rb[base + j];
                            q0s[u] = rb[base];
                            q1s[u] = rb[base + 1];
                        }
#pragma unroll
                        for (int u = 0; u < G; ++u)
                            if (b0 + u < nb) advance(qs[u], q0s[u], q1s[u]);
                    }
                }
            }
            if (++cs == nsteps) {
                // the tile's rows are complete
                if (chain) {
                    float res;
                    if constexpr (AVX2) {
                        // kore's hsum256 (kore.cpp:521-528): lanes k and k+4 first,
                        // then (l0 + l2) + (l1 + l3); parts 0..3 hold lanes {0,1},
                        // {4,5}, {2,3}, {6,7}
                        const float u = acc0 + quad_xor1f(acc0);     // part 0: l0, part 2: l2
                        const float v = acc1 + quad_xor1f(acc1);     // part 0: l1, part 2: l3
                        const float h8 = (u + quad_xor2f(u)) + (v + quad_xor2f(v));
                        if constexpr (TYPE == kQ4K) {
                            const float m = accm + quad_xor2f(accm); // hsum128 (kore.cpp:537-541)
                            res = h8 + (m + quad_xor1f(m));
                        } else {
                            res = h8 + accm;
                        }
                    } else {
                        res = acc0;
                    }
                    const int orow = (ct * 4 + wave) * RW + rho;
                    if (j == 0 && orow < rows) {
                        // kore's q += bq (kore.cpp:1422-1423), x += o (kore.cpp:1458, 1471)
                        const float v = md.bias ? res + md.bias[orow] : res;
                        md.out[orow] = md.accumulate ? md.out[orow] + v : v;
                    }
                    acc0 = acc1 = accm = 0.f;
                }
                cs = 0;
                ++ct;
            }
        }
    };

    if constexpr (PIPE == 0) {
        // D steps are computed, then the next D requested (a step past the
        // end repeats the last one's clamped addresses and is discarded); buf
        // keeps its registers across the back-edge, so no copy waits for its
        // loads.
        for (int k0 = 0;;) {
#pragma unroll
            for (int d = 0; d < D; ++d) step(buf[d], k0 + d);
            k0 += D;
            if (k0 >= total) break;
#pragma unroll
            for (int d = 0; d < D; ++d) buf[d] = load_next();
        }
    } else {
        // the next D steps are requested before the current D are computed
        // (two register sets, unrolled so that neither is copied)
        for (int k0 = 0;; k0 += 2 * D) {
            Raw nb[D];
#pragma unroll
            for (int d = 0; d < D; ++d) nb[d] = load_next();
#pragma unroll
            for (int d = 0; d < D; ++d) step(buf[d], k0 + d);
            if (k0 + D >= total) break;
#pragma unroll
            for (int d = 0; d < D; ++d) buf[d] = load_next();
#pragma unroll
            for (int d = 0; d < D; ++d) step(nb[d], k0 + D + d);
            if (k0 + 2 * D >= total) break;
        }
    }
}

// One launch over up to kMaxGroup matrices that read the same activations:
// workgroups [m.wg_begin, m.wg_begin + m.wg_count) belong to matrix m and
// split its tiles of 4 RW rows evenly in contiguous runs.
template <bool AVX2, int RW, bool FUSED, int D, int PIPE>
__global__ __launch_bounds__(kThreads) void matvec_group_kernel(GroupArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int g = blockIdx.x;
    MatDesc md = a.m[0];
#pragma unroll
    for (int k = 1; k < kMaxGroup; ++k)
        if (k < a.n_mat && g >= a.m[k].wg_begin) md = a.m[k];
    const int w = g - md.wg_begin;
    const int64_t tiles = (md.rows + 4 * RW - 1) / (4 * RW);
    const int tb = (int)(tiles * w / md.wg_count), te = (int)(tiles * (w + 1) / md.wg_count);
    if (tb >= te) return;
    if (md.type == kQ4K) matvec_body<kQ4K, AVX2, RW, FUSED, D, PIPE>(md, tb, te, a, smem);
    else matvec_body<kQ6K, AVX2, RW, FUSED, D, PIPE>(md, tb, te, a, smem);
}

// Q6_K upload: thread per output dword (52 body dwords + the scale per block).
__global__ __launch_bounds__(kThreads) void q6k_split_kernel(const uint16_t *__restrict__ raw, int64_t nblocks,
                                                             uint32_t *__restrict__ body,
                                                             uint16_t *__restrict__ d) {
    const int64_t g = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (g >= nblocks * 53) return;
    const int64_t blk = g / 53;
    const int q = (int)(g % 53);
    const uint16_t *src = raw + blk * (kQ6Bytes / 2);
    if (q < 52) body[blk * 52 + q] = (uint32_t)src[2 * q] | ((uint32_t)src[2 * q + 1] << 16);
    else d[blk] = src[104];
}

// Synthetic GGUF blocks: every 16-bit word a hash of (seed, index), the f16
// scales replaced by finite values in [2^-8, 2^-7) (d) and [2^-9, 2^-8) (dmin).
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ __launch_bounds__(kThreads) void synth_blocks_kernel(uint16_t *__restrict__ dst, int64_t n16,
                                                                int words_per_block, int d_word, int dmin_word,
                                                                uint64_t key) {
    const int64_t g = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (g >= n16) return;
    const uint32_t h = (uint32_t)splitmix64(key ^ (uint64_t)g);
    const int wi = (int)(g % words_per_block);
    uint16_t v = (uint16_t)h;
    if (wi == d_word) v = (uint16_t)(0x1C00u | (h & 0x3FFu));
    else if (wi == dmin_word) v = (uint16_t)(0x1800u | (h & 0x3FFu));
    dst[g] = v;
}

// Load pipelining (measured on 7B shapes): one step requested ahead of the
// step computed, except for grids of more workgroups than the device holds
// at once (the 152064-row output head: 2376), where batches of two steps,
// each requested after the one before is computed, leave more room for
// other workgroups' loads.  KORE_QMV_PIPE=0 / 1 forces either form.
template <bool AVX2, int RW, bool FUSED>
hipError_t launch_group_r(const GroupArgs &a, int grid, int num_cu, hipStream_t s) {
    const size_t lds = 2 * kThreads * sizeof(Rec) + xs_bytes(a.nblk);
    static const int forced = [] {
        const char *e = getenv("KORE_QMV_PIPE");
        return e ? atoi(e) : -1;
    }();
    const int pipe = forced >= 0 ? forced : (num_cu > 0 && grid > 4 * num_cu ? 0 : 1);
    if (pipe == 0) hipLaunchKernelGGL((matvec_group_kernel<AVX2, RW, FUSED, 2, 0>), dim3(grid), dim3(kThreads), lds, s, a);
    else hipLaunchKernelGGL((matvec_group_kernel<AVX2, RW, FUSED, 1, 1>), dim3(grid), dim3(kThreads), lds, s, a);
    return hipGetLastError();
}

template <bool AVX2, bool FUSED>
hipError_t launch_group_f(const GroupArgs &a, int rw, int grid, int num_cu, hipStream_t s) {
    switch (rw) {
        case 1: return launch_group_r<AVX2, 1, FUSED>(a, grid, num_cu, s);
        case 2: return launch_group_r<AVX2, 2, FUSED>(a, grid, num_cu, s);
        case 4: return launch_group_r<AVX2, 4, FUSED>(a, grid, num_cu, s);
        case 8: return launch_group_r<AVX2, 8, FUSED>(a, grid, num_cu, s);
        default: return launch_group_r<AVX2, 16, FUSED>(a, grid, num_cu, s);
    }
}

uint64_t splitmix64_host(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

}  // namespace

hipError_t launch_matvec_group(bool avx2, GroupArgs a, int rows_per_wave, int max_wgs, int num_cu, hipStream_t s) {
    if (a.n_mat < 1 || a.n_mat > kMaxGroup || a.nblk <= 0 || a.nblk > kMaxBlocks) return hipErrorInvalidValue;
    const int rw = rows_per_wave;
    if (rw != 1 && rw != 2 && rw != 4 && rw != 8 && rw != 16) return hipErrorInvalidValue;
    const int rows_per_tile = 4 * rw;
    const bool fused = a.x != nullptr;
    if (!fused && !a.xq) return hipErrorInvalidValue;
    if ((a.norm_w || a.up) && !fused) return hipErrorInvalidValue;   // pre-ops act on x
    if (a.norm_w && a.up) return hipErrorInvalidValue;
    // workgroups per matrix: one per row tile when the launch may have a
    // workgroup per tile (max_wgs 0 or at least the tiles); else in proportion
    // to its weight bytes, at least one, at most one per row tile, about
    // max_wgs in all.  (Proportional shares at one tile per workgroup would
    // give a Q4_K matrix grouped with a Q6_K one fewer workgroups than tiles:
    // q+k+v with a Q6_K attn_v had 13 workgroups walking two tiles, which
    // ended 3 us after the others.)
    int64_t tiles[kMaxGroup], bytes[kMaxGroup], all_tiles = 0, all_bytes = 0;
    for (int k = 0; k < a.n_mat; ++k) {
        const MatDesc &m = a.m[k];
        if (m.rows <= 0 || !m.w || !m.out || (m.type != kQ4K && m.type != kQ6K) || (m.type == kQ6K && !m.wd))
            return hipErrorInvalidValue;
        tiles[k] = (m.rows + rows_per_tile - 1) / rows_per_tile;
        bytes[k] = (int64_t)m.rows * (m.type == kQ4K ? kQ4Bytes : kQ6Bytes);
        all_tiles += tiles[k];
        all_bytes += bytes[k];
    }
    const bool per_tile = max_wgs <= 0 || max_wgs >= all_tiles;
    int64_t wg = 0;
    for (int k = 0; k < a.n_mat; ++k) {
        MatDesc &m = a.m[k];
        int64_t n = per_tile ? tiles[k] : ((int64_t)max_wgs * bytes[k] + all_bytes / 2) / all_bytes;
        n = std::max<int64_t>(1, std::min<int64_t>(n, tiles[k]));
        m.wg_begin = (int)wg;
        m.wg_count = (int)n;
        wg += n;
    }
    for (int k = a.n_mat; k < kMaxGroup; ++k) a.m[k] = a.m[a.n_mat - 1];
    if (wg > INT32_MAX) return hipErrorInvalidValue;
    const int grid = (int)wg;
    if (avx2)
        return fused ? launch_group_f<true, true>(a, rw, grid, num_cu, s) : launch_group_f<true, false>(a, rw, grid, num_cu, s);
    return fused ? launch_group_f<false, true>(a, rw, grid, num_cu, s) : launch_group_f<false, false>(a, rw, grid, num_cu, s);
}

hipError_t launch_quantize_q8k(const float *x, int64_t n, uint8_t *xq, bool image, hipStream_t s, PreOp pre) {
    const int64_t nb = n / 256;
    if (nb <= 0) return hipSuccess;
    if (image && nb > kMaxBlocks) return hipErrorInvalidValue;
    if (pre.norm_w && pre.up) return hipErrorInvalidValue;
    if (pre.norm_w && n > INT32_MAX) return hipErrorInvalidValue;
    if (pre.up) {
        if (nb > INT32_MAX) return hipErrorInvalidValue;
        if (image) hipLaunchKernelGGL(swiglu_quantize_kernel<true>, dim3((unsigned)nb), dim3(kThreads), 0, s, x, pre.up, xq, nb);
        else hipLaunchKernelGGL(swiglu_quantize_kernel<false>, dim3((unsigned)nb), dim3(kThreads), 0, s, x, pre.up, xq, nb);
        return hipGetLastError();
    }
    const int64_t grid = (nb + kThreads / 16 - 1) / (kThreads / 16);
    if (image) hipLaunchKernelGGL(quantize_q8k_kernel<true>, dim3((unsigned)grid), dim3(kThreads), 0, s, x, xq, nb, pre);
    else hipLaunchKernelGGL(quantize_q8k_kernel<false>, dim3((unsigned)grid), dim3(kThreads), 0, s, x, xq, nb, pre);
    return hipGetLastError();
}

hipError_t launch_synth_blocks(int type, int64_t nblocks, uint64_t seed, uint8_t *dst, hipStream_t s) {
    if (nblocks <= 0) return hipSuccess;
    const int wpb = (type == kQ4K ? kQ4Bytes : kQ6Bytes) / 2;
    const int64_t n16 = nblocks * wpb;
    const int64_t grid = (n16 + kThreads - 1) / kThreads;
    hipLaunchKernelGGL(synth_blocks_kernel, dim3((unsigned)grid), dim3(kThreads), 0, s, (uint16_t *)dst, n16, wpb,
                       type == kQ4K ? 0 : 104, type == kQ4K ? 1 : -1, splitmix64_host(seed));
    return hipGetLastError();
}

hipError_t launch_q6k_split(const uint8_t *raw, int64_t nblocks, uint8_t *body, uint16_t *d, hipStream_t s) {
    if (nblocks <= 0) return hipSuccess;
    const int64_t grid = (nblocks * 53 + kThreads - 1) / kThreads;
    hipLaunchKernelGGL(q6k_split_kernel, dim3((unsigned)grid), dim3(kThreads), 0, s, (const uint16_t *)raw,
                       nblocks, (uint32_t *)body, d);
    return hipGetLastError();
}

}  // namespace kore_qmv_gpu

// ------------------------------------------------------------------ row-wise steps of forward_batch

namespace kore_qmv_gpu {
namespace {

// kore's rmsnorm of one row of n values (n a multiple of 256 up to 4096, every
// pointer 16-byte aligned) that also writes the row as the fp16 batched
// matmul's split activations (g16_split_group, as gemm16_prep_kernel writes
// them, so the bytes are the pre-pass's own).  Thread t takes float4 groups
// t + 256 j: lane t % 64 of block 4 j + t / 64.
__device__ void rmsnorm_split_row(const float *xr, const float *__restrict__ w, int n, float eps, float *orow,
                                  uint8_t *__restrict__ x16, double *red, float *fred) {
    const int t = threadIdx.x, lane = t & 63, b = blockIdx.x, n4 = n / 4;
    const float4 *x4 = (const float4 *)xr, *w4 = (const float4 *)w;
    float4 v[4], wv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int f = min(t + j * kThreads, n4 - 1);
        v[j] = x4[f];
        wv[j] = w4[f];
    }
    // the certified scale of block_rms_scale_sum from each thread's plain
    // double sum of its exact squares (four chains)
    double sq[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const bool in = t + j * kThreads < n4;
        const float e[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) sq[k] += in ? (double)e[k] * (double)e[k] : 0.0;
    }
    const float scale = block_rms_scale_sum((sq[0] + sq[1]) + (sq[2] + sq[3]), xr, n, eps, red);
    float4 y[4];
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        y[j] = make_float4((v[j].x * scale) * wv[j].x, (v[j].y * scale) * wv[j].y, (v[j].z * scale) * wv[j].z,
                           (v[j].w * scale) * wv[j].w);
        if (t + j * kThreads < n4) {
            ((float4 *)orow)[t + j * kThreads] = y[j];
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(y[j].x), fabsf(y[j].y)), fmaxf(fabsf(y[j].z), fabsf(y[j].w))));
        }
    }
    amax = g16_wave_max(amax);
    if (lane == 0) fred[t >> 6] = amax;                // its own LDS words: red may still be read
    __syncthreads();
    amax = fmaxf(fmaxf(fred[0], fred[1]), fmaxf(fred[2], fred[3]));
    float s1, s2, inv;
    g16_split_scale(amax, s1, s2, inv);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (t + j * kThreads >= n4) break;             // whole waves: n4 is a multiple of 64
        const float ys[4] = {(y[j].x * s1) * s2, (y[j].y * s1) * s2, (y[j].z * s1) * s2, (y[j].w * s1) * s2};
        g16_split_group(x16, b, (t + j * kThreads) >> 6, lane, ys, inv);
    }
}

// kore's rmsnorm of row blockIdx.x (kore.cpp:1367-1372, 1522, 1573): the
// certified scale of block_rms_scale, then x * scale * w with kore's roundings.
__global__ __launch_bounds__(kThreads) void rmsnorm_rows_kernel(const float *x, const float *__restrict__ w, int n,
                                                                float eps, float *out, uint8_t *__restrict__ x16) {
    __shared__ double red[2 * kThreads / 64];
    __shared__ float fred[kThreads / 64];
    const float *xr = x + (int64_t)blockIdx.x * n;
    float *orow = out + (int64_t)blockIdx.x * n;
    constexpr int kPer = 16;
    if (x16) {
        rmsnorm_split_row(xr, w, n, eps, orow, x16, red, fred);
        return;
    }
    if (n > kPer * kThreads) {
        const float scale = block_rms_scale(xr, n, eps, red);
        for (int i = threadIdx.x; i < n; i += kThreads) orow[i] = (xr[i] * scale) * w[i];
        return;
    }
    // rows up to 4096: every load of x and w issued up front (clamped indexes,
    // so no load waits on a branch), the sum in block_rms_scale's order; a
    // slot past n adds 0.0, which leaves hi and lo unchanged
    float v[kPer], wv[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int i = min((int)threadIdx.x + j * kThreads, n - 1);
        v[j] = xr[i];
        wv[j] = w[i];
    }
    double hi = 0.0, lo = 0.0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const float xv = (int)threadIdx.x + j * kThreads < n ? v[j] : 0.0f;
        double s, e;
        two_sum(hi, (double)xv * (double)xv, s, e);
        hi = s;
        lo += e;
    }
    const float scale = block_rms_scale_from(hi, lo, xr, n, eps, red);
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int i = (int)threadIdx.x + j * kThreads;
        if (i < n) orow[i] = (v[j] * scale) * wv[j];
    }
}

__global__ __launch_bounds__(kThreads) void swiglu_kernel(float *__restrict__ g, const float *__restrict__ u, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) g[i] = kore_swiglu(g[i], u[i]);
}

}  // namespace

hipError_t launch_rmsnorm_rows(const float *x, const float *w, int n, int n_rows, float eps, float *out, hipStream_t s,
                               uint8_t *x16) {
    if (n <= 0 || n_rows <= 0 || !x || !w || !out) return hipErrorInvalidValue;
    if (x16 && (n % 256 || n > 16 * kThreads || n_rows > kGemmMaxB ||
                (((uintptr_t)x | (uintptr_t)w | (uintptr_t)out | (uintptr_t)x16) & 15)))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3((unsigned)n_rows), dim3(kThreads), 0, s, x, w, n, eps, out, x16);
    return hipGetLastError();
}

hipError_t launch_swiglu(float *g, const float *u, int64_t n, hipStream_t s) {
    if (n <= 0 || !g || !u) return hipErrorInvalidValue;
    hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((n + kThreads - 1) / kThreads)), dim3(kThreads), 0, s, g, u, n);
    return hipGetLastError();
}

}  // namespace kore_qmv_gpu

// ------------------------------------------------------------------ get_row

namespace kore_qmv_gpu {
namespace {

__device__ __forceinline__ float f16_at(const uint8_t *p) { return f16_bits((uint32_t)p[0] | ((uint32_t)p[1] << 8)); }

// kore's get_row (kore.cpp:384-407): value i of a row of n values, one thread
// per value.  Q4_K / Q6_K follow kore's dequantisers (kore.cpp:337-381) with
// their separate roundings (no fused multiply-add).
__global__ __launch_bounds__(kThreads) void get_row_kernel(int type, const uint8_t *__restrict__ row, int64_t n,
                                                           float *__restrict__ out) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    float v = 0.f;
    if (type == 0) {                                     // F32
        v = ((const float *)row)[i];
    } else if (type == 1) {                              // F16
        v = f16_at(row + 2 * i);
    } else if (type == 30) {                             // BF16: the high half of a float
        v = __uint_as_float(((uint32_t)row[2 * i] | ((uint32_t)row[2 * i + 1] << 8)) << 16);
    } else if (type == kQ4K) {
        const uint8_t *b = row + (i / 256) * kQ4Bytes;
        const int e = (int)(i % 256), j = e / 32, l = e % 32;   // sub-block j, value l
        const uint8_t *s = b + 4;
        const int sc = j < 4 ? (s[j] & 63) : ((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
        const int mn = j < 4 ? (s[j + 4] & 63) : ((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
        const float d1 = f16_at(b) * (float)sc, m1 = f16_at(b + 2) * (float)mn;
        const uint8_t qb = b[16 + 32 * (j / 2) + l];
        const int q = (j & 1) ? (qb >> 4) : (qb & 0xF);
        v = d1 * (float)q - m1;
    } else {                                             // Q6_K, kore's 210-byte blocks
        const uint8_t *b = row + (i / 256) * kQ6Bytes;
        const int e = (int)(i % 256), h = e / 128, k = (e % 128) / 32, l = e % 32;
        const uint8_t lo = b[64 * h + 32 * (k & 1) + l];
        const int ql = k < 2 ? (lo & 0xF) : (lo >> 4);
        const int qh = (b[128 + 32 * h + l] >> (2 * k)) & 3;
        const float sc = (float)(int8_t)b[192 + 8 * h + 2 * k + l / 16];
        v = (f16_at(b + 208) * sc) * (float)((ql | (qh << 4)) - 32);
    }
    out[i] = v;
}

}  // namespace

hipError_t launch_get_row(int type, const uint8_t *data, int64_t row, int64_t n, float *out, hipStream_t s) {
    int64_t per = 1, bytes = 4;
    if (type == 1 || type == 30) bytes = 2;
    else if (type == kQ4K) { per = 256; bytes = kQ4Bytes; }
    else if (type == kQ6K) { per = 256; bytes = kQ6Bytes; }
    else if (type != 0) return hipErrorInvalidValue;
    if (n <= 0 || n % per || row < 0) return hipErrorInvalidValue;
    const uint8_t *p = data + row * (n / per * bytes);
    hipLaunchKernelGGL(get_row_kernel, dim3((unsigned)((n + kThreads - 1) / kThreads)), dim3(kThreads), 0, s, type, p,
                       n, out);
    return hipGetLastError();
}

}  // namespace kore_qmv_gpu
