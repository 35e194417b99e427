// kore_qmv_kernels.h - launch interface of the gfx950 kernels behind the
// kore_qmv C ABI (quantised matrix-vector products).  Internal to
// libkore_qmv.so.
//
// Device layouts
//   activations  kore's BlockQ8K array (kore.cpp:415-420): per 256 values a
//                292-byte record {float d; int8 qs[256]; int16 bsums[16]}.
//   Q4_K weights kore's / GGUF's 144-byte blocks unchanged (kore.cpp:324-326):
//                rows x nblk blocks, row-major; every block is 16-byte aligned.
//   Q6_K weights the 210-byte GGUF block (kore.cpp:355-357) split in two
//                arrays so every load is aligned: `body` holds its first 208
//                bytes (ql[128], qh[64], int8 scales[16]) per block, `d` its
//                f16 scale, both indexed row * nblk + block.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <type_traits>

namespace kore_qmv_gpu {

constexpr int kQ8Bytes = 292;
constexpr int kQ4Bytes = 144;
constexpr int kQ6Bytes = 210;
constexpr int kQ6Body = 208;
constexpr int kMaxBlocks = 128;   // cols <= 32768: the staged activations fit in LDS

enum WeightType { kQ4K = 12, kQ6K = 14 };

// Rows are processed by waves: a wave owns `rows_per_wave` rows (1, 2, 4, 8
// or 16) of one matrix and walks their blocks in order; the four waves of a
// 256-thread workgroup take consecutive row groups and share the activations.
// One launch may cover up to kMaxGroup matrices that multiply the same
// activations (kore's q/k/v and gate/up matvecs share one quant(),
// kore.cpp:1418-1421, 1462-1464).
constexpr int kMaxGroup = 4;

struct MatDesc {
    const uint8_t *w;        // Q4_K blocks, or the Q6_K 208-byte bodies
    const uint16_t *wd;      // Q6_K f16 scales (nullptr for Q4_K)
    float *out;              // [rows]
    int rows;
    int type;                // kQ4K or kQ6K
    int wg_begin;            // first workgroup of this matrix   (set by the launcher)
    int wg_count;            // its number of workgroups          (set by the launcher)
    const float *bias;       // out = dot + bias[r] (kore's q/k/v biases), or nullptr
    int accumulate;          // out = out + dot (kore's residual adds)
};

struct GroupArgs {
    MatDesc m[kMaxGroup];
    int n_mat;
    int nblk;                // cols / 256, shared by the group
    const uint8_t *xq;       // nblk BlockQ8K records (16-byte aligned), or
    const float *x;          // nblk*256 floats (16-byte aligned) that every workgroup
                             // quantises into LDS itself (then xq is unused)
    int xq_image;            // xq holds launch_quantize_q8k(..., image = true)'s layout
    // applied to x before the in-kernel quantisation (not with xq):
    const float *norm_w;     // kore's rmsnorm with these weights (kore.cpp:1367-1372), or nullptr
    float norm_eps;
    const float *up;         // kore's SwiGLU, x = gate (kore.cpp:1465-1468), or nullptr
};

// What a quantiser does to its input first (at most one of the two).
struct PreOp {
    const float *norm_w;     // rmsnorm: x[i] * scale * norm_w[i]
    float norm_eps;
    const float *up;         // SwiGLU: x[i] / (1 + exp(-x[i])) * up[i]
};

// out[r] = row r . xq for every matrix of the group, with kore's summation:
// avx2 = true follows dot_q*_K_q8_K_avx2 (kore.cpp:535-632), false
// dot_q*_K_q8_K_ref (kore.cpp:450-506).  Bit-identical to kore's results in
// both orders, with or without the fused quantisation.  Tiles are 4 x
// rows_per_wave rows; about max_wgs workgroups (0: one per tile) share them,
// each a contiguous run.  num_cu (0 if unknown) selects the load pipelining:
// a grid that does not fit on the device at once takes batches of two steps.
hipError_t launch_matvec_group(bool avx2, GroupArgs a, int rows_per_wave, int max_wgs, int num_cu, hipStream_t s);

// kore's quantize_row_q8_K (kore.cpp:422-446): x[n] -> n/256 BlockQ8K records,
// or (image) the same values in the matvec's own layout (n/256 * 308 bytes,
// n/256 <= kMaxBlocks) for a following launch_matvec_group with xq_image.
hipError_t launch_quantize_q8k(const float *x, int64_t n, uint8_t *xq, bool image, hipStream_t s,
                               PreOp pre = PreOp{nullptr, 0.f, nullptr});

// Q6_K upload: raw GGUF blocks (rows*nblk x 210 bytes, any alignment of 2)
// -> body / d arrays above.
hipError_t launch_q6k_split(const uint8_t *raw, int64_t nblocks, uint8_t *body, uint16_t *d, hipStream_t s);

// kore's rmsnorm (kore.cpp:1367-1372) of each of n_rows rows of n values
// (out may be x), bit-identical to kore's sequential double sum; and kore's
// SwiGLU in place over n values (kore.cpp:1577-1581, exp rounded from double).
// With x16 (n a multiple of 256 up to 4096, n_rows <= 64) the normalised rows
// are also written as the fp16 batched matmul's split activations (the layout
// and values its own pre-pass would produce, bit for bit).
hipError_t launch_rmsnorm_rows(const float *x, const float *w, int n, int n_rows, float eps, float *out, hipStream_t s,
                               uint8_t *x16 = nullptr);
hipError_t launch_swiglu(float *g, const float *u, int64_t n, hipStream_t s);

// kore's get_row (kore.cpp:384-407): row `row` of a table of rows of n values
// of type F32 / F16 / BF16 / Q4_K / Q6_K (kore's block bytes) -> out[n] floats.
hipError_t launch_get_row(int type, const uint8_t *data, int64_t row, int64_t n, float *out, hipStream_t s);

// Synthetic GGUF-format weights for benchmarks: nblocks raw Q4_K / Q6_K blocks
// with hashed bytes and finite f16 scales (dst 2-byte aligned).
hipError_t launch_synth_blocks(int type, int64_t nblocks, uint64_t seed, uint8_t *dst, hipStream_t s);

// Batched prefill matmul (kore's matmul_batch_float, kore.cpp:783-845):
// out[b * rows + r] = dequantised row r . x[b], b < B <= kGemmMaxB; fp16 MFMA
// on exact integer weights and split activations (below), or fp32 MFMA;
// equal to kore's results to rounding.  One launch covers up to kMaxGroup
// matrices that share x (same cols), each with its own output.
//
// Work split (stream-K): the iteration space (row tile, 256-column block)
// of all the matrices is cut into `workers` equal contiguous runs, one per
// workgroup.  A tile whose blocks fall to several workers is finished by a
// second launch that adds their partial sums in worker order.
constexpr int kGemmMaxB = 64;            // kore's KORE_BMAX (kore.cpp:690)
constexpr int kGemmRowsPerTile = 64;
constexpr int kGemmSlotFloats = kGemmRowsPerTile * kGemmMaxB;   // one partial tile
struct GemmMat {
    const uint8_t *w;        // Q4_K blocks or Q6_K bodies
    const uint16_t *wd;      // Q6_K f16 scales
    float *out;              // [B][rows]
    int rows, type;
    int tile0;               // first tile of this matrix in the launch
    const float *bias;       // out = dot + bias[r] (kore's q/k/v biases), or nullptr
    int accumulate;          // out = out + dot (kore's residual adds)
};
struct GemmArgs {
    GemmMat m[kMaxGroup];
    int n_mat;
    const float *x;          // [B][nblk * 256], 16-byte aligned
    int B, nblk;
    int tiles;               // all matrices' tiles
    int workers;             // grid size (gemm_workers)
    float *partials;         // 2 * workers * kGemmSlotFloats floats
    uint8_t *x16;            // nblk * kG16BlockBytes: the fp16 split of x (fp16 path)
    int presplit;            // x16 already holds the split (x unused): no pre-pass
    int halves;              // 1, or 2 (fp16 path): work units of 32 activations per tile
    int glu;                 // fp16 path, m[0] = gate, m[1] = up (equal rows, no bias or
                             // accumulate): m[0].out = kore's SwiGLU of the two products,
                             // m[1].out scratch
};

// fp16 path of the batched matmul (the default): the weights enter the MFMA
// as small exact integers (Q4_K sc*q, Q6_K sc*(q-32) split in two fp16
// parts), the activations as two fp16 parts per value with a power-of-two
// scale per (activation, 256-column block); d, dmin and the Q4_K minimums
// are applied per block in fp32.  Tiles of 256 rows; per block the split
// activations take kG16BlockBytes: hi [64][32 chunks of 8 fp16], lo (same),
// the sub-block sums (8 hi, 8 lo fp16 per activation) and 1 / scale.
constexpr int kG16Rows = 256;
constexpr int kG16Lo = 64 * 512;
constexpr int kG16Sx = 2 * 64 * 512;
constexpr int kG16Inv = kG16Sx + 64 * 32;
constexpr int kG16BlockBytes = kG16Inv + 64 * 4;
constexpr int kG16SlotFloats = kG16Rows * kGemmMaxB;   // one partial tile
// Tiles of the fp16 path, or of the fp32 one (KORE_GEMM=fp32 in the
// environment selects it, for comparisons).
bool gemm_fp16();
int gemm_rows_per_tile();
// 2 when the fp16 path splits each tile's activations into two units of 32
// (B > 32 and fewer than two (tile, block) iterations per CU: the workers then
// cover all CUs with units half the size), else 1.  The workers and the
// partials are counted in units (tiles x halves).
int gemm_halves(int tiles, int nblk, int B, int num_cu);
// Workers of one launch: as many as fit on the CUs at once (by the LDS and
// registers of the kernel that B activations and the weight types select), at
// least two iterations each.
int gemm_workers(int tiles, int nblk, int B, bool has_q6k, int num_cu);
// Largest grid any launch on a device with num_cu CUs uses (sizes partials).
int gemm_max_workers(int num_cu);
hipError_t launch_gemm(GemmArgs a, hipStream_t s);

}  // namespace kore_qmv_gpu
