// kore_attn_kernels.h - launch interface of the gfx950 kernels behind the
// kore_attn C ABI.  Internal to libkore_attn.so.
//
// KV-cache layout in HBM (one allocation each for K and V):
//     [layer][kv_head][slot][head_dim]  fp32
// i.e. every kv-head of a layer is one contiguous run of `slots` rows of
// head_dim floats.  kore keeps [layer][pos][kv_head][head_dim]
// (kore.cpp:1260); the values are identical, only the order of rows
// differs, so kore_attn_read_kv() gives kore's layout back.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace kore_attn_gpu {

// Single-token decode, two launches.  The split kernel does RoPE of q and of
// the new k row, the append of the new k/v row, and flash-decoding attention
// of every (kv-head, split) over the cache slots [0, n_rows) in blocks of
// kDecodeBlock rows plus the new row itself; with one split it writes `out`,
// otherwise unnormalised split partials that the combine kernel merges.
constexpr int kDecodeBlock = 16;
constexpr int kMaxDecodeSplits = 256;   // splits per kv-head the combine merges in one round

struct DecodeArgs {
    const float *q;       // [n_head][hd]        post-bias, pre-RoPE
    const float *k;       // [n_head_kv][hd]     post-bias, pre-RoPE
    const float *v;       // [n_head_kv][hd]
    float *kc, *vc;       // layer base, [n_head_kv][slots][hd]
    float *out;           // [n_head][hd]
    float *part_o;        // [n_head][n_split][hd]   split partial outputs
    float *part_ml;       // [n_head][n_split][2]    split max / sum
    int slots;            // rows per kv-head in the cache (ctx)
    int n_rows;           // cache slots read: [0, n_rows), the new row excluded
                          // (a wrapped ring reads all slots and masks new_slot)
    int new_slot;         // slot receiving the new row
    int rows_per_split;   // whole blocks of kDecodeBlock rows plus at most 4 extra rows
    int n_split;
    int n_head_kv;
    int n_rep;            // q heads per kv head
    float scale;          // 1/sqrt(hd) as kore computes it (kore.cpp:1411)
    int wg_per_cu;        // split workgroups per CU: 1, or 2 when the grid has more than the CUs
};

// (cos, sin) of dims 0 .. hd/2 - 1 at the decode position, interleaved,
// built on the host (kore.cpp:1405-1410) and passed by value with the launch:
// a decode needs one row, so no device table has to cover its position (a
// ring decodes past ctx without bound).
constexpr int kMaxRopeHalf = 128;
struct RopeRow {
    float cs[2 * kMaxRopeHalf];
};

// Batched RoPE + append of n_tok rows starting at position pos0
// (kore.cpp:1535-1538).
struct AppendArgs {
    const float *k;       // [n_tok][n_head_kv][hd]
    const float *v;
    const float2 *cs;     // table base, row p = position p
    float *kc, *vc;       // layer base
    int slots;
    int pos0;
    int n_tok;
    int n_head_kv;
};

// Batched causal attention of n_tok query rows at positions pos0.. against
// cache rows [0, pos0 + n_tok) (kore.cpp:1542-1563).  q is pre-RoPE.
constexpr int kMaxPrefillUnits = 512;   // work units per kv-head of a split plan
struct PrefillArgs {
    const float *q;       // [n_tok][n_head][hd]
    const float2 *cs;     // table base
    const float *kc, *vc; // layer base
    float *out;           // [n_tok][n_head][hd]
    int slots;
    int pos0;
    int n_tok;
    int n_head_kv;
    int n_rep;
    int n_strips;         // ceil(n_tok / 32)
    float scale_log2;     // kore's 1/sqrt(hd) times log2(e)
    // Key segments: with n_kseg > 1 every workgroup item is split into
    // n_kseg launches over key tiles [seg * seg_tiles, (seg + 1) * seg_tiles)
    // that write unnormalised partials, merged by the prefill combine kernel.
    int n_kseg;
    int seg_tiles;
    float *part_o;        // [n_head_kv * n_rep * n_strips][n_kseg][32][hd]
    float *part_ml;       // [n_head_kv * n_rep * n_strips][n_kseg][32][2]
    // Workgroups b and b + fold (fold = CU count) usually share a CU: the
    // grid index is folded so that the second one runs the work list from
    // its short end (work index grid - 1 - (b - fold) for b >= fold).
    int fold;
    // Split plan (n_kseg == 1, between one and two workgroups per CU): items
    // 0 .. n_split - 1 of every kv-head (the longest) run as two workgroups
    // over the first and second half of their key tiles and write partials
    // [n_head_kv][n_split][4 waves][2 halves][32] (o, then max / sum), merged
    // by the prefill combine kernel; the other items run whole.  unit[r] is
    // the r-th longest of a kv-head's n_units work units, item << 2 | part
    // (part 0 whole, 1 first half, 2 second half); work index w runs unit
    // w / n_head_kv of kv-head w % n_head_kv, so the folded pairs of a CU
    // add up to about the same number of tiles.
    int n_split;
    int n_units;
    uint16_t unit[kMaxPrefillUnits];
};

// Any even head_dim up to kMaxGenericHeadDim and any n_rep (the geometries
// kore accepts, kore.cpp:1278-1290, that the MFMA kernels above do not
// cover): tiled attention on VALU with fp64 scores.  A workgroup takes `chunk`
// q-heads of one kv-head and one key range: a decode split of the cache rows
// (after a prep launch has roped q and appended the new row), or all keys
// 0..pos of one prefill row.
constexpr int kMaxGenericHeadDim = 2 * kMaxRopeHalf;
constexpr int kMaxGenericSplits = 128;   // decode splits per kv-head of the generic kernels
struct GenericArgs {
    const float *q;       // decode: roped q [n_head][hd]; prefill: pre-RoPE q [n_tok][n_head][hd]
    const float2 *cs;     // prefill: RoPE table (row p = position p); decode: null
    const float *kc, *vc; // layer base
    float *out;           // [n_tok][n_head][hd]
    float *part_o;        // decode with n_split > 1: [n_head][n_split][hd]
    float *part_ml;       //                          [n_head][n_split][2]
    int slots, hd, n_head_kv, n_rep;
    int chunk, n_chunks;  // q-heads per workgroup, workgroups per kv-head
    int tile;             // keys per LDS tile
    int pos0;             // prefill: position of row 0
    int n_rows;           // decode: cache rows attended, [0, n_rows), the new row included
    int rows_per_split, n_split;
    float scale;          // kore's 1/sqrt(hd) (kore.cpp:1411)
};
bool generic_supported(int head_dim);
// Launch shape of the generic kernels: tile, chunk and the split bound.
void generic_shape(int head_dim, int n_rep, int *tile, int *chunk, int *n_chunks);
int generic_max_split(int head_dim, int n_rep, int n_head_kv, int num_cu);
int generic_rows_per_split(int head_dim, int n_rep, int n_rows, int n_head_kv, int num_cu);
size_t generic_lds_bytes(int head_dim, int tile, int chunk);
// Decode: RoPE of q into q_out and of the new k row, append of k and v at
// new_slot, then the split attention and (n_split > 1) the merge.
hipError_t launch_generic_decode(const GenericArgs &a, const float *q, const float *k, const float *v,
                                 float *q_out, float *kc, float *vc, int n_head, int new_slot, const RopeRow &rr,
                                 hipStream_t s);
// Prefill rows after their append: grid (n_tok, n_head_kv * n_chunks).
hipError_t launch_generic_prefill(const GenericArgs &a, int n_tok, hipStream_t s);

// Counter-based synthetic inputs (identical bits to the CPU oracle's
// generator): dst[r*dim + c] for r < rows.
struct SynthArgs {
    float *dst;
    int rows, dim;
    uint64_t seed, stream, row0, tensor;
    uint32_t per_mille;
    float outlier_scale;
};

// The device's fixed scratch (a file-scope __device__ array of
// kStaticScratchFloats floats, 2.5 MiB): the split partials of the
// allocation-free decode entry point.  A decode has at most two split
// workgroups per CU and at most 8 q-heads per kv-head, so it needs at most
// 16 x num_cu x (hd + 2) floats: 532,480 on a 256-CU MI355X at head_dim 128.
// static_scratch() returns the array's address on `device` (made current by
// the caller), resolved with hipGetSymbolAddress on the first call for that
// device and remembered.
constexpr size_t kStaticScratchFloats = (size_t)5 << 17;
hipError_t static_scratch(int device, float **ptr);

// Rows per split the decode uses for n_rows cache rows (the host sizes the
// partial buffers from the maximum split count over all lengths).
int decode_rows_per_split(int head_dim, int n_rows, int n_head_kv, int num_cu);
// Geometries of the MFMA decode / prefill kernels; the others take the
// generic kernels.
bool decode_supported(int head_dim, int n_rep);
bool prefill_supported(int head_dim, int n_rep);

hipError_t launch_decode(const DecodeArgs &a, const RopeRow &rr, int head_dim, hipStream_t s);
hipError_t launch_append(const AppendArgs &a, int head_dim, hipStream_t s);
hipError_t launch_prefill(const PrefillArgs &a, int head_dim, hipStream_t s);
// Key segments the prefill uses for n_tok rows at pos0 (1 = none).
int prefill_key_segments(int n_tok, int pos0, int n_head_kv, int n_rep, int num_cu, int *seg_tiles);
// Fills a.n_split / a.n_units / a.unit for a chunk without key segments (its
// other fields set); n_split stays 0 where the plan does not apply.
void prefill_split_plan(PrefillArgs &a, int num_cu);
hipError_t launch_synth(const SynthArgs &a, hipStream_t s);

}  // namespace kore_attn_gpu
