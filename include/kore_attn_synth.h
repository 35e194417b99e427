/*
 * kore_attn_synth.h - synthetic inputs for benchmarks and tests of
 * libkore_attn.so.  Not part of the kore drop-in boundary (kore has no such
 * function): it fills device memory with the same counter-based values the
 * CPU test oracle generates, so that the GPU and CPU runs see identical
 * inputs without host-to-device copies of large arrays.
 *
 * Value of element (row, ch): the Irwin-Hall sum of twelve 24-bit uniforms
 * taken from splitmix64(key ^ (idx*8 + k)), k = 0..5 (bits 0..23 and 32..55
 * of each hash), idx = (row0 + row) * dim + ch, key =
 * splitmix64(splitmix64(seed) ^ stream), minus 6, times 2^-24: an
 * approximately N(0,1) fp32 value obtained by exact integer arithmetic and a
 * single rounding.  When per_mille > 0, channel ch is scaled by
 * outlier_scale if splitmix64(splitmix64(seed ^ 0x00571E50) ^ (tensor << 32)
 * ^ ch) % 1000 < per_mille.
 */
#ifndef KORE_ATTN_SYNTH_H
#define KORE_ATTN_SYNTH_H

#include <stdint.h>

#ifndef KORE_ATTN_API
#if defined(__GNUC__) || defined(__clang__)
#define KORE_ATTN_API __attribute__((visibility("default")))
#else
#define KORE_ATTN_API
#endif
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* dst: device pointer to rows*dim floats; stream: hipStream_t or NULL.
 * Asynchronous; 0 on success, KORE_ATTN_E_* otherwise. */
KORE_ATTN_API int kore_attn_synth_dev(float *dst, int rows, int dim, uint64_t seed, uint64_t stream_id,
                        uint64_t row0, uint64_t tensor, uint32_t per_mille, float outlier_scale,
                        void *stream);

#ifdef __cplusplus
}
#endif
#endif
