/*
 * kore_qmv_synth.h - synthetic weight matrices for benchmarks and tests of
 * libkore_qmv.so.  Not part of the kore drop-in boundary (kore reads its
 * weights from a GGUF file): it writes GGUF-format Q4_K / Q6_K blocks
 * straight into device memory so that multi-gigabyte benchmark weights need
 * no host generation or upload.
 *
 * Every 16-bit word of the rows x (cols/256) blocks is bits 0..15 of
 * splitmix64(splitmix64(seed) ^ w), w the word's index in the buffer, except
 * the f16 scales: d (Q4_K word 0, Q6_K word 104 of a block) becomes
 * 0x1C00 | (h & 0x3FF) and dmin (Q4_K word 1) 0x1800 | (h & 0x3FF), h the
 * same hash, so every scale is finite.
 */
#ifndef KORE_QMV_SYNTH_H
#define KORE_QMV_SYNTH_H

#include <stdint.h>

#ifndef KORE_QMV_API
#if defined(__GNUC__) || defined(__clang__)
#define KORE_QMV_API __attribute__((visibility("default")))
#else
#define KORE_QMV_API
#endif
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* dst: device buffer of rows*(cols/256) blocks of 144 (Q4_K) or 210 (Q6_K)
 * bytes, 2-byte aligned; stream: hipStream_t or NULL.  Asynchronous. */
KORE_QMV_API int kore_qmv_synth_dev(int type, int64_t rows, int64_t cols, uint64_t seed, void *dst,
                                    void *stream);

#ifdef __cplusplus
}
#endif
#endif
