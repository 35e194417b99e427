// ref_qmv_harness.cpp - drives kore's own Q8_K activation quantisation and
// Q4_K / Q6_K x Q8_K dot products (scalar reference and AVX2) to record what
// they produce.  TEST INFRASTRUCTURE ONLY: built by oracle/Makefile (target
// `ref`) from the kore.cpp found at $(KORE_SRC) into oracle/_ref/kore_qmv_ref,
// and used to write the golden fixtures tests/golden/qmv_*.npz and to
// cross-check the C restatement (oracle/kore_qmv_oracle.c).
//
// Job file (little endian): int32 type (12 Q4_K, 14 Q6_K), rows, cols;
//   weights: rows * cols/256 blocks (144 or 210 bytes each), row-major;
//   x: cols float32.
// Result file: the Q8_K blocks of x (cols/256 x 292 bytes, kore's BlockQ8K),
//   then out_ref[rows], then out_avx2[rows] (float32; out_avx2 equals out_ref
//   where the CPU has no AVX2/FMA).

#define main kore_ref_main
#include "kore.cpp"
#undef main

#include <cstdio>
#include <vector>

int main(int argc, char **argv) {
    if (argc != 3) { fprintf(stderr, "usage: kore_qmv_ref job.bin result.bin\n"); return 2; }
    FILE *in = fopen(argv[1], "rb");
    FILE *out = fopen(argv[2], "wb");
    if (!in || !out) { perror("open"); return 2; }
    int32_t hdr[3];
    if (fread(hdr, 4, 3, in) != 3) return 3;
    const int type = hdr[0];
    const int64_t rows = hdr[1], cols = hdr[2];
    if (cols % 256 != 0 || (type != GGML_Q4_K && type != GGML_Q6_K)) return 3;
    const int64_t nb = cols / 256, bb = type == GGML_Q4_K ? 144 : 210;
    std::vector<uint8_t> w((size_t)(rows * nb * bb));
    std::vector<float> x((size_t)cols);
    if (fread(w.data(), 1, w.size(), in) != w.size()) return 3;
    if (fread(x.data(), 4, x.size(), in) != x.size()) return 3;
    std::vector<BlockQ8K> xq((size_t)nb);
    quantize_row_q8_K(x.data(), xq.data(), cols);
    std::vector<float> o_ref((size_t)rows), o_avx((size_t)rows);
    const bool avx2 = cpu_has_avx2();
    for (int64_t r = 0; r < rows; r++) {
        const uint8_t *wr = w.data() + r * nb * bb;
        if (type == GGML_Q4_K) {
            o_ref[(size_t)r] = dot_q4_K_q8_K_ref(cols, wr, xq.data());
            o_avx[(size_t)r] = avx2 ? dot_q4_K_q8_K_avx2(cols, wr, xq.data()) : o_ref[(size_t)r];
        } else {
            o_ref[(size_t)r] = dot_q6_K_q8_K_ref(cols, wr, xq.data());
            o_avx[(size_t)r] = avx2 ? dot_q6_K_q8_K_avx2(cols, wr, xq.data()) : o_ref[(size_t)r];
        }
    }
    if (fwrite(xq.data(), sizeof(BlockQ8K), xq.size(), out) != xq.size()) return 4;
    if (fwrite(o_ref.data(), 4, o_ref.size(), out) != o_ref.size()) return 4;
    if (fwrite(o_avx.data(), 4, o_avx.size(), out) != o_avx.size()) return 4;
    fclose(out);
    fclose(in);
    return avx2 ? 0 : 10;   // 10: no AVX2 on this CPU, out_avx2 is the scalar result
}
