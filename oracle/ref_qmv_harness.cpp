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
//
// Batch mode (kore's matmul_batch_float, kore.cpp:783-845):
//   kore_qmv_ref --batch job.bin result.bin
// job: int32 type, rows, cols, B; the weights; x as B rows of cols float32.
// result: out[b * rows + r] of the AVX2 path, then of the scalar path (the
// AVX2 one equals the scalar one where the CPU has no AVX2/FMA).
//
// Timing mode (the CPU baseline of the benchmark):
//   kore_qmv_ref --time THREADS MIN_SECONDS COPIES job.bin [RUNS]
// keeps COPIES copies of the job's matrix (so that the weights streamed exceed
// the host's caches, as a model's do) and runs kore's own quant() + mv() pair
// on them in turn - quantize_row_q8_K then matvec_mt over all rows with
// THREADS threads and the AVX2 dot products where the CPU has them
// (kore.cpp:1387-1394, 677-682) - until MIN_SECONDS have passed; prints one
// JSON line {"reps", "seconds", "rows", "cols", "weight_bytes", "avx2",
// "threads", "copies", "run_reps", "run_seconds"} (RUNS timed runs of at least
// MIN_SECONDS each, default 1; the totals sum them).
//
//   kore_qmv_ref --gguf file.gguf
// runs kore's load_model (kore.cpp:188-285) on the file and prints one JSON
// line: {"ok", "hp": {...}, "data_start", "tensors": [{"name", "type",
// "n_dims", "dims", "nbytes", "has_data", "fnv"}...]} with the tensors sorted
// by name and fnv the 64-bit FNV-1a hash of the nbytes bytes the tensor points
// to (kore's stderr messages pass through).
//
//   kore_qmv_ref --time-batch THREADS MIN_SECONDS job.bin [RUNS]
// takes a batch-mode job and runs kore's matmul_batch_float on it with
// THREADS threads and the AVX2 path where the CPU has it (as forward_batch()
// calls it, kore.cpp:1524) until MIN_SECONDS have passed; prints one JSON line
// {"reps", "seconds", "rows", "cols", "B", "avx2", "threads", "run_reps",
// "run_seconds"} (RUNS timed runs as in --time).

#define main kore_ref_main
#include "kore.cpp"
#undef main

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <string>
#include <vector>

// "[a, b, ...]" of per-run values for the timing modes' JSON lines
static std::string json_list(const std::vector<double> &v, const char *fmt) {
    std::string out = "[";
    char buf[64];
    for (size_t i = 0; i < v.size(); ++i) {
        snprintf(buf, sizeof buf, fmt, v[i]);
        out += (i ? ", " : "") + std::string(buf);
    }
    return out + "]";
}

static int time_mode(unsigned nth, double min_s, int copies, const char *job, int runs) {
    FILE *in = fopen(job, "rb");
    if (!in) { perror("open"); return 2; }
    int32_t hdr[3];
    if (fread(hdr, 4, 3, in) != 3) return 3;
    const int type = hdr[0];
    const int64_t rows = hdr[1], cols = hdr[2];
    if (cols % 256 != 0 || (type != GGML_Q4_K && type != GGML_Q6_K)) return 3;
    const int64_t nb = cols / 256, bb = type == GGML_Q4_K ? 144 : 210;
    if (copies < 1) copies = 1;
    const size_t wb = (size_t)(rows * nb * bb);
    std::vector<std::vector<uint8_t>> w((size_t)copies, std::vector<uint8_t>(wb));
    std::vector<float> x((size_t)cols), out((size_t)rows);
    if (fread(w[0].data(), 1, wb, in) != wb) return 3;
    if (fread(x.data(), 4, x.size(), in) != x.size()) return 3;
    fclose(in);
    for (int c = 1; c < copies; ++c) memcpy(w[(size_t)c].data(), w[0].data(), wb);
    std::vector<Tensor> t((size_t)copies);
    for (int c = 0; c < copies; ++c) {
        t[(size_t)c].type = (uint32_t)type;
        t[(size_t)c].n_dims = 2;
        t[(size_t)c].dims[0] = (uint64_t)cols;
        t[(size_t)c].dims[1] = (uint64_t)rows;
        t[(size_t)c].nbytes = wb;
        t[(size_t)c].data = w[(size_t)c].data();
    }
    std::vector<BlockQ8K> xq((size_t)nb);
    const bool avx2 = cpu_has_avx2();
    for (int c = 0; c < copies; ++c) {   // warm-up: touch every copy once
        quantize_row_q8_K(x.data(), xq.data(), cols);
        matvec_mt(t[(size_t)c], xq.data(), out.data(), avx2, nth);
    }
    // RUNS timed runs of at least MIN_SECONDS each (kore_kernels times best-of-N)
    int reps = 0, k = 0;
    double el = 0;
    std::vector<double> run_reps, run_s;
    for (int run = 0; run < runs; ++run) {
        int r = 0;
        double e = 0;
        const auto t0 = std::chrono::steady_clock::now();
        do {
            quantize_row_q8_K(x.data(), xq.data(), cols);
            matvec_mt(t[(size_t)(k++ % copies)], xq.data(), out.data(), avx2, nth);
            ++r;
            e = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        } while (e < min_s);
        run_reps.push_back(r);
        run_s.push_back(e);
        reps += r;
        el += e;
    }
    printf("{\"reps\": %d, \"seconds\": %.6f, \"rows\": %lld, \"cols\": %lld, \"weight_bytes\": %zu, "
           "\"avx2\": %d, \"threads\": %u, \"copies\": %d, \"checksum\": %.9g, \"run_reps\": %s, "
           "\"run_seconds\": %s}\n",
           reps, el, (long long)rows, (long long)cols, wb, (int)avx2, nth, copies, (double)out[(size_t)rows / 2],
           json_list(run_reps, "%.0f").c_str(), json_list(run_s, "%.6f").c_str());
    return 0;
}

struct BatchJob {
    int type = 0, B = 0;
    int64_t rows = 0, cols = 0;
    std::vector<uint8_t> w;
    std::vector<float> x;
    Tensor t;
};

static int read_batch_job(const char *job, BatchJob &j) {
    FILE *in = fopen(job, "rb");
    if (!in) { perror("open"); return 2; }
    int32_t hdr[4];
    if (fread(hdr, 4, 4, in) != 4) return 3;
    j.type = hdr[0];
    j.B = hdr[3];
    j.rows = hdr[1];
    j.cols = hdr[2];
    if (j.cols % 256 != 0 || (j.type != GGML_Q4_K && j.type != GGML_Q6_K) || j.B <= 0 || j.B > KORE_BMAX) return 3;
    const int64_t nb = j.cols / 256, bb = j.type == GGML_Q4_K ? 144 : 210;
    j.w.resize((size_t)(j.rows * nb * bb));
    j.x.resize((size_t)(j.B * j.cols));
    if (fread(j.w.data(), 1, j.w.size(), in) != j.w.size()) return 3;
    if (fread(j.x.data(), 4, j.x.size(), in) != j.x.size()) return 3;
    fclose(in);
    j.t.type = (uint32_t)j.type;
    j.t.n_dims = 2;
    j.t.dims[0] = (uint64_t)j.cols;
    j.t.dims[1] = (uint64_t)j.rows;
    j.t.nbytes = j.w.size();
    j.t.data = j.w.data();
    return 0;
}

static int time_batch_mode(unsigned nth, double min_s, const char *job, int runs) {
    BatchJob j;
    if (int rc = read_batch_job(job, j)) return rc;
    const int B8 = (j.B + 7) & ~7;
    std::vector<float> xT((size_t)(j.cols * B8)), o((size_t)(j.rows * j.B));
    const bool avx2 = cpu_has_avx2();
    matmul_batch_float(j.t, j.x.data(), j.B, xT.data(), o.data(), avx2, nth);   // warm-up
    int reps = 0;
    double el = 0;
    std::vector<double> run_reps, run_s;
    for (int run = 0; run < runs; ++run) {
        int r = 0;
        double e = 0;
        const auto t0 = std::chrono::steady_clock::now();
        do {
            matmul_batch_float(j.t, j.x.data(), j.B, xT.data(), o.data(), avx2, nth);
            ++r;
            e = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        } while (e < min_s);
        run_reps.push_back(r);
        run_s.push_back(e);
        reps += r;
        el += e;
    }
    printf("{\"reps\": %d, \"seconds\": %.6f, \"rows\": %lld, \"cols\": %lld, \"B\": %d, \"avx2\": %d, "
           "\"threads\": %u, \"checksum\": %.9g, \"run_reps\": %s, \"run_seconds\": %s}\n",
           reps, el, (long long)j.rows, (long long)j.cols, j.B, (int)avx2, nth, (double)o[o.size() / 2],
           json_list(run_reps, "%.0f").c_str(), json_list(run_s, "%.6f").c_str());
    return 0;
}

static int batch_mode(const char *job, const char *res) {
    BatchJob j;
    if (int rc = read_batch_job(job, j)) return rc;
    FILE *out = fopen(res, "wb");
    if (!out) { perror("open"); return 2; }
    const int B8 = (j.B + 7) & ~7;
    std::vector<float> xT((size_t)(j.cols * B8)), o1((size_t)(j.rows * j.B)), o2((size_t)(j.rows * j.B));
    const bool avx2 = cpu_has_avx2();
    matmul_batch_float(j.t, j.x.data(), j.B, xT.data(), o1.data(), avx2, 1);
    matmul_batch_float(j.t, j.x.data(), j.B, xT.data(), o2.data(), false, 1);
    if (fwrite(o1.data(), 4, o1.size(), out) != o1.size()) return 4;
    if (fwrite(o2.data(), 4, o2.size(), out) != o2.size()) return 4;
    fclose(out);
    return avx2 ? 0 : 10;
}

static int gguf_mode(const char *path) {
    Model m;
    const bool ok = load_model(path, m);
    printf("{\"ok\": %s", ok ? "true" : "false");
    if (ok) {
        const Hparams &h = m.hp;
        printf(", \"hp\": {\"n_layer\": %u, \"n_embd\": %u, \"n_ff\": %u, \"n_head\": %u, \"n_head_kv\": %u, "
               "\"n_ctx\": %u, \"n_vocab\": %u, \"rope_base\": %.9g, \"rms_eps\": %.9g}, \"data_start\": %llu, "
               "\"tensors\": [",
               h.n_layer, h.n_embd, h.n_ff, h.n_head, h.n_head_kv, h.n_ctx, h.n_vocab, (double)h.rope_base,
               (double)h.rms_eps, (unsigned long long)m.data_start);
        std::vector<std::string> names;
        for (const auto &kv : m.tensors) names.push_back(kv.first);
        std::sort(names.begin(), names.end());
        for (size_t i = 0; i < names.size(); ++i) {
            const Tensor &t = m.tensors.at(names[i]);
            uint64_t fnv = 0xcbf29ce484222325ull;
            if (t.data)
                for (uint64_t b = 0; b < t.nbytes; ++b) fnv = (fnv ^ t.data[b]) * 0x100000001b3ull;
            printf("%s{\"name\": \"%s\", \"type\": %u, \"n_dims\": %u, \"dims\": [%llu, %llu, %llu, %llu], "
                   "\"nbytes\": %llu, \"has_data\": %s, \"fnv\": \"%016llx\"}",
                   i ? ", " : "", names[i].c_str(), t.type, t.n_dims, (unsigned long long)t.dims[0],
                   (unsigned long long)t.dims[1], (unsigned long long)t.dims[2], (unsigned long long)t.dims[3],
                   (unsigned long long)t.nbytes, t.data ? "true" : "false", (unsigned long long)fnv);
        }
        printf("]");
    }
    printf("}\n");
    return 0;
}

int main(int argc, char **argv) {
    if (argc == 3 && std::string(argv[1]) == "--gguf") return gguf_mode(argv[2]);
    if (argc == 4 && std::string(argv[1]) == "--batch") return batch_mode(argv[2], argv[3]);
    if ((argc == 5 || argc == 6) && std::string(argv[1]) == "--time-batch")
        return time_batch_mode((unsigned)atoi(argv[2]), atof(argv[3]), argv[4], argc == 6 ? std::max(1, atoi(argv[5])) : 1);
    if ((argc == 6 || argc == 7) && std::string(argv[1]) == "--time")
        return time_mode((unsigned)atoi(argv[2]), atof(argv[3]), atoi(argv[4]), argv[5],
                         argc == 7 ? std::max(1, atoi(argv[6])) : 1);
    if (argc != 3) {
        fprintf(stderr, "usage: kore_qmv_ref job.bin result.bin | --batch job.bin result.bin | --time THREADS SECONDS COPIES "
                        "job.bin | --time-batch THREADS SECONDS job.bin\n");
        return 2;
    }
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
