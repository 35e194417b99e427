// ref_layer_harness.cpp - drives kore's own forward() (kore.cpp:1397-1484) over
// layers with real Q4_K / Q6_K weights, norms and biases, to record what it
// produces.  TEST INFRASTRUCTURE ONLY: built by oracle/Makefile (target `ref`)
// from the kore.cpp found at $(KORE_SRC) into oracle/_ref/kore_layer_ref, and
// used to write tests/golden/layer_*.npz, which pin the oracle's composition
// of rmsnorm, quantisation, matvecs, biases, RoPE, attention, SwiGLU and the
// residual adds.
//
//   kore_layer_ref job.bin result.bin
//
// Job (little endian):
//   int32 n_layer, n_head, n_head_kv, head_dim, n_ff, ctx, avx2, n_steps;
//   float32 rope_base, rms_eps;
//   per layer: int32 types[7] (12 Q4_K / 14 Q6_K for wq wk wv wo w_gate w_up
//              w_down), float32 attn_norm[E], ffn_norm[E], bq[E], bk[kvd],
//              bv[kvd], then the 7 matrices' GGUF block bytes (rows x cols/256
//              blocks);
//   float32 emb[n_steps][E] (step s runs token s, whose embedding row is emb[s]);
//   int32 pos[n_steps].
// Result: float32 x[n_steps][E] (the residual after the last layer, kore's
//   e.x: forward() is called without logits), then the K and V caches
//   ([n_layer][ctx][kvd] each).
//
// GGUF mode (pins the loader and the whole token on a real file):
//   kore_layer_ref --gguf-forward file.gguf CTX_MAX TOKEN...
//   kore_layer_ref --gguf-forward-batch file.gguf CTX_MAX SPLIT TOKEN...
//   kore_layer_ref --time-batch THREADS SECONDS [RUNS]  (forward_batch() of 64-token
//   chunks at positions 0, 64, .., 448 on the synthetic 7B engine of --time)
// runs kore's load_model + engine_init(ctx_max, 4 threads, quantised path) and
// forward(token, pos, logits) for the tokens at positions 0, 1, ...; prints one
// JSON line {"ok", "ctx", "n_vocab", "avx2", "logits": [[...], ...]} (logits as
// the hex of their float bits), or {"ok": false} when kore refuses the file.
//
// Built with -DKORE_GPU_ATTN against the kore.cpp that oracle/make_kore_gpu.py
// writes (INTEGRATION.md's binding applied: RoPE, the KV cache and attention
// through libkore_attn.so), as oracle/_ref/kore_layer_gpu: the same modes then
// run kore's own forward() / forward_batch() with the attention on the GPU;
// the engines built here by hand get their attention handle from attach_gpu
// (engine_init does it for the GGUF modes), and the job mode reads the K/V
// rows back from the handle.
//
// Timing mode (the CPU baseline of the benchmark's whole-token leg):
//   kore_layer_ref --time THREADS MIN_SECONDS POS [RUNS]
// builds a Qwen2.5-7B-shape engine (28 layers, 3584 / 18944, 28 / 4 heads of
// 128, 152064-row Q6_K output head; Q4_K weights with attn_v and ffn_down in
// Q6_K on the layers Q4_K_M files keep them there) from synthetic block bytes,
// then runs kore's forward() with logits for tokens at positions POS, POS + 1,
// ... with THREADS threads until MIN_SECONDS have passed; prints one JSON line
// {"tokens", "seconds", "threads", "avx2", "pos"}.
#define main kore_ref_main
#include "kore.cpp"
#undef main

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

namespace {

bool rd(FILE *f, void *p, size_t n) { return fread(p, 1, n, f) == n; }
bool wr(FILE *f, const void *p, size_t n) { return fwrite(p, 1, n, f) == n; }

struct OwnedTensor {
    std::vector<uint8_t> bytes;
    Tensor t;
};

bool read_tensor(FILE *f, OwnedTensor &o, uint32_t type, uint64_t cols, uint64_t rows) {
    const uint64_t bb = type == GGML_Q4_K ? 144 : type == GGML_Q6_K ? 210 : type == GGML_F32 ? 1024 : 0;
    if (!bb || cols % 256) return false;
    o.bytes.resize(cols / 256 * bb * rows);
    o.t.type = type;
    o.t.n_dims = 2;
    o.t.dims[0] = cols;
    o.t.dims[1] = rows;
    o.t.nbytes = o.bytes.size();
    return rd(f, o.bytes.data(), o.bytes.size());
}

uint64_t mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// Hashed block bytes with f16 scales of a trained model's size (subnormal f16:
// Q4_K d 2.0e-5, dmin 5.0e-6; Q6_K d 4.0e-6).
void synth(OwnedTensor &o, uint32_t type, uint64_t cols, uint64_t rows, uint64_t seed) {
    const uint64_t bb = type == GGML_Q4_K ? 144 : 210;
    o.bytes.resize(cols / 256 * bb * rows);
    for (size_t i = 0; i < o.bytes.size(); i += 8) {
        const uint64_t r = mix64(seed * 0x100000001b3ull + i);
        memcpy(o.bytes.data() + i, &r, std::min<size_t>(8, o.bytes.size() - i));
    }
    for (size_t b = 0; b < o.bytes.size(); b += bb) {
        uint8_t *p = o.bytes.data() + b;
        if (type == GGML_Q4_K) { p[0] = 0x4F; p[1] = 0x01; p[2] = 0x54; p[3] = 0x00; }
        else { p[208] = 0x43; p[209] = 0x00; }
    }
    o.t.type = type;
    o.t.n_dims = 2;
    o.t.dims[0] = cols;
    o.t.dims[1] = rows;
    o.t.nbytes = o.bytes.size();
    o.t.data = o.bytes.data();
}

#ifdef KORE_GPU_ATTN
// The attention handle engine_init creates in the patched kore, for the
// engines built here without engine_init.
bool attach_gpu(Engine &e) {
    const Hparams &h = e.hp;
    if (kore_attn_create(&e.attn.h, (int)h.n_layer, e.ctx, (int)h.n_head, (int)h.n_head_kv, e.head_dim, h.rope_base,
                         0) != KORE_ATTN_OK) {
        fprintf(stderr, "attention: %s\n", kore_attn_last_error(nullptr));
        return false;
    }
    return true;
}
#endif

// "[a, b, ...]" of per-run values for the timing modes' JSON lines
std::string json_list(const std::vector<double> &v, const char *fmt) {
    std::string out = "[";
    char buf[64];
    for (size_t i = 0; i < v.size(); ++i) {
        snprintf(buf, sizeof buf, fmt, v[i]);
        out += (i ? ", " : "") + std::string(buf);
    }
    return out + "]";
}

int time_mode(unsigned nth, double min_s, int pos0, bool batch, int runs) {
    const int NL = 28, E = 3584, FF = 18944, NH = 28, NKV = 4, HD = 128, VOCAB = 152064;
    const int kvd = NKV * HD, ctx = batch ? 512 : pos0 + 256;
    Engine e;
    e.hp.n_layer = NL; e.hp.n_embd = E; e.hp.n_ff = FF; e.hp.n_head = NH; e.hp.n_head_kv = NKV;
    e.hp.n_ctx = (uint32_t)ctx; e.hp.n_vocab = VOCAB; e.hp.rope_base = 1e6f; e.hp.rms_eps = 1e-6f;
    e.head_dim = HD; e.kv_dim = kvd; e.n_rep = NH / NKV; e.ctx = ctx; e.n_vocab = VOCAB;
    e.nth = nth; e.use_float = false;
    e.avx2 = KORE_HAVE_AVX2 && cpu_has_avx2();
#ifdef KORE_GPU_ATTN
    if (!attach_gpu(e)) return 5;
#endif
    std::vector<OwnedTensor> mats((size_t)NL * 7);
    std::vector<float> ones((size_t)E, 1.0f), zeros((size_t)E, 0.0f);
    for (int l = 0; l < NL; l++) {
        const bool more = l < NL / 8 || l >= 7 * NL / 8 || (l - NL / 8) % 3 == 2;
        const uint32_t hi = more ? GGML_Q6_K : GGML_Q4_K;
        const uint32_t types[7] = {GGML_Q4_K, GGML_Q4_K, hi, GGML_Q4_K, GGML_Q4_K, GGML_Q4_K, hi};
        const uint64_t rows[7] = {(uint64_t)E, (uint64_t)kvd, (uint64_t)kvd, (uint64_t)E, (uint64_t)FF, (uint64_t)FF,
                                  (uint64_t)E};
        const uint64_t cols[7] = {(uint64_t)E, (uint64_t)E, (uint64_t)E, (uint64_t)E, (uint64_t)E, (uint64_t)E,
                                  (uint64_t)FF};
        OwnedTensor *m = &mats[(size_t)l * 7];
        for (int j = 0; j < 7; j++) synth(m[j], types[j], cols[j], rows[j], (uint64_t)l * 7 + j + 1);
        Layer L;
        L.wq = &m[0].t; L.wk = &m[1].t; L.wv = &m[2].t; L.wo = &m[3].t;
        L.w_gate = &m[4].t; L.w_up = &m[5].t; L.w_down = &m[6].t;
        L.attn_norm = ones.data(); L.ffn_norm = ones.data();
        L.bq = zeros.data(); L.bk = zeros.data(); L.bv = zeros.data();
        e.layers.push_back(L);
    }
    OwnedTensor head, tok;
    synth(head, GGML_Q6_K, (uint64_t)E, (uint64_t)VOCAB, 999);
    tok.bytes.assign((size_t)E * 4, 0);
    for (int i = 0; i < E; i++) { const float v = (float)((int)(mix64(7 + i) % 2001) - 1000) * 1e-3f; memcpy(&tok.bytes[(size_t)i * 4], &v, 4); }
    tok.t.type = GGML_F32; tok.t.n_dims = 2; tok.t.dims[0] = (uint64_t)E; tok.t.dims[1] = 1;
    tok.t.nbytes = tok.bytes.size(); tok.t.data = tok.bytes.data();
    e.tok_embd = &tok.t;
    e.out_w = &head.t;
    e.out_norm = ones.data();
    const int half = HD / 2;
    e.inv_freq.resize((size_t)half);
    for (int i = 0; i < half; i++) e.inv_freq[(size_t)i] = (float)std::pow((double)e.hp.rope_base, -2.0 * i / HD);
    e.rope_c.resize((size_t)half); e.rope_s.resize((size_t)half);
    e.kcache.assign((size_t)NL * ctx * kvd, 0.0f);
    e.vcache.assign((size_t)NL * ctx * kvd, 0.0f);
    e.emb.resize((size_t)E); e.x.resize((size_t)E); e.xb.resize((size_t)E); e.q.resize((size_t)E);
    e.att.resize((size_t)E); e.o.resize((size_t)E);
    e.k.resize((size_t)kvd); e.v.resize((size_t)kvd);
    e.gate.resize((size_t)FF); e.up.resize((size_t)FF);
    e.scores.resize((size_t)ctx); e.logits.resize((size_t)VOCAB);
    e.xq_e.resize((size_t)(E / 256 + 1)); e.xq_f.resize((size_t)FF / 256);
    e.scratch.resize((size_t)E);
    if (batch) {                                               // engine_init's batch buffers (kore.cpp:1354-1363)
        const size_t B = 64;
        e.bsz = 64;
        e.bemb.resize(B * E); e.bx.resize(B * E); e.bxb.resize(B * E); e.bq.resize(B * E); e.batt.resize(B * E);
        e.bo.resize(B * E); e.bk.resize(B * kvd); e.bv.resize(B * kvd); e.bgate.resize(B * FF); e.bup.resize(B * FF);
        e.bscores.resize(B * (size_t)ctx); e.bc_rope.resize(B * (size_t)half); e.bs_rope.resize(B * (size_t)half);
        e.bxt.resize(B * FF);
        std::vector<int> toks(B, 0);
        if (!forward_batch(e, toks.data(), 64, 0, true)) return 5;   // warm-up
        int chunks = 0;
        double el = 0;
        std::vector<double> run_chunks, run_s;
        for (int run = 0; run < runs; ++run) {                 // RUNS timed runs of at least MIN_SECONDS
            int c = 0;
            double t = 0;
            const auto t0 = std::chrono::steady_clock::now();
            do {                                               // 64-token chunks at 0, 64, .., 448 in turn;
                // logits after the 8-chunk prompt's last chunk (kore's prefill loop, kore.cpp:1729-1730)
                if (!forward_batch(e, toks.data(), 64, 64 * (c % 8), c % 8 == 7)) return 5;
                ++c;
                t = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
            } while (t < min_s);
            run_chunks.push_back(c);
            run_s.push_back(t);
            chunks += c;
            el += t;
        }
        printf("{\"tokens\": %d, \"chunks\": %d, \"seconds\": %.6f, \"threads\": %u, \"avx2\": %d, "
               "\"checksum\": %.9g, \"run_chunks\": %s, \"run_seconds\": %s}\n", chunks * 64, chunks, el, nth,
               (int)e.avx2, (double)e.logits[(size_t)VOCAB / 2], json_list(run_chunks, "%.0f").c_str(),
               json_list(run_s, "%.6f").c_str());
        return 0;
    }
    if (!forward(e, 0, pos0, true)) return 5;                  // warm-up
    int tokens = 0;
    double el = 0;
    std::vector<double> run_tokens, run_s;
    for (int run = 0; run < runs; ++run) {                     // RUNS timed runs of at least MIN_SECONDS
        int n = 0;
        double t = 0;
        const auto t0 = std::chrono::steady_clock::now();
        do {
            if (!forward(e, 0, pos0 + 1 + tokens % 200, true)) return 5;
            ++tokens;
            ++n;
            t = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        } while (t < min_s);
        run_tokens.push_back(n);
        run_s.push_back(t);
        el += t;
    }
    printf("{\"tokens\": %d, \"seconds\": %.6f, \"threads\": %u, \"avx2\": %d, \"pos\": %d, \"checksum\": %.9g, "
           "\"run_tokens\": %s, \"run_seconds\": %s}\n",
           tokens, el, nth, (int)e.avx2, pos0, (double)e.logits[(size_t)VOCAB / 2], json_list(run_tokens, "%.0f").c_str(),
           json_list(run_s, "%.6f").c_str());
    return 0;
}

}  // namespace

int gguf_forward(const char *path, int ctx_max, int n, char **toks) {
    Model m;
    Engine e;
    if (!load_model(path, m) || !engine_init(e, m, ctx_max, 4, false)) {
        printf("{\"ok\": false}\n");
        return 0;
    }
    printf("{\"ok\": true, \"ctx\": %d, \"n_vocab\": %d, \"avx2\": %d, \"logits\": [", e.ctx, e.n_vocab, (int)e.avx2);
    for (int i = 0; i < n; ++i) {
        if (!forward(e, atoi(toks[i]), i, true)) { printf("]}\n"); return 5; }
        printf("%s[", i ? ", " : "");
        for (int v = 0; v < e.n_vocab; ++v) {
            uint32_t u;
            memcpy(&u, &e.logits[(size_t)v], 4);
            printf("%s\"%08x\"", v ? ", " : "", u);
        }
        printf("]");
    }
    printf("]}\n");
    return 0;
}

// kore_layer_ref --gguf-forward-batch file.gguf CTX_MAX SPLIT TOKEN...: kore's
// forward_batch() over the tokens in two chunks, [0, SPLIT) at position 0
// without logits and the rest at position SPLIT with logits; prints the last
// chunk's residual rows (e.bx) and the logits as float bit patterns.
int gguf_forward_batch(const char *path, int ctx_max, int split, int n, char **toks) {
    Model m;
    Engine e;
    if (!load_model(path, m) || !engine_init(e, m, ctx_max, 4, false)) {
        printf("{\"ok\": false}\n");
        return 0;
    }
    std::vector<int> t((size_t)n);
    for (int i = 0; i < n; ++i) t[(size_t)i] = atoi(toks[i]);
    if (split <= 0 || split >= n || !forward_batch(e, t.data(), split, 0, false) ||
        !forward_batch(e, t.data() + split, n - split, split, true)) {
        printf("{\"ok\": false}\n");
        return 0;
    }
    auto hex = [](const float *a, size_t k) {
        for (size_t i = 0; i < k; ++i) {
            uint32_t u;
            memcpy(&u, a + i, 4);
            printf("%s\"%08x\"", i ? ", " : "", u);
        }
    };
    printf("{\"ok\": true, \"ctx\": %d, \"bsz\": %d, \"avx2\": %d, \"x\": [", e.ctx, e.bsz, (int)e.avx2);
    hex(e.bx.data(), (size_t)(n - split) * m.hp.n_embd);
    printf("], \"logits\": [");
    hex(e.logits.data(), (size_t)e.n_vocab);
    printf("]}\n");
    return 0;
}

int main(int argc, char **argv) {
    if (argc >= 6 && std::string(argv[1]) == "--gguf-forward-batch")
        return gguf_forward_batch(argv[2], atoi(argv[3]), atoi(argv[4]), argc - 5, argv + 5);
    if (argc >= 4 && std::string(argv[1]) == "--gguf-forward")
        return gguf_forward(argv[2], atoi(argv[3]), argc - 4, argv + 4);
    if ((argc == 5 || argc == 6) && std::string(argv[1]) == "--time")
        return time_mode((unsigned)atoi(argv[2]), atof(argv[3]), atoi(argv[4]), false,
                         argc == 6 ? std::max(1, atoi(argv[5])) : 1);
    if ((argc == 4 || argc == 5) && std::string(argv[1]) == "--time-batch")
        return time_mode((unsigned)atoi(argv[2]), atof(argv[3]), 0, true, argc == 5 ? std::max(1, atoi(argv[4])) : 1);
    if (argc != 3) { fprintf(stderr, "usage: kore_layer_ref job.bin result.bin | --time THREADS SECONDS POS\n"); return 2; }
    FILE *in = fopen(argv[1], "rb");
    FILE *out = fopen(argv[2], "wb");
    if (!in || !out) { perror("open"); return 2; }
    int32_t hdr[8];
    float fp[2];
    if (!rd(in, hdr, sizeof hdr) || !rd(in, fp, sizeof fp)) return 3;
    const int n_layer = hdr[0], nh = hdr[1], nkv = hdr[2], hd = hdr[3], FF = hdr[4], ctx = hdr[5];
    const int avx2 = hdr[6], n_steps = hdr[7];
    const int E = nh * hd, kvd = nkv * hd;
    if (E % 256 || FF % 256 || nh % nkv || n_steps < 1) return 3;

    Engine e;
    e.hp.n_layer = (uint32_t)n_layer; e.hp.n_embd = (uint32_t)E; e.hp.n_ff = (uint32_t)FF;
    e.hp.n_head = (uint32_t)nh; e.hp.n_head_kv = (uint32_t)nkv; e.hp.n_ctx = (uint32_t)ctx;
    e.hp.n_vocab = (uint32_t)n_steps; e.hp.rope_base = fp[0]; e.hp.rms_eps = fp[1];
    e.head_dim = hd; e.kv_dim = kvd; e.n_rep = nh / nkv; e.ctx = ctx; e.n_vocab = n_steps;
    e.nth = 4; e.use_float = false;
    e.avx2 = KORE_HAVE_AVX2 && cpu_has_avx2() && avx2;
#ifdef KORE_GPU_ATTN
    if (!attach_gpu(e)) return 5;
#endif

    std::vector<std::vector<float>> vecs((size_t)n_layer * 5);
    std::vector<OwnedTensor> mats((size_t)n_layer * 7);
    const uint64_t rows_of[7] = {(uint64_t)E, (uint64_t)kvd, (uint64_t)kvd, (uint64_t)E, (uint64_t)FF, (uint64_t)FF,
                                 (uint64_t)E};
    const uint64_t cols_of[7] = {(uint64_t)E, (uint64_t)E, (uint64_t)E, (uint64_t)E, (uint64_t)E, (uint64_t)E,
                                 (uint64_t)FF};
    for (int l = 0; l < n_layer; l++) {
        int32_t types[7];
        if (!rd(in, types, sizeof types)) return 3;
        const size_t sizes[5] = {(size_t)E, (size_t)E, (size_t)E, (size_t)kvd, (size_t)kvd};
        for (int j = 0; j < 5; j++) {
            std::vector<float> &v = vecs[(size_t)l * 5 + j];
            v.resize(sizes[j]);
            if (!rd(in, v.data(), v.size() * 4)) return 3;
        }
        for (int j = 0; j < 7; j++)
            if (!read_tensor(in, mats[(size_t)l * 7 + j], (uint32_t)types[j], cols_of[j], rows_of[j])) return 3;
    }
    OwnedTensor tok;
    tok.bytes.resize((size_t)n_steps * E * 4);
    if (!rd(in, tok.bytes.data(), tok.bytes.size())) return 3;
    tok.t.type = GGML_F32; tok.t.n_dims = 2; tok.t.dims[0] = (uint64_t)E; tok.t.dims[1] = (uint64_t)n_steps;
    tok.t.nbytes = tok.bytes.size(); tok.t.data = tok.bytes.data();
    std::vector<int32_t> pos((size_t)n_steps);
    if (!rd(in, pos.data(), pos.size() * 4)) return 3;

    std::vector<float> ones((size_t)E, 1.0f);
    e.tok_embd = &tok.t;
    e.out_norm = ones.data();
    for (int l = 0; l < n_layer; l++) {
        OwnedTensor *m = &mats[(size_t)l * 7];
        for (int j = 0; j < 7; j++) m[j].t.data = m[j].bytes.data();
        Layer L;
        L.wq = &m[0].t; L.wk = &m[1].t; L.wv = &m[2].t; L.wo = &m[3].t;
        L.w_gate = &m[4].t; L.w_up = &m[5].t; L.w_down = &m[6].t;
        std::vector<float> *v = &vecs[(size_t)l * 5];
        L.attn_norm = v[0].data(); L.ffn_norm = v[1].data();
        L.bq = v[2].data(); L.bk = v[3].data(); L.bv = v[4].data();
        e.layers.push_back(L);
    }

    // Buffer sizes as engine_init gives them (kore.cpp:1336-1363).
    const int half = hd / 2;
    e.inv_freq.resize((size_t)half);
    for (int i = 0; i < half; i++) e.inv_freq[(size_t)i] = (float)std::pow((double)e.hp.rope_base, -2.0 * i / hd);
    e.rope_c.resize((size_t)half); e.rope_s.resize((size_t)half);
    e.kcache.assign((size_t)n_layer * ctx * kvd, 0.0f);
    e.vcache.assign((size_t)n_layer * ctx * kvd, 0.0f);
    e.emb.resize((size_t)E); e.x.resize((size_t)E); e.xb.resize((size_t)E); e.q.resize((size_t)E);
    e.att.resize((size_t)E); e.o.resize((size_t)E);
    e.k.resize((size_t)kvd); e.v.resize((size_t)kvd);
    e.gate.resize((size_t)FF); e.up.resize((size_t)FF);
    e.scores.resize((size_t)ctx); e.logits.resize(1);
    e.xq_e.resize((size_t)(E / 256 + 1)); e.xq_f.resize((size_t)FF / 256);
    e.scratch.resize((size_t)E);

    for (int st = 0; st < n_steps; st++) {
        if (!forward(e, st, pos[(size_t)st], false)) { fprintf(stderr, "forward failed at step %d\n", st); return 5; }
        if (!wr(out, e.x.data(), sizeof(float) * E)) return 6;
    }
#ifdef KORE_GPU_ATTN
    for (int l = 0; l < n_layer; l++)   // the cache lives on the GPU: kore's layout back
        if (kore_attn_read_kv(e.attn.h, l, 0, ctx, e.kcache.data() + (size_t)l * ctx * kvd,
                              e.vcache.data() + (size_t)l * ctx * kvd) != KORE_ATTN_OK)
            return 6;
#endif
    if (!wr(out, e.kcache.data(), sizeof(float) * e.kcache.size()) ||
        !wr(out, e.vcache.data(), sizeof(float) * e.vcache.size())) return 6;
    fclose(out);
    fclose(in);
    return 0;
}
