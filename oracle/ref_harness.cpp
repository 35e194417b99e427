// ref_harness.cpp - drives kore's own forward()/forward_batch() to record what
// its RoPE / KV-append / attention code produces.  TEST INFRASTRUCTURE ONLY:
// built by oracle/Makefile (target `ref`) from the kore.cpp found at
// $(KORE_SRC) into oracle/_ref/kore_ref, and used to write the golden
// fixtures under tests/golden/ and to cross-check the C restatement.
//
// How kore's inline attention is isolated (kore.cpp:1397-1598):
//   * every weight tensor is zero, so the QKV projections return exact +0 and
//     q/k/v equal the layer biases bq/bk/bv bit for bit (kore.cpp:1419-1423,
//     1524-1534); the caller sets the biases per step;
//   * the attention output is zero-projected by Wo, so x stays zero and every
//     layer sees exactly its own biases;
//   * decode runs forward() with use_float (F32 zero weights, kore.cpp:1409,
//     849-861); prefill runs forward_batch() on zero Q4_K weights so the
//     batched AVX2 (or scalar, with avx2 forced off) attention is taken.
// After each call kore's own buffers hold the result: e.att / e.batt (last
// layer's attention), e.q / e.bq (last layer's roped q), e.kcache/e.vcache.
// engine_init (kore.cpp:1275) is not called because it rejects n_embd % 256
// (kore.cpp:1283) which the 0.5B geometry needs; the harness sizes kore's
// Engine buffers itself, to the sizes engine_init gives them.
//
// Job file (little endian):
//   int32 mode (0 decode, 1 prefill), n_layer, n_head, n_head_kv, head_dim,
//         ctx, avx2 (prefill: 1 = AVX2 helpers, 0 = scalar), n_steps
//   float rope_base
//   per step: int32 pos, int32 nb; per layer: q[E], k[kvd], v[kvd]
// Result file: per step: att[nb][E], q_roped[nb][E] (last layer);
//   then kcache, vcache ([n_layer][ctx][kvd]), inv_freq[hd/2].

#define main kore_ref_main
#include "kore.cpp"
#undef main

#include <cstdio>
#include <vector>

namespace {

struct ZeroTensor {
    std::vector<uint8_t> bytes;
    Tensor t;
};

ZeroTensor make_zero(uint32_t type, uint64_t cols, uint64_t rows) {
    ZeroTensor z;
    uint64_t nbytes = 0;
    if (type == GGML_F32) nbytes = cols * rows * 4;
    else nbytes = cols / 256 * 144 * rows;   // Q4_K block: 144 bytes per 256 values
    z.bytes.assign(nbytes ? nbytes : 4, 0);
    z.t.type = type;
    z.t.n_dims = 2;
    z.t.dims[0] = cols;
    z.t.dims[1] = rows;
    z.t.nbytes = nbytes;
    return z;
}

bool rd(FILE *f, void *p, size_t n) { return fread(p, 1, n, f) == n; }
bool wr(FILE *f, const void *p, size_t n) { return fwrite(p, 1, n, f) == n; }

}  // namespace

int main(int argc, char **argv) {
    if (argc != 3) { fprintf(stderr, "usage: kore_ref job.bin result.bin\n"); return 2; }
    FILE *in = fopen(argv[1], "rb");
    FILE *out = fopen(argv[2], "wb");
    if (!in || !out) { perror("open"); return 2; }
    int32_t hdr[8];
    float rope_base;
    if (!rd(in, hdr, sizeof hdr) || !rd(in, &rope_base, 4)) return 3;
    const int mode = hdr[0], n_layer = hdr[1], nh = hdr[2], nkv = hdr[3], hd = hdr[4];
    const int ctx = hdr[5], avx2 = hdr[6], n_steps = hdr[7];
    const int E = nh * hd, kvd = nkv * hd, FF = 256;
    const bool use_float = (mode == 0);
    if (!use_float && (E % 256 != 0)) { fprintf(stderr, "prefill needs E %% 256 == 0\n"); return 3; }

    Engine e;
    e.hp.n_layer = (uint32_t)n_layer; e.hp.n_embd = (uint32_t)E; e.hp.n_ff = FF;
    e.hp.n_head = (uint32_t)nh; e.hp.n_head_kv = (uint32_t)nkv; e.hp.n_ctx = (uint32_t)ctx;
    e.hp.n_vocab = 1; e.hp.rope_base = rope_base; e.hp.rms_eps = 1e-6f;
    e.head_dim = hd; e.kv_dim = kvd; e.n_rep = nh / nkv; e.ctx = ctx; e.n_vocab = 1;
    e.nth = 4; e.use_float = use_float;
    e.avx2 = KORE_HAVE_AVX2 && cpu_has_avx2() && (use_float || avx2);

    const uint32_t wtype = use_float ? GGML_F32 : GGML_Q4_K;
    ZeroTensor tok = make_zero(GGML_F32, (uint64_t)E, 1);
    std::vector<ZeroTensor> w;   // per layer: wq wk wv wo gate up down
    w.reserve((size_t)n_layer * 7);
    std::vector<float> ones((size_t)E, 1.0f);
    std::vector<std::vector<float>> bias((size_t)n_layer * 3);
    e.tok_embd = &tok.t;
    e.out_norm = ones.data();
    for (int l = 0; l < n_layer; l++) {
        const size_t base = w.size();
        w.push_back(make_zero(wtype, (uint64_t)E, (uint64_t)E));     // wq
        w.push_back(make_zero(wtype, (uint64_t)E, (uint64_t)kvd));   // wk
        w.push_back(make_zero(wtype, (uint64_t)E, (uint64_t)kvd));   // wv
        w.push_back(make_zero(wtype, (uint64_t)E, (uint64_t)E));     // wo
        w.push_back(make_zero(wtype, (uint64_t)E, (uint64_t)FF));    // gate
        w.push_back(make_zero(wtype, (uint64_t)E, (uint64_t)FF));    // up
        w.push_back(make_zero(wtype, (uint64_t)FF, (uint64_t)E));    // down
        bias[(size_t)l * 3 + 0].assign((size_t)E, 0.0f);
        bias[(size_t)l * 3 + 1].assign((size_t)kvd, 0.0f);
        bias[(size_t)l * 3 + 2].assign((size_t)kvd, 0.0f);
        (void)base;
    }
    for (int l = 0; l < n_layer; l++) {
        ZeroTensor *lw = &w[(size_t)l * 7];
        for (int j = 0; j < 7; j++) lw[j].t.data = lw[j].bytes.data();
        Layer L;
        L.wq = &lw[0].t; L.wk = &lw[1].t; L.wv = &lw[2].t; L.wo = &lw[3].t;
        L.w_gate = &lw[4].t; L.w_up = &lw[5].t; L.w_down = &lw[6].t;
        L.attn_norm = ones.data(); L.ffn_norm = ones.data();
        L.bq = bias[(size_t)l * 3 + 0].data();
        L.bk = bias[(size_t)l * 3 + 1].data();
        L.bv = bias[(size_t)l * 3 + 2].data();
        e.layers.push_back(L);
    }
    tok.t.data = tok.bytes.data();

    // Buffer sizes as engine_init gives them (kore.cpp:1336-1363).
    const int half = hd / 2;
    e.inv_freq.resize((size_t)half);
    for (int i = 0; i < half; i++) e.inv_freq[(size_t)i] = (float)std::pow((double)rope_base, -2.0 * i / hd);
    e.rope_c.resize((size_t)half); e.rope_s.resize((size_t)half);
    e.kcache.assign((size_t)n_layer * ctx * kvd, 0.0f);
    e.vcache.assign((size_t)n_layer * ctx * kvd, 0.0f);
    e.emb.resize((size_t)E); e.x.resize((size_t)E); e.xb.resize((size_t)E); e.q.resize((size_t)E);
    e.att.resize((size_t)E); e.o.resize((size_t)E);
    e.k.resize((size_t)kvd); e.v.resize((size_t)kvd);
    e.gate.resize(FF); e.up.resize(FF);
    e.scores.resize((size_t)ctx); e.logits.resize(1);
    e.xq_e.resize((size_t)(E / 256 + 1)); e.xq_f.resize(FF / 256);
    e.bsz = std::min(KORE_BMAX, ctx);
    const size_t bsz = (size_t)e.bsz;
    e.scratch.resize((size_t)E);
    e.bemb.resize(bsz * E); e.bx.resize(bsz * E); e.bxb.resize(bsz * E);
    e.bq.resize(bsz * E); e.batt.resize(bsz * E); e.bo.resize(bsz * E);
    e.bk.resize(bsz * kvd); e.bv.resize(bsz * kvd);
    e.bgate.resize(bsz * FF); e.bup.resize(bsz * FF);
    e.bscores.resize(bsz * (size_t)ctx);
    e.bc_rope.resize(bsz * (size_t)half); e.bs_rope.resize(bsz * (size_t)half);
    e.bxt.resize(((bsz + 7) & ~(size_t)7) * FF * 2 + (size_t)E * ((bsz + 7) & ~(size_t)7));

    std::vector<int> toks((size_t)KORE_BMAX, 0);
    for (int st = 0; st < n_steps; st++) {
        int32_t pn[2];
        if (!rd(in, pn, sizeof pn)) return 4;
        const int pos = pn[0], nb = pn[1];
        for (int l = 0; l < n_layer; l++) {
            if (!rd(in, bias[(size_t)l * 3 + 0].data(), sizeof(float) * E) ||
                !rd(in, bias[(size_t)l * 3 + 1].data(), sizeof(float) * kvd) ||
                !rd(in, bias[(size_t)l * 3 + 2].data(), sizeof(float) * kvd)) return 4;
        }
        if (mode == 0) {
            if (nb != 1 || !forward(e, 0, pos, false)) { fprintf(stderr, "forward failed at %d\n", pos); return 5; }
            if (!wr(out, e.att.data(), sizeof(float) * E) || !wr(out, e.q.data(), sizeof(float) * E)) return 6;
        } else {
            if (!forward_batch(e, toks.data(), nb, pos, false)) { fprintf(stderr, "forward_batch failed at %d+%d\n", pos, nb); return 5; }
            if (!wr(out, e.batt.data(), sizeof(float) * (size_t)nb * E) ||
                !wr(out, e.bq.data(), sizeof(float) * (size_t)nb * E)) return 6;
        }
    }
    if (!wr(out, e.kcache.data(), sizeof(float) * e.kcache.size()) ||
        !wr(out, e.vcache.data(), sizeof(float) * e.vcache.size()) ||
        !wr(out, e.inv_freq.data(), sizeof(float) * (size_t)half)) return 6;
    fclose(out);
    fclose(in);
    return 0;
}
