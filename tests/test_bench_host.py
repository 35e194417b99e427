"""Host-side logic of bench.py (no GPU): the report builders of the matvec
and batched-matmul legs turn the per-kind launch timings into the JSON fields
the bench line carries, and the workload tables match the 7B shapes."""
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

import bench  # noqa: E402


def _mats():
    return bench.qmv_token_matrices()


def test_token_matrices_are_the_7b_layout():
    mats = _mats()
    assert len(mats) == 7 * bench.NL + 1
    q6 = sum(1 for _, t, _, _ in mats if t == bench.QMV_Q6K)
    assert q6 == 2 * 14 + 1                      # attn_v and ffn_down on 14 layers, the output head
    wbytes = sum(bench.qmv_weight_bytes(t, r, c) for _, t, r, c in mats)
    assert 4.3e9 < wbytes < 4.45e9


def test_matvec_report_fields():
    mats = _mats()
    op_mats = [(0, 1, 2), (3,), (4, 5), (6,)] + [(7 * bench.NL,)]
    class_ms = {bench._mv_key(mats, ts): [0.01, 0.01] for ts in op_mats}
    g = dict(mats=mats, op_mats=op_mats, wall_ms=20.0, region_ms=16.0, class_ms=class_ms)
    r = bench.matvec_report(g, 10)
    assert set(r["per_matrix"]) == {"attn_q_q4k+attn_k_q4k+attn_v_q6k", "attn_output_q4k",
                                    "ffn_gate_q4k+ffn_up_q4k", "ffn_down_q6k", "output"}
    assert r["per_matrix"]["attn_output_q4k"]["us_mean"] == 10.0
    assert r["ms_per_token_gpu"] == 1.6 and r["launches_per_token"] == len(op_mats)
    assert r["roofline"]["bound"] == "hbm" and r["roofline"]["unit"] == "GB/s"
    assert 0 < r["roofline"]["frac"] < 1


def test_gemm_report_fields():
    mats = _mats()
    op_mats = []
    for l in range(bench.NL):
        b = 7 * l
        op_mats += [(b, b + 1, b + 2), (b + 3,), (b + 4, b + 5), (b + 6,)]
    # launch times proportional to their flops: the dominant launch is gate+up
    per = np.array([sum(2 * bench.GEMM_B * mats[i][2] * mats[i][3] for i in ts) for ts in op_mats]) / 1e11
    class_ms = {bench._gemm_key(mats, ts): [float(ms)] * 3 for ts, ms in zip(op_mats, per)}
    g = dict(mats=mats, op_mats=op_mats, wall_ms=50.0, region_ms=50.0, class_ms=class_ms)
    r = bench.gemm_report(g, 5)
    flop = sum(2 * bench.GEMM_B * mats[i][2] * mats[i][3] for i in range(7 * bench.NL))
    assert r["flop_per_chunk"] == flop
    assert abs(r["tflops"] - flop / 0.01 / 1e12) < 0.01
    # the fp16 path (the default): fp16 MFMA peak, MFMA work = flops x passes
    assert r["roofline"]["bound"] == "mfma" and r["roofline"]["peak"] == bench.FP16_MFMA_PEAK_TFLOPS
    assert r["roofline"]["kernel"] == "ffn_gate_q4k+ffn_up_q4k"
    gu = r["per_matrix"]["ffn_gate_q4k+ffn_up_q4k"]
    assert abs(gu["mfma_tflops"] - gu["tflops"] * bench.GEMM16_PASSES[bench.QMV_Q4K]) < 0.02
    assert abs(r["roofline"]["frac"] - gu["mfma_tflops"] / bench.FP16_MFMA_PEAK_TFLOPS) < 1e-4


def test_token_and_prompt_report_fields():
    mats = _mats()
    t = bench.token_report({"region_ms": 64.0, "wall_ms": 64.5, "tokens": 32}, mats)
    assert t["ms_per_token_gpu"] == 2.0 and t["tokens_per_s"] == 500.0
    assert abs(t["gbs"] - (t["weight_bytes_per_token"] + t["kv_bytes_per_token"]) / 2e-3 / 1e9) < 0.1
    p = bench.prompt_report({"region_ms": 80.0, "wall_ms": 80.4, "chunks": 8, "tokens": 512}, mats)
    # the seven matrices of 28 layers at 64 rows: 2 * 64 * rows * cols, the head not counted
    flops = 2 * 64 * bench.NL * (3584 * 3584 * 2 + 512 * 3584 * 2 + 18944 * 3584 * 3)
    assert p["matmul_flop_per_chunk"] == flops
    assert p["ms_per_chunk_gpu"] == 10.0 and p["tokens_per_s"] == 6400.0
    assert abs(p["matmul_tflops_effective"] - flops / 1e-2 / 1e12) < 0.01


def test_runs_summary():
    r = bench._runs([2.0, 5.0, 3.0], "GB/s")
    assert r["median"] == 3.0 and r["best"] == 5.0 and r["runs"] == [2.0, 5.0, 3.0]


class _OracleCache:
    """Stands in for the GPU handle in decode_parity: its cache rows are the
    oracle's own (roped K, V) rows of the decode workload."""

    def __init__(self, n_layers, n_pos):
        import oracle
        inv_f = oracle.inv_freq(bench.HD, bench.ROPE_BASE)
        self.rows = []
        for l in range(n_layers):
            k = oracle.synth(n_pos, bench.KVD, bench.DEC_SEED, bench.k_stream(l), 0, 2, bench.DEC_PER_MILLE,
                             bench.DEC_OUTLIER)
            v = oracle.synth(n_pos, bench.KVD, bench.DEC_SEED, bench.v_stream(l), 0, 3, bench.DEC_PER_MILLE,
                             bench.DEC_OUTLIER)
            self.rows.append((oracle.rope_rows(k, np.arange(n_pos), bench.NKV, bench.HD, inv_f), v))

    def read_kv(self, layer, pos0, n):
        k, v = self.rows[layer]
        return k[pos0:pos0 + n], v[pos0:pos0 + n]


def _oracle_outputs(n_layers, n_steps):
    import oracle
    kv = oracle.KV(n_layers, bench.DEC_POS0 + n_steps, bench.NH, bench.NKV, bench.HD, bench.ROPE_BASE)
    inv_f = oracle.inv_freq(bench.HD, bench.ROPE_BASE)
    kc, vc = kv.kcache(), kv.vcache()
    outs = np.zeros((n_steps, n_layers, bench.E), np.float32)
    for l in range(n_layers):
        k0 = oracle.synth(bench.DEC_POS0, bench.KVD, bench.DEC_SEED, bench.k_stream(l), 0, 2, bench.DEC_PER_MILLE,
                          bench.DEC_OUTLIER)
        kc[l, :bench.DEC_POS0] = oracle.rope_rows(k0, np.arange(bench.DEC_POS0), bench.NKV, bench.HD, inv_f)
        vc[l, :bench.DEC_POS0] = oracle.synth(bench.DEC_POS0, bench.KVD, bench.DEC_SEED, bench.v_stream(l), 0, 3,
                                              bench.DEC_PER_MILLE, bench.DEC_OUTLIER)
    for st in range(n_steps):
        pos = bench.DEC_POS0 + st
        for l in range(n_layers):
            q, k, v = (oracle.synth(1, d, bench.DEC_SEED, sf(l), pos, t, bench.DEC_PER_MILLE, bench.DEC_OUTLIER)[0]
                       for d, sf, t in ((bench.E, bench.q_stream, 1), (bench.KVD, bench.k_stream, 2),
                                        (bench.KVD, bench.v_stream, 3)))
            outs[st, l] = kv.decode(l, pos, q, k, v)
    kv.close()
    return outs


def test_decode_parity_finds_a_planted_error():
    """decode_parity on outputs that are the oracle's own (zero error, cache
    equal) and with one planted difference, which it must report at the
    right step and layer; the float64 budget puts kore's own error below the
    1e-4 bound."""
    nl, ns = 2, 3
    outs = _oracle_outputs(nl, ns)
    cache = _OracleCache(nl, bench.DEC_POS0 + ns)
    r = bench.decode_parity(outs, cache, 4, n_layers=nl, n_steps=ns)
    assert r["decode_max_rel_err"] == 0.0 and r["decode_kv_bitwise"]
    assert len(r["decode_step_max_rel_err"]) == ns
    assert 0 < r["decode_error_budget"]["kore_vs_float64_max"] < 1e-4
    bad = outs.copy()
    scale = float(np.max(np.abs(outs[2, 1])))
    bad[2, 1, 77] += 3e-4 * scale
    r = bench.decode_parity(bad, cache, 4, n_layers=nl, n_steps=ns)
    assert r["decode_max_rel_err"] > 2e-4
    assert r["decode_max_rel_err_at"] == {"step": 2, "position": bench.DEC_POS0 + 2, "layer": 1}
    cache.rows[1][0][5, 3] += 1.0                      # one cache bit off
    assert not bench.decode_parity(outs, cache, 4, n_layers=nl, n_steps=ns)["decode_kv_bitwise"]


def test_reference_timing_runs():
    """kore's own timing harness (built from kore.cpp) reports one entry per
    timed run, which the CPU baselines take the median and best of."""
    import json
    import struct
    import subprocess
    import tempfile

    import oracle
    import pytest
    if not os.path.exists(oracle.REF_QMV_BIN):
        pytest.skip("kore's reference harness is not built here")
    rows, cols = 64, 512
    rng = np.random.default_rng(1)
    w = rng.integers(0, 256, size=(rows, cols // 256, 144), dtype=np.uint8)
    w[:, :, 0:4] = np.frombuffer(np.float16([1e-3, 1e-3]).tobytes(), np.uint8)
    x = rng.standard_normal(cols).astype(np.float32)
    with tempfile.TemporaryDirectory() as td:
        job = os.path.join(td, "job.bin")
        with open(job, "wb") as f:
            f.write(struct.pack("<3i", bench.QMV_Q4K, rows, cols))
            f.write(w.tobytes())
            f.write(x.tobytes())
        out = subprocess.run([oracle.REF_QMV_BIN, "--time", "2", "0.02", "2", job, "3"], capture_output=True,
                             text=True, check=True).stdout
    j = json.loads(out)
    assert len(j["run_reps"]) == 3 and len(j["run_seconds"]) == 3
    assert sum(j["run_reps"]) == j["reps"] and all(t >= 0.02 for t in j["run_seconds"])


def _small_decode_outs(n_layer, rows, nh, nkv, hd, seed, pos_first, n_steps, window=0):
    """The oracle's own outputs of a small decode workload laid out as the
    bench's other-workload legs fill and decode it."""
    import oracle
    kvd, E_ = nkv * hd, nh * hd
    inv_f = oracle.inv_freq(hd, bench.ROPE_BASE)
    ctx = window if window else rows + n_steps
    kv = oracle.KV(n_layer, ctx, nh, nkv, hd, bench.ROPE_BASE, window=window)
    outs = np.zeros((n_steps, n_layer, E_), np.float32)
    for l in range(n_layer):
        k0 = oracle.synth(rows, kvd, seed, bench.k_stream(l), 0, 2)
        kv.kcache()[l, :rows] = oracle.rope_rows(k0, np.arange(rows), nkv, hd, inv_f)
        kv.vcache()[l, :rows] = oracle.synth(rows, kvd, seed, bench.v_stream(l), 0, 3)
        for s in range(n_steps):
            p = pos_first + s
            outs[s, l] = kv.decode(l, p, oracle.synth(1, E_, seed, bench.q_stream(l), p, 1)[0],
                                   oracle.synth(1, kvd, seed, bench.k_stream(l), p, 2)[0],
                                   oracle.synth(1, kvd, seed, bench.v_stream(l), p, 3)[0])
    k, v = kv.kcache().copy(), kv.vcache().copy()
    kv.close()
    return outs, k, v


def test_other_workload_parity_finds_a_planted_error():
    """_parity_decode_layers (the bench's C1 / C4 / C5 decode parity): zero on
    the oracle's own outputs and cache rows, the planted difference and the
    flipped cache bit found; the window ring (C5's sliding decode) too."""
    nl, rows, nh, nkv, hd, seed = 2, 40, 4, 2, 64, 3
    outs, k, v = _small_decode_outs(nl, rows, nh, nkv, hd, seed, rows, 1)
    rows_of = lambda l: (k[l], v[l])   # noqa: E731
    r = bench._parity_decode_layers(nl, rows, nh, nkv, hd, seed, rows, outs, 2, kv_rows=rows_of)
    assert r["max_rel_err"] == 0.0 and r["kv_bitwise"] and r["layers"] == nl and r["steps"] == 1
    bad = outs.copy()
    bad[0, 1, 5] += 5e-4 * float(np.max(np.abs(outs[0, 1])))
    assert bench._parity_decode_layers(nl, rows, nh, nkv, hd, seed, rows, bad, 2)["max_rel_err"] > 4e-4
    k[1, 7, 3] += 1.0
    assert not bench._parity_decode_layers(nl, rows, nh, nkv, hd, seed, rows, outs, 2, kv_rows=rows_of)["kv_bitwise"]
    W = 32
    outs_w, _, _ = _small_decode_outs(1, W, nh, nkv, hd, seed, W, 6, window=W)
    r = bench._parity_decode_layers(1, W, nh, nkv, hd, seed, W, outs_w, 1, window=W)
    assert r["max_rel_err"] == 0.0 and r["steps"] == 6
    outs_w[4, 0, 0] += 1e-3 * float(np.max(np.abs(outs_w[4, 0])))
    assert bench._parity_decode_layers(1, W, nh, nkv, hd, seed, W, outs_w, 1, window=W)["max_rel_err"] > 5e-4


def test_summary_is_last_and_names_every_config():
    res = {"decode": {"us_per_layer_gpu": 8.0, "floor": {"read_plus_dependent_launch_us": 6.5,
                                                         "layer_over_floor": 1.23}},
           "roofline": {"frac": 0.26}, "prefill": {"us_per_layer_gpu": 270.0, "roofline": {"frac": 0.71}},
           "other_workloads": {"decode_3b_pos32767": {"us_per_layer_gpu": 19.0, "roofline": {"frac": 0.44}}},
           "parity": {"decode_max_rel_err": 4e-5, "c4_decode_3b": {"max_rel_err": 1e-6}}}
    s = bench._summary(res)
    assert s["c2_decode_7b_us_per_layer"] == 8.0 and s["c2_over_floor"] == 1.23 and s["c4_frac"] == 0.44
    assert s["c1_decode_0p5b_us"] is None
    assert set(s["parity_max_rel_err"]) == {"c1_decode_0p5b", "c2_decode_7b", "c3_prefill_7b", "c4_decode_3b",
                                            "c5_chunk_1p5b", "c5_sliding_decode_1p5b"}
    assert s["parity_max_rel_err"]["c4_decode_3b"] == 1e-6
