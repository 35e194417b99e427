"""Host-side logic of bench.py (no GPU): the report builders of the matvec
and batched-matmul legs turn per-launch timings into the JSON fields the
bench line carries, and the workload tables match the 7B shapes."""
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
    g = dict(mats=mats, op_mats=op_mats, wall_ms=20.0, region_ms=16.0, op_ms=np.full((2, len(op_mats)), 0.01))
    r = bench.matvec_report(g, 10)
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
    g = dict(mats=mats, op_mats=op_mats, wall_ms=50.0, region_ms=50.0, op_ms=np.tile(per, (3, 1)))
    r = bench.gemm_report(g, 5)
    flop = sum(2 * bench.GEMM_B * mats[i][2] * mats[i][3] for i in range(7 * bench.NL))
    assert r["flop_per_chunk"] == flop
    assert abs(r["tflops"] - flop / 0.01 / 1e12) < 0.01
    assert r["roofline"]["bound"] == "mfma" and r["roofline"]["peak"] == bench.FP32_MFMA_PEAK_TFLOPS
    assert r["roofline"]["kernel"] == "ffn_gate_q4k+ffn_up_q4k"


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
