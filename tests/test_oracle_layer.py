"""The oracle's composition of kore's forward() layer (rmsnorm, Q8_K
quantisation, q/k/v matvecs and biases, RoPE, append, attention, Wo and the
residual add, rmsnorm, gate/up, SwiGLU, down and the residual add;
kore.cpp:1415-1472) against kore's own forward() run on the same weights
(tests/golden/layer_2x256: two layers, Q4_K and Q6_K, five decode steps, both
matvec orders), and rmsnorm / SwiGLU against what their formulas fix.
"""
import json
import os

import numpy as np
import pytest

import oracle

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_layer_fixture():
    man = json.load(open(os.path.join(GOLD, "layer_2x256.json")))
    z = np.load(os.path.join(GOLD, "layer_2x256.npz"))
    layers = []
    for l in range(man["n_layer"]):
        layers.append(oracle.LayerWeights(man["types"][l], [z[f"l{l}_{n}"] for n in oracle.LayerWeights.NAMES],
                                          z[f"l{l}_attn_norm"], z[f"l{l}_ffn_norm"], z[f"l{l}_bq"], z[f"l{l}_bk"],
                                          z[f"l{l}_bv"]))
    return man, z, layers


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("tag,avx2", [("avx2", True), ("ref", False)])
def test_layer_composition_matches_kore_forward(tag, avx2):
    man, z, layers = load_layer_fixture()
    kv = oracle.KV(man["n_layer"], man["ctx"], man["n_head"], man["n_head_kv"], man["head_dim"], man["rope_base"])
    for st in range(man["steps"]):
        x = z["emb"][st]
        for l, lw in enumerate(layers):
            x = oracle.layer_forward(kv, l, st, x, lw, man["n_ff"], man["rms_eps"], avx2=avx2)
        assert np.array_equal(_bits(x), _bits(z[f"x_{tag}"][st])), f"step {st}"
    assert np.array_equal(_bits(kv.kcache()), _bits(z[f"kcache_{tag}"]))
    assert np.array_equal(_bits(kv.vcache()), _bits(z[f"vcache_{tag}"]))


def test_layer_fixture_orders_differ():
    man, z, _ = load_layer_fixture()
    assert not np.array_equal(_bits(z["x_avx2"]), _bits(z["x_ref"]))


def test_rmsnorm_closed_forms():
    # constant vector: scale = 1/sqrt(c^2 + eps); unit weights give c * scale
    for c, n in ((0.5, 256), (3.0, 3584), (1e-20, 512)):
        x = np.full(n, c, np.float32)
        out = oracle.rmsnorm(x, np.ones(n, np.float32), 1e-6)
        ss = np.float64(c) * np.float64(c) * n
        scale = np.float32(1.0) / np.sqrt(np.float32(ss / n) + np.float32(1e-6))
        assert np.all(out == np.float32(np.float32(c) * scale))
    # against float64 on random data: within 2 ulp of the float64 result
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(3584) * rng.choice([1e-3, 1.0, 30.0], 3584)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(3584)).astype(np.float32)
    out = oracle.rmsnorm(x, w, 1e-6).astype(np.float64)
    ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * w
    assert np.all(np.abs(out - ref) <= 2.5e-7 * np.abs(ref) + 1e-30)
    # all zero: scale = 1/sqrt(eps), outputs zero
    assert np.all(oracle.rmsnorm(np.zeros(256, np.float32), np.ones(256, np.float32), 1e-6) == 0)


def test_swiglu_closed_forms():
    g = np.array([0.0, 1.0, -1.0, 20.0, -20.0, 100.0, -100.0], np.float32)
    u = np.ones_like(g)
    out = oracle.swiglu(g, u).astype(np.float64)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))
    assert out[0] == 0.0
    assert np.all(np.abs(out - ref) <= 2.5e-7 * np.abs(ref) + 1e-30)
    assert oracle.swiglu(np.array([-1000.0], np.float32), np.ones(1, np.float32))[0] == 0.0   # exp overflow
