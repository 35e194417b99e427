#!/usr/bin/env python3
"""Write the golden fixture of kore's forward() over two layers with real
quantised weights: tests/golden/layer_2x256.npz / .json.

Runs kore's own forward() (kore.cpp:1397-1484) through
oracle/_ref/kore_layer_ref (built by ``make -C oracle ref`` from the kore.cpp
sources; see oracle/ref_layer_harness.cpp) on a small geometry (E = 256 =
2 heads x 128, one kv head, n_ff = 512, rope base 1e6, eps 1e-6) for five
decode steps, once with kore's AVX2 matvec order and once with the scalar
one, and stores the weights, norms, biases, embeddings and, per order, kore's
residual x after each step and the final K/V caches.  Layer 0 keeps wv and
w_down in Q6_K (as Q4_K_M files do on some layers), layer 1 is all Q4_K.
Weights (random block bytes, scales of a trained model's size) and inputs
are synthetic (numpy PCG64, fixed seed).  Needs the kore
sources, so it runs only where they are present; the tests read the fixture.
"""
from __future__ import annotations

import hashlib
import json
import os
import struct
import subprocess
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

import oracle  # noqa: E402
from make_golden_qmv import synth_x  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
N_LAYER, NH, NKV, HD, FF, CTX, STEPS = 2, 2, 1, 128, 512, 8, 5
E, KVD = NH * HD, NKV * HD
ROPE_BASE, EPS = 1e6, 1e-6
Q4, Q6 = oracle.TYPE_Q4K, oracle.TYPE_Q6K
TYPES = [[Q4, Q4, Q6, Q4, Q4, Q4, Q6], [Q4] * 7]
SHAPES = [(E, E), (KVD, E), (KVD, E), (E, E), (FF, E), (FF, E), (E, FF)]   # rows, cols


def layer_weights(wtype: int, rows: int, nblk: int, rng: np.random.Generator) -> np.ndarray:
    """Random block bytes with f16 scales of a trained model's size (the matvec
    fixtures cover extreme scales; a two-layer stack of them would overflow)."""
    bb = oracle.BLOCK_BYTES[wtype]
    w = rng.integers(0, 256, size=(rows, nblk, bb), dtype=np.uint8)

    def f16(lo, hi):   # f16 subnormals at these sizes: the dequantisers must take them
        return (lo + (hi - lo) * rng.random((rows, nblk))).astype(np.float16).view(np.uint8).reshape(rows, nblk, 2)

    if wtype == oracle.TYPE_Q4K:      # |w| <= d * 63 * 15 + dmin * 63: about 0.03
        w[:, :, 0:2] = f16(1e-5, 3e-5)
        w[:, :, 2:4] = f16(0.0, 1e-5)
    else:                             # |w| <= d * 128 * 32: about 0.03
        w[:, :, 208:210] = f16(2e-6, 6e-6)
    return w.reshape(-1)


def make_inputs(seed: int = 31):
    rng = np.random.default_rng(seed)
    layers = []
    for l in range(N_LAYER):
        mats = [layer_weights(TYPES[l][j], r, c // 256, rng) for j, (r, c) in enumerate(SHAPES)]
        attn_norm = (1.0 + 0.1 * rng.standard_normal(E)).astype(np.float32)
        ffn_norm = (1.0 + 0.1 * rng.standard_normal(E)).astype(np.float32)
        bq = (0.5 * rng.standard_normal(E)).astype(np.float32)
        bk = (0.5 * rng.standard_normal(KVD)).astype(np.float32)
        bv = (0.5 * rng.standard_normal(KVD)).astype(np.float32)
        layers.append(dict(mats=mats, attn_norm=attn_norm, ffn_norm=ffn_norm, bq=bq, bk=bk, bv=bv))
    emb = np.stack([synth_x(E, rng) for _ in range(STEPS)])
    return layers, emb


def run_kore(layers, emb, avx2: int):
    with tempfile.TemporaryDirectory() as td:
        job, res = os.path.join(td, "job.bin"), os.path.join(td, "res.bin")
        with open(job, "wb") as f:
            f.write(struct.pack("<8i", N_LAYER, NH, NKV, HD, FF, CTX, avx2, STEPS))
            f.write(struct.pack("<2f", ROPE_BASE, EPS))
            for l, ly in enumerate(layers):
                f.write(struct.pack("<7i", *TYPES[l]))
                for a in (ly["attn_norm"], ly["ffn_norm"], ly["bq"], ly["bk"], ly["bv"]):
                    f.write(a.astype("<f4").tobytes())
                for m in ly["mats"]:
                    f.write(m.tobytes())
            f.write(emb.astype("<f4").tobytes())
            f.write(np.arange(STEPS, dtype="<i4").tobytes())
        rc = subprocess.run([oracle.REF_LAYER_BIN, job, res]).returncode
        if rc != 0:
            raise RuntimeError(f"kore_layer_ref failed ({rc})")
        out = np.fromfile(res, "<f4")
    xs = out[:STEPS * E].reshape(STEPS, E)
    kc = out[STEPS * E:STEPS * E + N_LAYER * CTX * KVD].reshape(N_LAYER, CTX, KVD)
    vc = out[STEPS * E + N_LAYER * CTX * KVD:].reshape(N_LAYER, CTX, KVD)
    return xs, kc, vc


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main():
    if not os.path.exists(oracle.REF_LAYER_BIN):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "ref"], check=True)
    layers, emb = make_inputs()
    arrays = {"emb": emb}
    for l, ly in enumerate(layers):
        for k in ("attn_norm", "ffn_norm", "bq", "bk", "bv"):
            arrays[f"l{l}_{k}"] = ly[k]
        for j, m in enumerate(ly["mats"]):
            arrays[f"l{l}_{oracle.LayerWeights.NAMES[j]}"] = m
    for avx2 in (1, 0):
        xs, kc, vc = run_kore(layers, emb, avx2)
        tag = "avx2" if avx2 else "ref"
        arrays[f"x_{tag}"], arrays[f"kcache_{tag}"], arrays[f"vcache_{tag}"] = xs, kc, vc
    np.savez_compressed(os.path.join(HERE, "layer_2x256.npz"), **arrays)
    man = {"n_layer": N_LAYER, "n_head": NH, "n_head_kv": NKV, "head_dim": HD, "n_ff": FF, "ctx": CTX,
           "steps": STEPS, "rope_base": ROPE_BASE, "rms_eps": EPS, "types": TYPES,
           "source": "kore.cpp forward() (quantised path, both matvec orders) via oracle/_ref/kore_layer_ref",
           "sha256": {k: sha(v) for k, v in arrays.items()}}
    with open(os.path.join(HERE, "layer_2x256.json"), "w") as f:
        json.dump(man, f, indent=1)
    print("layer_2x256:", {k: float(np.max(np.abs(arrays[k]))) for k in ("x_avx2", "x_ref")})


if __name__ == "__main__":
    main()
