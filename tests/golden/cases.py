"""Golden-fixture case definitions shared by make_golden.py and the tests.

Each case is a sequence of kore calls on one KV store: decode steps
(``forward()``, one position each) or prefill chunks (``forward_batch()``,
``nb`` positions from ``pos``).  Inputs are the counter-based synthetic
values of ``oracle.synth``: for step ``st`` and layer ``l`` the q/k/v rows
are row ``st`` of streams ``(1<<32)|l``, ``(2<<32)|l`` and ``(3<<32)|l``
(outlier tensors 1, 2, 3).  A prefill chunk uses the same q/k/v for all of
its rows (in kore those are the layer biases, see oracle/ref_harness.cpp);
the case of one-row prefill steps gives every row its own q/k/v.
"""
from __future__ import annotations

import hashlib
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def _decode_steps(n):
    return [[p, 1] for p in range(n)]


CASES = [
    # 0.5B geometry (14/2/64, n_rep 7), decode through pos 511 (the 0.5B
    # single-layer decode workload), full KV kept in the fixture.
    dict(name="decode_c1", mode="decode", n_layer=1, n_head=14, n_head_kv=2, head_dim=64,
         ctx=512, rope_base=1e6, avx2=1, seed=11, per_mille=0, steps=_decode_steps(512),
         sample_steps=[0, 1, 2, 3, 31, 64, 255, 500, 510, 511], keep_kv=True),
    # 7B geometry (28/4/128, n_rep 7), two layers, 1 % outlier channels x20.
    dict(name="decode_7b", mode="decode", n_layer=2, n_head=28, n_head_kv=4, head_dim=128,
         ctx=160, rope_base=1e6, avx2=1, seed=12, per_mille=10, steps=_decode_steps(160),
         sample_steps=[0, 1, 77, 158, 159], keep_kv=False),
    # 3B geometry (16/2/128, n_rep 8).
    dict(name="decode_3b", mode="decode", n_layer=1, n_head=16, n_head_kv=2, head_dim=128,
         ctx=96, rope_base=1e6, avx2=1, seed=13, per_mille=0, steps=_decode_steps(96),
         sample_steps=[0, 50, 95], keep_kv=False),
    # Batched causal prefill through kore's AVX2 hd_dot/hd_fma, n_rep 7,
    # chunks of every size class up to kore's 64-row limit.
    dict(name="prefill_7b_avx2", mode="prefill", n_layer=2, n_head=14, n_head_kv=2, head_dim=128,
         ctx=256, rope_base=1e6, avx2=1, seed=21, per_mille=0,
         steps=[[0, 1], [1, 7], [8, 64], [72, 33], [105, 64], [169, 50], [219, 37]],
         sample_steps=[0, 1, 2, 6], keep_kv=False),
    # Same geometry on kore's scalar hd_dot/hd_fma fallback.
    dict(name="prefill_7b_scalar", mode="prefill", n_layer=1, n_head=14, n_head_kv=2,
         head_dim=128, ctx=96, rope_base=1e6, avx2=0, seed=22, per_mille=0,
         steps=[[0, 5], [5, 64], [69, 27]], sample_steps=[0, 2], keep_kv=False),
    # head_dim 64, theta 1e4, n_rep 7.
    dict(name="prefill_hd64_avx2", mode="prefill", n_layer=1, n_head=28, n_head_kv=4,
         head_dim=64, ctx=160, rope_base=1e4, avx2=1, seed=23, per_mille=0,
         steps=[[0, 64], [64, 1], [65, 64], [129, 31]], sample_steps=[0, 3], keep_kv=False),
    # 1.5B geometry (12/2/128, n_rep 6).
    dict(name="prefill_1p5b_avx2", mode="prefill", n_layer=1, n_head=12, n_head_kv=2,
         head_dim=128, ctx=128, rope_base=1e6, avx2=1, seed=24, per_mille=0,
         steps=[[0, 64], [64, 64]], sample_steps=[1], keep_kv=False),
    # Distinct q/k/v on every row of the batched path: forward_batch() with one
    # row per call (kore's batched attention, AVX2 hd_dot/hd_fma, 1 % outlier
    # channels x20); row z attends positions 0..z exactly as row z of one
    # 64-row chunk would, so a GPU chunk of all 64 rows replays it.
    dict(name="prefill_rows_7b_avx2", mode="prefill", n_layer=1, n_head=14, n_head_kv=2, head_dim=128,
         ctx=64, rope_base=1e6, avx2=1, seed=27, per_mille=10, steps=[[p, 1] for p in range(64)],
         sample_steps=list(range(64)), keep_kv=True),
    # head_dim 40: 16-float FMA steps plus an 8-float scalar tail in hd_dot.
    dict(name="prefill_hd40_avx2", mode="prefill", n_layer=1, n_head=32, n_head_kv=8,
         head_dim=40, ctx=80, rope_base=1e6, avx2=1, seed=25, per_mille=0,
         steps=[[0, 16], [16, 64]], sample_steps=[1], keep_kv=False),
    # head_dim 36: scalar tails in both hd_dot (4) and hd_fma (4).
    dict(name="prefill_hd36_avx2", mode="prefill", n_layer=1, n_head=64, n_head_kv=16,
         head_dim=36, ctx=48, rope_base=1e6, avx2=1, seed=26, per_mille=0,
         steps=[[0, 48]], sample_steps=[0], keep_kv=False),
]


def case_by_name(name):
    for c in CASES:
        if c["name"] == name:
            return c
    raise KeyError(name)


def step_inputs(case, st, layer):
    """(q [E], k [kvd], v [kvd]) for step ``st`` and ``layer``."""
    import oracle

    E = case["n_head"] * case["head_dim"]
    kvd = case["n_head_kv"] * case["head_dim"]
    seed, pm = case["seed"], case["per_mille"]
    q = oracle.synth(1, E, seed, (1 << 32) | layer, row0=st, tensor=1, per_mille=pm)[0]
    k = oracle.synth(1, kvd, seed, (2 << 32) | layer, row0=st, tensor=2, per_mille=pm)[0]
    v = oracle.synth(1, kvd, seed, (3 << 32) | layer, row0=st, tensor=3, per_mille=pm)[0]
    return q, k, v


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a, dtype="<f4").tobytes()).hexdigest()


def manifest_path(name):
    return os.path.join(HERE, f"{name}.json")


def npz_path(name):
    return os.path.join(HERE, f"{name}.npz")


def load(name):
    with open(manifest_path(name)) as f:
        man = json.load(f)
    data = dict(np.load(npz_path(name), allow_pickle=False))
    return man, data
