#!/usr/bin/env python3
"""Write the golden fixtures of kore's quantised matvec and batched matmul.

Runs kore's own quantize_row_q8_K and its Q4_K / Q6_K x Q8_K dot products,
scalar and AVX2 (kore.cpp:422-632), through oracle/_ref/kore_qmv_ref (built by
``make -C oracle ref`` from the kore.cpp sources; see
oracle/ref_qmv_harness.cpp) on the cases below and stores, per case:

* ``qmv_<case>.npz``: the weight bytes, the input x, kore's Q8_K blocks of x
  (292 bytes each) and kore's row results, scalar and AVX2;
* ``qmv_<case>.json``: the case and the sha256 of every array;
* ``qmm_<case>.npz`` / ``.json``: kore's matmul_batch_float (kore.cpp:783-845),
  AVX2 and scalar paths, for B activations at once.

The weights and inputs are synthetic (numpy PCG64, fixed seeds) and include
the corner cases the formats and the quantiser have: an all-zero block of x, a
block whose largest magnitude appears twice with both signs, a constant block,
subnormal inputs, f16 scales that are zero, subnormal or negative, and all-ones
scale bytes.  Needs the kore sources, so it runs only where they are present;
the tests read the fixtures it wrote.
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

import oracle  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))

CASES = [
    # name, type, rows, cols, seed
    ("q4k_mix", oracle.TYPE_Q4K, 40, 2560, 11),
    ("q6k_mix", oracle.TYPE_Q6K, 40, 2560, 12),
    ("q6k_odd", oracle.TYPE_Q6K, 24, 2304, 13),      # 9 blocks: rows start 2 bytes off a word
    ("q4k_3584", oracle.TYPE_Q4K, 32, 3584, 14),     # Qwen2.5-7B attention / gate / up width
    ("q6k_18944", oracle.TYPE_Q6K, 8, 18944, 15),    # Qwen2.5-7B ffn_down width: 74 blocks
]


def f16_bits(v) -> np.ndarray:
    return np.asarray(v, np.float16).view(np.uint16)


BATCH_CASES = [
    # name, type, rows, cols, B, seed
    ("q4k_b5", oracle.TYPE_Q4K, 40, 1024, 5, 21),
    ("q6k_b64", oracle.TYPE_Q6K, 33, 768, 64, 22),
    ("q4k_b13_odd", oracle.TYPE_Q4K, 17, 2304, 13, 23),
    ("q6k_b1", oracle.TYPE_Q6K, 8, 512, 1, 24),
]


def synth_weights(wtype: int, rows: int, nblk: int, rng: np.random.Generator) -> np.ndarray:
    """rows x nblk blocks of random bytes with plausible f16 scales, plus
    special scale values on a few blocks."""
    bb = oracle.BLOCK_BYTES[wtype]
    w = rng.integers(0, 256, size=(rows, nblk, bb), dtype=np.uint8)
    d = f16_bits(np.abs(rng.standard_normal((rows, nblk))) * 2e-3 + 1e-4)
    if wtype == oracle.TYPE_Q4K:
        dmin = f16_bits(np.abs(rng.standard_normal((rows, nblk))) * 1e-3)
        w[:, :, 0:2] = d.view(np.uint8).reshape(rows, nblk, 2)
        w[:, :, 2:4] = dmin.view(np.uint8).reshape(rows, nblk, 2)
        specials = [(0, 0, 0x0000, None), (1, 1, 0x0001, 0x8001), (2, 2, 0x83FF, 0x3C00),
                    (3, 0, 0xB800, 0x0000)]
        for r, b, dv, mv in specials:
            if r < rows and b < nblk:
                w[r, b, 0:2] = np.frombuffer(struct.pack("<H", dv), np.uint8)
                if mv is not None:
                    w[r, b, 2:4] = np.frombuffer(struct.pack("<H", mv), np.uint8)
        if rows > 4:
            w[4, 0, 4:16] = 0xFF                            # every 6-bit scale and min at 63
    else:
        w[:, :, 208:210] = d.view(np.uint8).reshape(rows, nblk, 2)
        for r, b, dv in [(0, 0, 0x0000), (1, 1, 0x0001), (2, 2, 0x83FF), (3, 0, 0xB800)]:
            if r < rows and b < nblk:
                w[r, b, 208:210] = np.frombuffer(struct.pack("<H", dv), np.uint8)
        if rows > 4:
            w[4, 0, 192:208] = 0x80                         # every int8 scale at -128
            w[4, 0, 0:192] = 0xFF                           # every 6-bit value at 63
    return w.reshape(-1)


def synth_x(cols: int, rng: np.random.Generator) -> np.ndarray:
    x = rng.standard_normal(cols).astype(np.float32)
    ch = rng.random(cols) < 0.01
    x[ch] *= 20.0                                           # 1% outlier channels
    nb = cols // 256
    blk = lambda i: slice(256 * i, 256 * (i + 1))           # noqa: E731
    if nb > 1:
        x[blk(1)] = 0.0                                     # zero block: d = 0, qs = 0
    if nb > 2:
        v = x[blk(2)]
        m = float(np.max(np.abs(v))) * 1.5
        v[17], v[200] = -m, m                               # tie of |x|: the first (negative) wins
    if nb > 3:
        x[blk(3)] = np.float32(0.3)                         # constant block
    if nb > 4:
        v = x[blk(4)]
        v[:] = (v * np.float32(1e-39)).astype(np.float32)   # subnormal inputs
        v[5] = np.float32(3e-38)
    if nb > 5:
        v = x[blk(5)]
        v[:] = np.round(v * 8.0) / 8.0                      # many exact halves after scaling
        v[9] = np.float32(-127.0 / 8.0)
    return x


def run_ref(wtype: int, rows: int, cols: int, w: np.ndarray, x: np.ndarray):
    nb = cols // 256
    with tempfile.TemporaryDirectory() as td:
        job, res = os.path.join(td, "job.bin"), os.path.join(td, "res.bin")
        with open(job, "wb") as f:
            f.write(struct.pack("<3i", wtype, rows, cols))
            f.write(w.tobytes())
            f.write(x.astype("<f4").tobytes())
        rc = subprocess.run([oracle.REF_QMV_BIN, job, res]).returncode
        if rc not in (0, 10):
            raise RuntimeError(f"kore_qmv_ref failed ({rc})")
        if rc == 10:
            raise RuntimeError("this CPU has no AVX2: kore's AVX2 results cannot be recorded here")
        raw = open(res, "rb").read()
    xq = np.frombuffer(raw[:292 * nb], np.uint8).copy()
    outs = np.frombuffer(raw[292 * nb:], "<f4")
    assert outs.size == 2 * rows
    return xq, outs[:rows].copy(), outs[rows:].copy()


def run_ref_batch(wtype: int, rows: int, cols: int, B: int, w: np.ndarray, x: np.ndarray):
    with tempfile.TemporaryDirectory() as td:
        job, res = os.path.join(td, "job.bin"), os.path.join(td, "res.bin")
        with open(job, "wb") as f:
            f.write(struct.pack("<4i", wtype, rows, cols, B))
            f.write(w.tobytes())
            f.write(x.astype("<f4").tobytes())
        rc = subprocess.run([oracle.REF_QMV_BIN, "--batch", job, res]).returncode
        if rc != 0:
            raise RuntimeError(f"kore_qmv_ref --batch failed ({rc})")
        outs = np.fromfile(res, "<f4")
    assert outs.size == 2 * rows * B
    return outs[:rows * B].copy(), outs[rows * B:].copy()


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main():
    if not os.path.exists(oracle.REF_QMV_BIN):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "ref"], check=True)
    for name, wtype, rows, cols, seed in CASES:
        rng = np.random.default_rng(seed)
        w = synth_weights(wtype, rows, cols // 256, rng)
        x = synth_x(cols, rng)
        xq, out_ref, out_avx2 = run_ref(wtype, rows, cols, w, x)
        np.savez_compressed(os.path.join(HERE, f"qmv_{name}.npz"), weights=w, x=x, xq=xq,
                            out_ref=out_ref, out_avx2=out_avx2)
        man = {"name": name, "type": wtype, "rows": rows, "cols": cols, "seed": seed,
               "source": "kore.cpp quantize_row_q8_K, dot_q{4,6}_K_q8_K_{ref,avx2} via oracle/_ref/kore_qmv_ref",
               "sha256": {k: sha(v) for k, v in (("weights", w), ("x", x), ("xq", xq),
                                                  ("out_ref", out_ref), ("out_avx2", out_avx2))}}
        with open(os.path.join(HERE, f"qmv_{name}.json"), "w") as f:
            json.dump(man, f, indent=1)
        print(f"qmv_{name}: {rows} x {cols}, max|out| {float(np.max(np.abs(out_ref))):.4g}")
    for name, wtype, rows, cols, B, seed in BATCH_CASES:
        rng = np.random.default_rng(seed)
        w = synth_weights(wtype, rows, cols // 256, rng)
        x = np.stack([synth_x(cols, rng) for _ in range(B)])
        out_avx2, out_ref = run_ref_batch(wtype, rows, cols, B, w, x)
        np.savez_compressed(os.path.join(HERE, f"qmm_{name}.npz"), weights=w, x=x, out_avx2=out_avx2,
                            out_ref=out_ref)
        man = {"name": name, "type": wtype, "rows": rows, "cols": cols, "B": B, "seed": seed,
               "source": "kore.cpp matmul_batch_float (AVX2 and scalar) via oracle/_ref/kore_qmv_ref --batch",
               "sha256": {k: sha(v) for k, v in (("weights", w), ("x", x), ("out_avx2", out_avx2),
                                                  ("out_ref", out_ref))}}
        with open(os.path.join(HERE, f"qmm_{name}.json"), "w") as f:
            json.dump(man, f, indent=1)
        print(f"qmm_{name}: {rows} x {cols}, B {B}, max|out| {float(np.max(np.abs(out_avx2))):.4g}")


if __name__ == "__main__":
    main()
