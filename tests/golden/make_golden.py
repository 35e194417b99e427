#!/usr/bin/env python3
"""Write the golden fixtures of kore's attention path.

Runs kore's own forward()/forward_batch() through oracle/_ref/kore_ref (built
by ``make -C oracle ref`` from the kore.cpp sources; see
oracle/ref_harness.cpp) on the cases of ``cases.py`` and stores, per case:

* ``<case>.json``: the case, sha256 of every input and of kore's complete
  outputs (attention output and roped q of every step, the whole K and V
  caches, inv_freq);
* ``<case>.npz``: kore's outputs at the sampled steps, inv_freq, and either
  the whole KV cache or a few of its rows.

Needs the kore sources, so it runs only where they are present; the tests
read the fixtures it wrote.
"""
from __future__ import annotations

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
from tests.golden import cases as C  # noqa: E402


def run_case(case):
    nl, nh, nkv, hd, ctx = (case[k] for k in ("n_layer", "n_head", "n_head_kv", "head_dim", "ctx"))
    E, kvd = nh * hd, nkv * hd
    mode = 0 if case["mode"] == "decode" else 1
    steps = case["steps"]
    inputs = []
    with tempfile.TemporaryDirectory() as td:
        job = os.path.join(td, "job.bin")
        res = os.path.join(td, "res.bin")
        with open(job, "wb") as f:
            f.write(struct.pack("<8i", mode, nl, nh, nkv, hd, ctx, case["avx2"], len(steps)))
            f.write(struct.pack("<f", case["rope_base"]))
            for st, (pos, nb) in enumerate(steps):
                f.write(struct.pack("<2i", pos, nb))
                for layer in range(nl):
                    q, k, v = C.step_inputs(case, st, layer)
                    inputs += [q, k, v]
                    f.write(q.astype("<f4").tobytes())
                    f.write(k.astype("<f4").tobytes())
                    f.write(v.astype("<f4").tobytes())
        subprocess.run([oracle.REF_BIN, job, res], check=True)
        raw = np.fromfile(res, dtype="<f4")
    off = 0
    att, qr = [], []
    for pos, nb in steps:
        att.append(raw[off:off + nb * E].reshape(nb, E)); off += nb * E
        qr.append(raw[off:off + nb * E].reshape(nb, E)); off += nb * E
    n = nl * ctx * kvd
    kc = raw[off:off + n].reshape(nl, ctx, kvd); off += n
    vc = raw[off:off + n].reshape(nl, ctx, kvd); off += n
    inv_f = raw[off:off + hd // 2]; off += hd // 2
    assert off == raw.size, (off, raw.size)
    return np.concatenate(inputs), att, qr, kc, vc, inv_f


def main(names=None):
    if not os.path.exists(oracle.REF_BIN):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "ref"], check=True)
    for case in C.CASES:
        if names and case["name"] not in names:
            continue
        inputs, att, qr, kc, vc, inv_f = run_case(case)
        ctx = case["ctx"]
        last = sum(nb for _, nb in case["steps"])
        kv_rows = sorted({0, 1, last // 2, last - 1})
        man = dict(case)
        man["sha256"] = dict(
            inputs=C.sha(inputs),
            att=C.sha(np.concatenate([a.reshape(-1) for a in att])),
            q_roped=C.sha(np.concatenate([a.reshape(-1) for a in qr])),
            kcache=C.sha(kc), vcache=C.sha(vc), inv_freq=C.sha(inv_f))
        man["kv_rows"] = kv_rows
        man["filled"] = last
        man["generator"] = "kore.cpp forward()/forward_batch() via oracle/ref_harness.cpp"
        arrays = {"inv_freq": inv_f}
        sample_rows = {}
        for st in case["sample_steps"]:
            nb = case["steps"][st][1]
            rows = sorted({0, nb // 2, nb - 1})
            sample_rows[str(st)] = rows
            arrays[f"att_{st}"] = att[st][rows]
            arrays[f"qr_{st}"] = qr[st][rows]
        man["sample_rows"] = sample_rows
        if case["keep_kv"]:
            arrays["kcache"] = kc
            arrays["vcache"] = vc
        else:
            arrays["kc_rows"] = kc[:, kv_rows, :]
            arrays["vc_rows"] = vc[:, kv_rows, :]
        assert ctx >= last
        with open(C.manifest_path(case["name"]), "w") as f:
            json.dump(man, f, indent=1)
        np.savez_compressed(C.npz_path(case["name"]), **arrays)
        print(f"{case['name']}: steps={len(case['steps'])} att sha={man['sha256']['att'][:16]}")


if __name__ == "__main__":
    main(sys.argv[1:] or None)
