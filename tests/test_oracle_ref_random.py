"""The C oracle against kore's own forward()/forward_batch() on fresh random
inputs (not the committed fixtures): oracle/_ref/kore_ref, built from the
kore.cpp sources by `make -C oracle ref`, runs kore's code on the same job and
every output and cache bit must agree.  Skipped where the reference build is
absent (it needs the kore sources)."""
import os
import struct
import subprocess
import tempfile

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.skipif(not os.path.exists(oracle.REF_BIN), reason="kore's reference build is absent")


def _run_kore(mode, nl, nh, nkv, hd, ctx, avx2, steps, base, inputs):
    E, kvd = nh * hd, nkv * hd
    with tempfile.TemporaryDirectory() as td:
        job, res = os.path.join(td, "job.bin"), os.path.join(td, "res.bin")
        with open(job, "wb") as f:
            f.write(struct.pack("<8i", mode, nl, nh, nkv, hd, ctx, avx2, len(steps)))
            f.write(struct.pack("<f", base))
            for st, (pos, nb) in enumerate(steps):
                f.write(struct.pack("<2i", pos, nb))
                for l in range(nl):
                    for a in inputs[st][l]:
                        f.write(np.asarray(a, "<f4").tobytes())
        subprocess.run([oracle.REF_BIN, job, res], check=True)
        raw = np.fromfile(res, dtype="<f4")
    att, off = [], 0
    for pos, nb in steps:
        att.append(raw[off:off + nb * E].reshape(nb, E))
        off += 2 * nb * E                                   # att, then roped q
    n = nl * ctx * kvd
    kc = raw[off:off + n].reshape(nl, ctx, kvd)
    vc = raw[off + n:off + 2 * n].reshape(nl, ctx, kvd)
    return att, kc, vc


@pytest.mark.parametrize("mode,nh,nkv,hd,avx2,steps,seed", [
    (0, 28, 4, 128, 1, [[p, 1] for p in range(40)], 101),             # 7B decode geometry
    (0, 14, 2, 64, 1, [[p, 1] for p in range(33)], 102),              # 0.5B decode geometry
    (1, 16, 2, 128, 1, [[0, 9], [9, 1], [10, 30]], 103),               # 3B prefill, AVX2 helpers
    (1, 12, 2, 128, 0, [[0, 17], [17, 20]], 104),                      # 1.5B prefill, scalar helpers
    (1, 32, 8, 40, 1, [[0, 5], [5, 12]], 105),                         # head_dim 40: scalar tails (E % 256 == 0)
])
def test_oracle_matches_kore_on_random_inputs(mode, nh, nkv, hd, avx2, steps, seed):
    rng = np.random.default_rng(seed)
    nl, base = 2, float(rng.choice([1e4, 1e6]))
    ctx = sum(nb for _, nb in steps)
    E, kvd = nh * hd, nkv * hd
    # heavy-tailed values: N(0,1) with a few channels scaled x20 per step
    inputs = []
    for _ in steps:
        per = []
        for _ in range(nl):
            q, k, v = (rng.standard_normal(d).astype(np.float32) for d in (E, kvd, kvd))
            for a in (q, k, v):
                a[rng.integers(0, a.size, size=max(1, a.size // 100))] *= 20
            per.append((q, k, v))
        inputs.append(per)
    att, kc, vc = _run_kore(mode, nl, nh, nkv, hd, ctx, avx2, steps, base, inputs)
    kv = oracle.KV(nl, ctx, nh, nkv, hd, base)
    for st, (pos, nb) in enumerate(steps):
        for l in range(nl):
            q, k, v = inputs[st][l]
            if mode == 0:
                out = kv.decode(l, pos, q, k, v)[None, :]
            else:
                out = kv.prefill(l, pos, np.tile(q, (nb, 1)), np.tile(k, (nb, 1)), np.tile(v, (nb, 1)),
                                 avx2=bool(avx2))
        np.testing.assert_array_equal(out.view(np.uint32), att[st].view(np.uint32), err_msg=f"step {st}")
    np.testing.assert_array_equal(kv.kcache(), kc)
    np.testing.assert_array_equal(kv.vcache(), vc)
