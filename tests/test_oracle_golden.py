"""The C oracle reproduces kore's own outputs bit for bit.

The fixtures under tests/golden/ were written by tests/golden/make_golden.py,
which drives kore.cpp's real forward() (decode, kore.cpp:1397-1480) and
forward_batch() (prefill, kore.cpp:1486-1598) through oracle/ref_harness.cpp.
Every comparison here is exact: sha256 over the complete output streams and
the complete K/V caches, plus array equality on the stored samples.
"""
import numpy as np
import pytest

import oracle
from tests.golden import cases as C


def _replay(case):
    nl, nh, nkv, hd, ctx = (case[k] for k in ("n_layer", "n_head", "n_head_kv", "head_dim", "ctx"))
    kv = oracle.KV(nl, ctx, nh, nkv, hd, case["rope_base"])
    inv_f = oracle.inv_freq(hd, case["rope_base"])
    inputs, att, qr = [], [], []
    for st, (pos, nb) in enumerate(case["steps"]):
        out = None
        for layer in range(nl):
            q, k, v = C.step_inputs(case, st, layer)
            inputs += [q, k, v]
            if case["mode"] == "decode":
                out = kv.decode(layer, pos, q, k, v)[None, :]
            else:
                out = kv.prefill(layer, pos, np.tile(q, (nb, 1)), np.tile(k, (nb, 1)),
                                 np.tile(v, (nb, 1)), avx2=bool(case["avx2"]))
        # roped q of the last layer, per row (kore leaves it in e.q / e.bq)
        rows = []
        for z in range(nb):
            c, s = oracle.rope_cs(pos + z, hd, inv_f)
            rows.append(oracle.rope_neox(q, nh, hd, c, s))
        att.append(out)
        qr.append(np.stack(rows))
    return np.concatenate(inputs), att, qr, kv, inv_f


@pytest.mark.parametrize("name", [c["name"] for c in C.CASES])
def test_oracle_matches_kore_bitwise(name):
    man, data = C.load(name)
    case = C.case_by_name(name)
    inputs, att, qr, kv, inv_f = _replay(case)
    sha = man["sha256"]
    assert C.sha(inputs) == sha["inputs"], "synthetic input generator drifted"
    assert C.sha(inv_f) == sha["inv_freq"]
    np.testing.assert_array_equal(inv_f, data["inv_freq"])
    for st in case["sample_steps"]:
        rows = man["sample_rows"][str(st)]
        np.testing.assert_array_equal(qr[st][rows], data[f"qr_{st}"], err_msg=f"roped q step {st}")
        np.testing.assert_array_equal(att[st][rows], data[f"att_{st}"], err_msg=f"attention step {st}")
    assert C.sha(np.concatenate([a.reshape(-1) for a in qr])) == sha["q_roped"]
    assert C.sha(np.concatenate([a.reshape(-1) for a in att])) == sha["att"]
    kc, vc = kv.kcache(), kv.vcache()
    if case["keep_kv"]:
        np.testing.assert_array_equal(kc, data["kcache"])
        np.testing.assert_array_equal(vc, data["vcache"])
    else:
        np.testing.assert_array_equal(kc[:, man["kv_rows"], :], data["kc_rows"])
        np.testing.assert_array_equal(vc[:, man["kv_rows"], :], data["vc_rows"])
    assert C.sha(kc) == sha["kcache"]
    assert C.sha(vc) == sha["vcache"]
    kv.close()


def test_fixture_discriminates_fused_rope():
    """A RoPE whose multiply-subtract were contracted into an FMA (hipcc's
    default for HIP code) would not match kore's cache bits: the fixture check
    above is strong enough to catch that mistake."""
    man, data = C.load("decode_c1")
    case = C.case_by_name("decode_c1")
    hd, nkv = case["head_dim"], case["n_head_kv"]
    inv_f = data["inv_freq"]
    half = hd // 2
    mismatches = 0
    for pos in (3, 100, 400):
        _, k, _ = C.step_inputs(case, pos, 0)
        c, s = oracle.rope_cs(pos, hd, inv_f)
        x = k.reshape(nkv, hd).astype(np.float64)
        x0, x1 = x[:, :half], x[:, half:]
        # fma(x0, c, -(x1*s)): exact product, one rounding at the end
        fused_lo = (x0 * c - (x1 * s).astype(np.float32)).astype(np.float32)
        exact = data["kcache"][0, pos].reshape(nkv, hd)[:, :half]
        mismatches += int(np.sum(fused_lo != exact))
    assert mismatches > 0


def test_fixture_discriminates_scalar_vs_avx2_prefill():
    """kore's AVX2 and scalar prefill paths round differently; the two
    fixtures differ, and the oracle follows each (checked above)."""
    a = C.load("prefill_7b_avx2")[0]["sha256"]["att"]
    b = C.load("prefill_7b_scalar")[0]["sha256"]["att"]
    assert a != b
