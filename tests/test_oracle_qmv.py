"""The CPU oracle of kore's quantised matvec against kore's own outputs and
against what the block formats fix.

* Golden vectors: tests/golden/qmv_*.npz hold kore's quantize_row_q8_K blocks
  and kore's scalar and AVX2 dot products (kore.cpp:422-632) of synthetic
  Q4_K / Q6_K rows; the oracle must reproduce every bit.
* Formats, independently of the oracle's code: the dot product equals, up to
  fp32 rounding, the float64 product of the dequantised weights (the
  dequantisation written here from the block layouts, kore.cpp:324-381) with
  the dequantised Q8_K activations.
* The quantiser's closed forms: a constant block maps to -127 everywhere, a
  zero block to zeros, the first of two equal magnitudes sets the sign,
  sums of 16 are the sums of the int8 values.
"""
import json
import os

import numpy as np
import pytest

import oracle

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASES = sorted(f[4:-5] for f in os.listdir(GOLD) if f.startswith("qmv_") and f.endswith(".json"))


def _load(name):
    man = json.load(open(os.path.join(GOLD, f"qmv_{name}.json")))
    z = np.load(os.path.join(GOLD, f"qmv_{name}.npz"))
    return man, {k: z[k] for k in z.files}


def _bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def test_fixture_set_present():
    assert {"q4k_mix", "q6k_mix", "q6k_odd", "q4k_3584", "q6k_18944"} <= set(CASES)


@pytest.mark.parametrize("name", CASES)
def test_quantize_matches_kore_bits(name):
    man, z = _load(name)
    xq = oracle.quantize_q8K(z["x"])
    assert xq.view(np.uint8).tobytes() == z["xq"].tobytes()


@pytest.mark.parametrize("name", CASES)
@pytest.mark.parametrize("avx2", [False, True])
def test_matvec_matches_kore_bits(name, avx2):
    man, z = _load(name)
    xq = np.frombuffer(z["xq"].tobytes(), oracle.Q8K_DTYPE)
    out = oracle.qmatvec(man["type"], z["weights"], man["rows"], man["cols"], xq, avx2=avx2)
    assert _bits_equal(out, z["out_avx2" if avx2 else "out_ref"])


def test_scalar_and_avx2_orders_differ_on_the_fixtures():
    # the two summation orders are distinct functions: each fixture pins both
    for name in CASES:
        man, z = _load(name)
        assert not _bits_equal(z["out_ref"], z["out_avx2"]), name


@pytest.mark.parametrize("name", [c for c in CASES if c.startswith("q6k")])
def test_q6k_bias_step_is_one_fused_multiply_add(name):
    man, z = _load(name)
    xq = np.frombuffer(z["xq"].tobytes(), oracle.Q8K_DTYPE)
    nb = man["cols"] // 256
    rb = nb * 210
    rows = [z["weights"][r * rb:(r + 1) * rb] for r in range(man["rows"])]
    fused = np.array([oracle.dot(oracle.TYPE_Q6K, w, xq, True, 1) for w in rows], np.float32)
    split = np.array([oracle.dot(oracle.TYPE_Q6K, w, xq, True, 0) for w in rows], np.float32)
    assert _bits_equal(fused, z["out_avx2"])
    assert not _bits_equal(split, z["out_avx2"])


# ---------------------------------------------------------------- formats

def _f16(b2):
    return np.frombuffer(bytes(b2), "<f2").astype(np.float64)[0]


def dequant_q4k(block: np.ndarray) -> np.ndarray:
    """256 values of one Q4_K block: eight 32-value sub-blocks, sub-block j
    from the low (j even) or high (j odd) nibbles of bytes 16+32*(j//2)...,
    value = d * scale_j * nibble - dmin * min_j with 6-bit scale/min pairs
    packed in bytes 4..15."""
    d, dmin = _f16(block[0:2]), _f16(block[2:4])
    s = block[4:16].astype(np.int64)
    sc = np.zeros(8, np.int64)
    mn = np.zeros(8, np.int64)
    sc[:4], mn[:4] = s[0:4] & 63, s[4:8] & 63
    sc[4:] = (s[8:12] & 15) | ((s[0:4] >> 6) << 4)
    mn[4:] = (s[8:12] >> 4) | ((s[4:8] >> 6) << 4)
    qs = block[16:144].astype(np.int64).reshape(4, 32)
    out = np.zeros(256)
    for j in range(8):
        nib = (qs[j // 2] & 15) if j % 2 == 0 else (qs[j // 2] >> 4)
        out[32 * j:32 * j + 32] = d * sc[j] * nib - dmin * mn[j]
    return out


def dequant_q6k(block: np.ndarray) -> np.ndarray:
    """256 values of one Q6_K block: value v = 128h + 32k + l has its low
    four bits in byte 64h + 32(k&1) + l (low nibble for k < 2, high above),
    its top two bits at bits 2k..2k+1 of byte 128 + 32h + l, and scale
    int8[192 + 8h + 2k + l//16]; value = d * scale * (q - 32)."""
    ql = block[0:128].astype(np.int64)
    qh = block[128:192].astype(np.int64)
    sc = block[192:208].view(np.int8).astype(np.int64)
    d = _f16(block[208:210])
    out = np.zeros(256)
    for h in range(2):
        for k in range(4):
            l = np.arange(32)
            lo = ql[64 * h + 32 * (k & 1) + l]
            lo = (lo & 15) if k < 2 else (lo >> 4)
            q = lo | (((qh[32 * h + l] >> (2 * k)) & 3) << 4)
            out[128 * h + 32 * k + l] = d * sc[8 * h + 2 * k + l // 16] * (q - 32)
    return out


@pytest.mark.parametrize("name", CASES)
def test_dot_equals_dequantised_product(name):
    man, z = _load(name)
    t, rows, cols = man["type"], man["rows"], man["cols"]
    nb, bb = cols // 256, oracle.BLOCK_BYTES[t]
    xq = np.frombuffer(z["xq"].tobytes(), oracle.Q8K_DTYPE)
    xd = (xq["d"].astype(np.float64)[:, None] * xq["qs"].astype(np.float64)).reshape(-1)
    deq = dequant_q4k if t == oracle.TYPE_Q4K else dequant_q6k
    w = z["weights"].reshape(rows, nb, bb)
    for avx2 in (False, True):
        out = z["out_avx2" if avx2 else "out_ref"].astype(np.float64)
        for r in range(rows):
            wd = np.concatenate([deq(w[r, i]) for i in range(nb)])
            exact = float(np.dot(wd, xd))
            mag = float(np.sum(np.abs(wd * xd))) + 1e-30
            assert abs(out[r] - exact) <= 2e-6 * mag, (name, avx2, r, out[r], exact, mag)


# ---------------------------------------------------------------- quantiser

def test_quantize_constant_block():
    for c in (0.3, -2.5, 1e-20, 3e38):
        xq = oracle.quantize_q8K(np.full(256, c, np.float32))[0]
        assert np.all(xq["qs"] == -127)
        assert np.all(xq["bsums"] == -127 * 16)
        iscale = np.float32(-127.0) / np.float32(c)
        assert xq["d"] == np.float32(1.0) / iscale


def test_quantize_zero_block():
    xq = oracle.quantize_q8K(np.zeros(512, np.float32))
    assert np.all(xq["d"] == 0) and np.all(xq["qs"] == 0) and np.all(xq["bsums"] == 0)


def test_quantize_tie_first_wins():
    x = np.linspace(-1, 1, 256).astype(np.float32)
    x[10], x[100] = 4.0, -4.0
    q = oracle.quantize_q8K(x)[0]
    assert q["qs"][10] == -127 and q["qs"][100] == 127 and q["d"] < 0
    x[10], x[100] = -4.0, 4.0
    q = oracle.quantize_q8K(x)[0]
    assert q["qs"][10] == -127 and q["qs"][100] == 127 and q["d"] > 0


def test_quantize_rounds_half_to_even_and_sums():
    # maxv = -127 gives iscale = 1 exactly: qs = rint(x), halves to even
    x = np.zeros(256, np.float32)
    x[0] = -127.0
    x[1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, 126.5, -3.5, 2.4999998]
    q = oracle.quantize_q8K(x)[0]
    assert list(q["qs"][:9]) == [-127, 0, 2, 2, 0, -2, 126, -4, 2]
    assert np.array_equal(q["bsums"], q["qs"].astype(np.int64).reshape(16, 16).sum(1))
    assert q["d"] == np.float32(1.0)


def test_quantize_matches_numpy_restatement_on_random_blocks():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(256 * 64) * rng.choice([1e-3, 1.0, 50.0], 256 * 64)).astype(np.float32)
    q = oracle.quantize_q8K(x)
    xb = x.reshape(64, 256)
    first = np.argmax(np.abs(xb), axis=1)            # first index of the largest magnitude
    maxv = xb[np.arange(64), first]
    iscale = (np.float32(-127.0) / maxv).astype(np.float32)
    qs = np.minimum(np.rint((iscale[:, None] * xb).astype(np.float32)), 127).astype(np.int8)
    assert np.array_equal(q["qs"], qs)
    assert np.array_equal(q["d"], (np.float32(1.0) / iscale).astype(np.float32))


# ---------------------------------------------------------------- batched matmul

BATCH = sorted(f[4:-5] for f in os.listdir(GOLD) if f.startswith("qmm_") and f.endswith(".json"))


def _load_batch(name):
    man = json.load(open(os.path.join(GOLD, f"qmm_{name}.json")))
    z = np.load(os.path.join(GOLD, f"qmm_{name}.npz"))
    return man, {k: z[k] for k in z.files}


def test_batch_fixture_set_present():
    assert {"q4k_b5", "q6k_b64", "q4k_b13_odd", "q6k_b1"} <= set(BATCH)


@pytest.mark.parametrize("name", BATCH)
@pytest.mark.parametrize("avx2", [False, True])
def test_matmul_batch_matches_kore_bits(name, avx2):
    man, z = _load_batch(name)
    out = oracle.matmul_batch(man["type"], z["weights"], man["rows"], man["cols"], z["x"], avx2=avx2)
    assert _bits_equal(out.reshape(-1), z["out_avx2" if avx2 else "out_ref"])


def test_matmul_batch_orders_differ():
    for name in BATCH:
        man, z = _load_batch(name)
        assert not _bits_equal(z["out_avx2"], z["out_ref"]), name


@pytest.mark.parametrize("name", BATCH)
def test_dequant_and_batch_against_float64(name):
    """kore's float dequantisation equals the block layout's values to fp32
    rounding, and every output is the float64 dot product of those values
    with x to within fp32 accumulation error."""
    man, z = _load_batch(name)
    t, rows, cols = man["type"], man["rows"], man["cols"]
    nb, bb = cols // 256, oracle.BLOCK_BYTES[t]
    deq = dequant_q4k if t == oracle.TYPE_Q4K else dequant_q6k
    w = z["weights"].reshape(rows, nb, bb)
    x = z["x"].astype(np.float64)
    for r in range(rows):
        exact = np.concatenate([deq(w[r, i]) for i in range(nb)])
        got = oracle.dequant_row(t, w[r].reshape(-1), cols).astype(np.float64)
        assert np.all(np.abs(got - exact) <= 2.5e-7 * np.abs(exact) + 1e-30), (name, r)
        ref = x @ exact
        mag = np.abs(x) @ np.abs(exact) + 1e-30
        for key in ("out_avx2", "out_ref"):
            o = z[key].reshape(man["B"], rows)[:, r].astype(np.float64)
            assert np.all(np.abs(o - ref) <= 1e-5 * mag), (name, key, r)
