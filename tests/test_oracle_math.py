"""Checks of the oracle that do not rely on kore: closed forms, invariants and
a double-precision brute force.  These pin what the golden fixtures leave
open (other seeds and shapes, the sliding-window decode kore does not have,
the synthetic generator) and each is chosen so that a plausible slip (wrong
sign, swapped pair, wrong kv-head, dropped scale) fails it."""
import math

import numpy as np
import pytest

import oracle


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


# ------------------------------------------------------------------- RoPE

def test_inv_freq_closed_form():
    for hd, base in ((64, 1e6), (128, 1e6), (128, 1e4), (40, 5e5)):
        f = oracle.inv_freq(hd, base)
        expect = np.array([np.float32(base ** (-2.0 * i / hd)) for i in range(hd // 2)], np.float32)
        np.testing.assert_array_equal(f, expect)
        assert f[0] == 1.0


def test_rope_pos0_is_identity_and_v_is_copied():
    kv = oracle.KV(1, 8, 4, 2, 64, 1e6)
    q, k, v = _rand(256, 1), _rand(128, 2), _rand(128, 3)
    kv.decode(0, 0, q, k, v)
    np.testing.assert_array_equal(kv.kcache()[0, 0], k)   # cos 0 = 1, sin 0 = 0
    np.testing.assert_array_equal(kv.vcache()[0, 0], v)
    kv.decode(0, 5, q, k, v)
    np.testing.assert_array_equal(kv.vcache()[0, 5], v)   # V is never rotated
    assert not np.array_equal(kv.kcache()[0, 5], k)


def test_rope_rotation_matches_complex_multiply():
    """NEOX pairs (i, i+hd/2) rotate by angle pos*inv_freq[i]."""
    hd, nh = 128, 3
    inv_f = oracle.inv_freq(hd, 1e6)
    x = _rand(nh * hd, 4)
    for pos in (1, 17, 4095, 32767):
        c, s = oracle.rope_cs(pos, hd, inv_f)
        y = oracle.rope_neox(x, nh, hd, c, s).reshape(nh, hd).astype(np.float64)
        xx = x.reshape(nh, hd).astype(np.float64)
        ang = pos * inv_f.astype(np.float64)
        z = (xx[:, :hd // 2] + 1j * xx[:, hd // 2:]) * np.exp(1j * ang)
        np.testing.assert_allclose(y[:, :hd // 2], z.real, atol=2e-5 * (1 + pos / 1000))
        np.testing.assert_allclose(y[:, hd // 2:], z.imag, atol=2e-5 * (1 + pos / 1000))
        # norm preserved per pair
        np.testing.assert_allclose(np.hypot(y[:, :hd // 2], y[:, hd // 2:]),
                                   np.abs(z), rtol=1e-5)


def test_rope_relative_position():
    """<R(m)q, R(n)k> depends only on m - n."""
    hd = 128
    inv_f = oracle.inv_freq(hd, 1e4)
    q, k = _rand(hd, 5), _rand(hd, 6)

    def rot(x, p):
        c, s = oracle.rope_cs(p, hd, inv_f)
        return oracle.rope_neox(x, 1, hd, c, s).astype(np.float64)

    base = rot(q, 10) @ rot(k, 3)
    for m in (50, 200, 1007):
        assert abs(rot(q, m) @ rot(k, m - 7) - base) < 1e-3 * (1 + abs(base))


# -------------------------------------------------------------- attention

def test_decode_pos0_returns_v_exactly():
    nh, nkv, hd = 14, 2, 64
    kv = oracle.KV(1, 4, nh, nkv, hd, 1e6)
    q, k, v = _rand(nh * hd, 7), _rand(nkv * hd, 8), _rand(nkv * hd, 9)
    out = kv.decode(0, 0, q, k, v).reshape(nh, hd)
    vr = v.reshape(nkv, hd)
    for h in range(nh):
        np.testing.assert_array_equal(out[h], vr[h // (nh // nkv)])


def test_decode_zero_query_gives_mean_of_v():
    nh, nkv, hd, n = 8, 2, 64, 37
    kv = oracle.KV(1, 64, nh, nkv, hd, 1e6)
    vs = []
    for p in range(n):
        v = _rand(nkv * hd, 100 + p)
        vs.append(v)
        out = kv.decode(0, p, np.zeros(nh * hd, np.float32), _rand(nkv * hd, 200 + p), v)
    mean = np.mean(np.stack(vs).astype(np.float64), axis=0).reshape(nkv, hd)
    out = out.reshape(nh, hd)
    for h in range(nh):
        np.testing.assert_allclose(out[h], mean[h // (nh // nkv)], rtol=0, atol=2e-6)


def test_gqa_heads_share_their_kv_head():
    """Two q-heads of one group with the same q give the same output; heads
    of different groups (different K/V) do not."""
    nh, nkv, hd = 6, 2, 64
    kv = oracle.KV(1, 32, nh, nkv, hd, 1e6)
    for p in range(20):
        qh = _rand(hd, 300 + p)
        q = np.tile(qh, nh)
        out = kv.decode(0, p, q, _rand(nkv * hd, 400 + p), _rand(nkv * hd, 500 + p)).reshape(nh, hd)
    np.testing.assert_array_equal(out[0], out[1])
    np.testing.assert_array_equal(out[3], out[5])
    assert not np.allclose(out[0], out[3])


@pytest.mark.parametrize("nh,nkv,hd,n", [(14, 2, 64, 300), (28, 4, 128, 150), (16, 2, 128, 90)])
def test_decode_matches_double_brute_force(nh, nkv, hd, n):
    kv = oracle.KV(1, n, nh, nkv, hd, 1e6)
    inv_f = oracle.inv_freq(hd, 1e6)
    for p in range(n):
        q = _rand(nh * hd, 1000 + p) * 3
        out = kv.decode(0, p, q, _rand(nkv * hd, 2000 + p), _rand(nkv * hd, 3000 + p))
    c, s = oracle.rope_cs(n - 1, hd, inv_f)
    qr = oracle.rope_neox(q, nh, hd, c, s)
    ref = oracle.attn_ref64(qr, kv.kcache()[0], kv.vcache()[0], np.arange(n), nh, nkv, hd)
    assert np.max(np.abs(out - ref)) <= 1e-5 * np.max(np.abs(ref))


@pytest.mark.parametrize("avx2", [True, False])
def test_prefill_rows_equal_decode(avx2):
    """Prefill row z attends exactly what a decode at pos0+z attends."""
    nh, nkv, hd, n0, nb = 14, 2, 128, 20, 33
    a = oracle.KV(1, 64, nh, nkv, hd, 1e6)
    b = oracle.KV(1, 64, nh, nkv, hd, 1e6)
    q = _rand((n0 + nb, nh * hd), 11)
    k = _rand((n0 + nb, nkv * hd), 12)
    v = _rand((n0 + nb, nkv * hd), 13)
    a.prefill(0, 0, q[:n0], k[:n0], v[:n0], avx2=avx2)
    outp = a.prefill(0, n0, q[n0:], k[n0:], v[n0:], avx2=avx2)
    outd = np.stack([b.decode(0, p, q[p], k[p], v[p]) for p in range(n0 + nb)])
    np.testing.assert_array_equal(a.kcache(), b.kcache())
    np.testing.assert_array_equal(a.vcache(), b.vcache())
    assert np.max(np.abs(outp - outd[n0:])) <= 1e-5 * np.max(np.abs(outd))


def test_window_decode_matches_brute_force_over_last_w():
    nh, nkv, hd, W, n = 12, 2, 128, 64, 150
    kv = oracle.KV(1, W, nh, nkv, hd, 1e6, window=W)
    ks, vs = [], []
    for p in range(n):
        q = _rand(nh * hd, 5000 + p)
        k, v = _rand(nkv * hd, 6000 + p), _rand(nkv * hd, 7000 + p)
        out = kv.decode(0, p, q, k, v)
        c, s = oracle.rope_cs(p, hd, oracle.inv_freq(hd, 1e6))
        ks.append(oracle.rope_neox(k, nkv, hd, c, s))
        vs.append(v)
    # ring slot of position p is p % W
    np.testing.assert_array_equal(kv.kcache()[0, (n - 1) % W], ks[-1])
    np.testing.assert_array_equal(kv.vcache()[0, (n - 2) % W], vs[-2])
    qr = oracle.rope_neox(q, nh, hd, c, s)
    K = np.stack(ks[n - W:])
    V = np.stack(vs[n - W:])
    ref = oracle.attn_ref64(qr, K, V, np.arange(W), nh, nkv, hd)
    assert np.max(np.abs(out - ref)) <= 1e-5 * np.max(np.abs(ref))


def test_kore_guards():
    kv = oracle.KV(2, 16, 4, 2, 64, 1e6)
    z = np.zeros(256, np.float32)
    with pytest.raises(ValueError):
        kv.decode(0, 16, z, z[:128], z[:128])          # pos >= ctx (kore.cpp:1400)
    with pytest.raises(ValueError):
        kv.decode(2, 0, z, z[:128], z[:128])           # bad layer
    with pytest.raises(ValueError):
        kv.prefill(0, 10, np.zeros((7, 256), np.float32), np.zeros((7, 128), np.float32),
                   np.zeros((7, 128), np.float32))      # pos0 + nb > ctx (kore.cpp:1490)
    with pytest.raises(ValueError):
        oracle.KV(1, 16, 6, 4, 64)                      # n_head % n_head_kv (kore.cpp:1278)
    with pytest.raises(ValueError):
        oracle.KV(1, 16, 4, 2, 63)                      # odd head_dim (kore.cpp:1288)


# ------------------------------------------------------------- hd_dot/fma

def test_hd_dot_avx2_order():
    """The AVX2 dot is lane-wise FMA over two 8-lane accumulators and an
    hsum256 tree; restated here in float64-then-round per step."""
    a, b = _rand(128, 21), _rand(128, 22)
    acc = np.zeros((2, 8), np.float32)
    for i in range(0, 128, 16):
        for h in range(2):
            prod = a[i + 8 * h:i + 8 * h + 8].astype(np.float64) * b[i + 8 * h:i + 8 * h + 8]
            acc[h] = (prod + acc[h]).astype(np.float32)   # exact product, one rounding
    v = (acc[0] + acc[1]).astype(np.float32)
    lo = (v[:4] + v[4:]).astype(np.float32)
    s = np.float32(np.float32(lo[0] + lo[2]) + np.float32(lo[1] + lo[3]))
    assert oracle.hd_dot(a, b, True) == s
    seq = np.float32(0)
    for x, y in zip(a, b):
        seq = np.float32(seq + np.float32(x * y))
    assert oracle.hd_dot(a, b, False) == seq


# --------------------------------------------------------------- generator

def test_synth_generator_exact_restatement():
    """Python restatement of the generator formula from its definition."""
    M = (1 << 64) - 1

    def sm(x):
        z = (x + 0x9E3779B97F4A7C15) & M
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        return z ^ (z >> 31)

    seed, stream = 1234, (2 << 32) | 5
    key = sm(sm(seed) ^ stream)
    got = oracle.synth(3, 7, seed, stream, row0=4)
    for r in range(3):
        for c in range(7):
            idx = (4 + r) * 7 + c
            tot = 0
            for kk in range(6):
                h = sm(key ^ ((idx * 8 + kk) & M))
                tot += (h & 0xFFFFFF) + ((h >> 32) & 0xFFFFFF)
            expect = np.float32(np.float32(tot - 6 * (1 << 24)) * np.float32(2.0 ** -24))
            assert got[r, c] == expect
    assert oracle.splitmix64(0) == sm(0)


def test_synth_statistics_and_outliers():
    x = oracle.synth(2000, 512, 7, 1)
    assert abs(float(x.mean())) < 5e-3 and abs(float(x.std()) - 1) < 5e-3
    y = oracle.synth(50, 3584, 7, 1, tensor=1, per_mille=10, outlier_scale=20.0)
    big = np.abs(y).max(axis=0) > 6.0
    frac = big.mean()
    assert 0.005 < frac < 0.02           # about 1 % of the channels
    z = oracle.synth(50, 3584, 7, 1)
    np.testing.assert_array_equal(y[:, big], z[:, big] * np.float32(20.0))
    np.testing.assert_array_equal(y[:, ~big], z[:, ~big])
    assert math.isclose(float(np.var(oracle.synth(1, 200000, 3, 9))), 1.0, rel_tol=0.02)
