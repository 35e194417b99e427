"""GPU parity of the generic-geometry kernels: every even head_dim up to 256
and any number of q-heads per kv-head that kore accepts (kore.cpp:1278-1290)
and the MFMA kernels do not cover (head_dim other than 64 / 128, or more than
8 q-heads per kv-head in the decode).

Bar as everywhere: K/V cache rows bit-identical to the oracle's (kore's RoPE),
attention outputs within max|d| <= 1e-4 * max|ref| of the oracle's
restatement of kore's loops.  kore's own outputs at head_dim 40 and 36 are
checked by tests/test_gpu_parity.py::test_golden_replay (prefill fixtures).
"""
import sys

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def _close(out, ref, what=""):
    ref = np.asarray(ref, np.float64)
    err = float(np.max(np.abs(np.asarray(out, np.float64) - ref)))
    scale = float(np.max(np.abs(ref)))
    assert err <= TOL * scale, f"{what}: max|d| = {err:.3e} > 1e-4 * {scale:.3e}"


def _attn(*a, **kw):
    from kore_amd import KoreAttn
    return KoreAttn(*a, **kw)


# (n_head, n_head_kv, head_dim): head_dims 40 / 36 of the golden fixtures,
# 96, 256 (largest), 2 and 6 (smallest tiles), and 12 / 16 q-heads per
# kv-head at head_dim 128 / 64 (the MFMA prefill, generic decode).
GEOMETRIES = [(32, 8, 40), (64, 16, 36), (33, 3, 96), (8, 2, 256), (4, 1, 2), (6, 3, 6),
              (24, 2, 128), (16, 1, 64)]


@pytest.mark.parametrize("nh,nkv,hd", GEOMETRIES)
def test_generic_prefill_then_decode(nh, nkv, hd):
    """Prefill chunks (one of a single row) and then decode steps, every
    output against the oracle's kore loops, the whole cache bitwise."""
    ctx, steps = 200, [(0, 70), (70, 1), (71, 45)]
    _say(f"generic prefill+decode {nh}/{nkv}/{hd}")
    rng = np.random.default_rng(hd * 1000 + nh)
    kv = oracle.KV(1, ctx, nh, nkv, hd, 1e6)
    with _attn(1, ctx, nh, nkv, hd, 1e6) as attn:
        for pos0, n in steps:
            q = rng.standard_normal((n, nh * hd)).astype(np.float32)
            k = rng.standard_normal((n, nkv * hd)).astype(np.float32)
            v = rng.standard_normal((n, nkv * hd)).astype(np.float32)
            _close(attn.prefill(0, pos0, q, k, v), kv.prefill(0, pos0, q, k, v), f"prefill {pos0}+{n}")
        for pos in range(116, ctx):
            q = rng.standard_normal(nh * hd).astype(np.float32)
            k = rng.standard_normal(nkv * hd).astype(np.float32)
            v = rng.standard_normal(nkv * hd).astype(np.float32)
            _close(attn.decode(0, pos, q, k, v), kv.decode(0, pos, q, k, v), f"decode {pos}")
        kg, vg = attn.read_kv(0, 0, ctx)
    np.testing.assert_array_equal(kg, kv.kcache()[0])
    np.testing.assert_array_equal(vg, kv.vcache()[0])


@pytest.mark.parametrize("nh,nkv,hd,n0", [(32, 8, 40, 3000), (24, 2, 128, 5000), (8, 2, 256, 2100)])
def test_generic_long_context(nh, nkv, hd, n0):
    """A long generic prefill (many key tiles per row) and a decode over many
    splits (the merge of split partials): sampled prefill rows and the
    decode against the oracle, the cache bitwise against kore's RoPE."""
    _say(f"generic long context {nh}/{nkv}/{hd} rows {n0}")
    seed = 17
    q0 = oracle.synth(n0, nh * hd, seed, 1 << 32)
    k0 = oracle.synth(n0, nkv * hd, seed, 2 << 32)
    v0 = oracle.synth(n0, nkv * hd, seed, 3 << 32)
    inv_f = oracle.inv_freq(hd, 1e6)
    ctx = n0 + 1
    with _attn(1, ctx, nh, nkv, hd, 1e6) as attn:
        outs = attn.prefill(0, 0, q0, k0, v0)
        q = oracle.synth(1, nh * hd, seed, 1 << 32, row0=n0)[0]
        k = oracle.synth(1, nkv * hd, seed, 2 << 32, row0=n0)[0]
        v = oracle.synth(1, nkv * hd, seed, 3 << 32, row0=n0)[0]
        out = attn.decode(0, n0, q, k, v)
        kg, vg = attn.read_kv(0, 0, ctx)
    K = oracle.rope_rows(np.concatenate([k0, k[None]]), np.arange(ctx), nkv, hd, inv_f)
    V = np.concatenate([v0, v[None]])
    np.testing.assert_array_equal(kg, K)
    np.testing.assert_array_equal(vg, V)
    for z in (0, 1, 63, 64, n0 // 2, n0 - 1):
        qr = oracle.rope_rows(q0[z:z + 1], [z], nh, hd, inv_f)
        ref = oracle.attn_batch(qr, z, K, V, nh, nkv, hd)[0]
        _close(outs[z], ref, f"prefill row {z}")
    qr = oracle.rope_rows(q[None], [n0], nh, hd, inv_f)[0]
    _close(out, oracle.attn_decode(qr, K, V, n0, nh, nkv, hd), f"decode pos {n0}")


@pytest.mark.parametrize("nh,nkv,hd,W", [(32, 8, 40, 100), (24, 2, 128, 70)])
def test_generic_window_decode(nh, nkv, hd, W):
    """Sliding ring of W slots on the generic decode: two turns past W, the
    new slot holding the new row, every output and the ring bitwise."""
    _say(f"generic window {W} {nh}/{nkv}/{hd}")
    kv = oracle.KV(1, W, nh, nkv, hd, 1e6, window=W)
    rng = np.random.default_rng(W * 7 + hd)
    with _attn(1, W, nh, nkv, hd, 1e6, window=W) as attn:
        q = rng.standard_normal((W, nh * hd)).astype(np.float32)
        k = rng.standard_normal((W, nkv * hd)).astype(np.float32)
        v = rng.standard_normal((W, nkv * hd)).astype(np.float32)
        _close(attn.prefill(0, 0, q, k, v), kv.prefill(0, 0, q, k, v), "window prefill")
        for p in range(W, 3 * W + 1):
            q = rng.standard_normal(nh * hd).astype(np.float32)
            k = rng.standard_normal(nkv * hd).astype(np.float32)
            v = rng.standard_normal(nkv * hd).astype(np.float32)
            _close(attn.decode(0, p, q, k, v), kv.decode(0, p, q, k, v), f"window pos {p}")
        kg, vg = attn.read_kv(0, 2 * W + 1, W)
    slots = np.arange(2 * W + 1, 3 * W + 1) % W
    np.testing.assert_array_equal(kg, kv.kcache()[0, slots])
    np.testing.assert_array_equal(vg, kv.vcache()[0, slots])
