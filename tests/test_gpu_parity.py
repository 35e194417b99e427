"""GPU parity: the HIP path through the C ABI against the oracle and kore's
own golden outputs.

Bar: K/V cache rows bit-identical to kore's (memcmp, as kore_kernels.cpp:760
checks its threads), attention outputs within max|d| <= 1e-4 * max|ref|
(kore_kernels.cpp:742).  Every test names its case before it touches the GPU.
"""
import sys

import numpy as np
import pytest

import oracle
from tests.golden import cases as C

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


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


# ---------------------------------------------------------------- golden

GPU_CASES = [c["name"] for c in C.CASES]


@pytest.mark.parametrize("name", GPU_CASES)
def test_golden_replay(name):
    """Replay a golden case through kore_attn_decode / kore_attn_prefill: the
    K/V caches must hash to kore's, the sampled outputs must match kore's to
    1e-4, and every step's output must match the oracle's to 1e-4."""
    man, data = C.load(name)
    case = C.case_by_name(name)
    nl, nh, nkv, hd, ctx = (case[k] for k in ("n_layer", "n_head", "n_head_kv", "head_dim", "ctx"))
    _say(f"golden {name} geometry {nh}/{nkv}/{hd} ctx {ctx} layers {nl}")
    kv = oracle.KV(nl, ctx, nh, nkv, hd, case["rope_base"])
    with _attn(nl, ctx, nh, nkv, hd, case["rope_base"]) as attn:
        for st, (pos, nb) in enumerate(case["steps"]):
            for layer in range(nl):
                q, k, v = C.step_inputs(case, st, layer)
                if case["mode"] == "decode":
                    out = attn.decode(layer, pos, q, k, v)[None, :]
                    ref = kv.decode(layer, pos, q, k, v)[None, :]
                else:
                    Q, K, V = np.tile(q, (nb, 1)), np.tile(k, (nb, 1)), np.tile(v, (nb, 1))
                    out = attn.prefill(layer, pos, Q, K, V)
                    ref = kv.prefill(layer, pos, Q, K, V, avx2=bool(case["avx2"]))
                _close(out, ref, f"{name} step {st} layer {layer}")
            if st in case["sample_steps"]:
                rows = man["sample_rows"][str(st)]
                _close(out[rows], data[f"att_{st}"], f"{name} step {st} vs kore")
        filled = man["filled"]
        kc = np.stack([attn.read_kv(layer, 0, filled)[0] for layer in range(nl)])
        vc = np.stack([attn.read_kv(layer, 0, filled)[1] for layer in range(nl)])
    assert filled == ctx
    assert C.sha(kc) == man["sha256"]["kcache"], "K cache differs from kore's bits"
    assert C.sha(vc) == man["sha256"]["vcache"], "V cache differs from kore's bits"


def test_golden_rows_as_one_chunk():
    """kore's one-row forward_batch() steps with distinct q/k/v on every row
    (fixture prefill_rows_7b_avx2) replayed as ONE 64-row causal chunk: row z
    of the chunk attends positions 0..z like kore's row at step z, so every
    row must match kore's output to 1e-4 and the cache must hash to kore's."""
    name = "prefill_rows_7b_avx2"
    man, data = C.load(name)
    case = C.case_by_name(name)
    nh, nkv, hd, ctx = (case[k] for k in ("n_head", "n_head_kv", "head_dim", "ctx"))
    n = len(case["steps"])
    _say(f"golden {name} as one {n}-row chunk")
    rows = [C.step_inputs(case, st, 0) for st in range(n)]
    Q, K, V = (np.stack([r[i] for r in rows]) for i in range(3))
    with _attn(1, ctx, nh, nkv, hd, case["rope_base"]) as attn:
        out = attn.prefill(0, 0, Q, K, V)
        kc, vc = attn.read_kv(0, 0, n)
    for st in range(n):
        _close(out[st:st + 1], data[f"att_{st}"], f"{name} row {st} vs kore")
    assert C.sha(kc[None]) == man["sha256"]["kcache"], "K cache differs from kore's bits"
    assert C.sha(vc[None]) == man["sha256"]["vcache"], "V cache differs from kore's bits"


def test_head_dim_above_256_is_refused():
    import kore_amd
    _say("create with head_dim 258")
    with pytest.raises(kore_amd.KoreAttnError) as ei:
        _attn(1, 80, 4, 2, 258)
    assert ei.value.code == kore_amd.KORE_ATTN_E_UNSUPPORTED


# -------------------------------------------------------------- decode

DECODE_GEOMS = [(14, 2, 64), (28, 4, 128), (16, 2, 128), (12, 2, 128), (8, 8, 128), (40, 8, 128),
                (20, 4, 64), (24, 8, 64)]


@pytest.mark.parametrize("nh,nkv,hd", DECODE_GEOMS)
def test_decode_lengths(nh, nkv, hd):
    """Attended lengths across split boundaries (1 row up to 4 splits of
    every tile size), against kore's scalar decode."""
    lengths = [1, 2, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 256, 257, 300]
    ctx = max(lengths) + 1
    _say(f"decode lengths {nh}/{nkv}/{hd}")
    kv = oracle.KV(1, ctx, nh, nkv, hd, 1e6)
    rng = np.random.default_rng(nh * 1000 + hd)
    with _attn(1, ctx, nh, nkv, hd, 1e6) as attn:
        for p in range(max(lengths)):
            q = rng.standard_normal(nh * hd).astype(np.float32) * 2
            k = rng.standard_normal(nkv * hd).astype(np.float32)
            v = rng.standard_normal(nkv * hd).astype(np.float32)
            out = attn.decode(0, p, q, k, v)
            ref = kv.decode(0, p, q, k, v)
            if p + 1 in lengths:
                _close(out, ref, f"L={p + 1}")
        kg, vg = attn.read_kv(0, 0, max(lengths))
    np.testing.assert_array_equal(kg, kv.kcache()[0, :max(lengths)])
    np.testing.assert_array_equal(vg, kv.vcache()[0, :max(lengths)])


def test_decode_7b_ctx4096_outliers():
    """Qwen2.5-7B decode shape at ctx 4096 with 1 % outlier channels x20, the
    benchmark's workload: layers 0 and 2 of a three-layer cache filled to 4096
    through the prefill append path, then 32 consecutive decode steps on both
    (layer-inner, like forward()), every output against kore's scalar decode
    and every appended row bit for bit; layer 1 stays untouched."""
    nh, nkv, hd, ctx, n0, steps = 28, 4, 128, 8192, 4096, 32
    layers = (0, 2)
    _say(f"decode 7b ctx4096 outliers: {steps} steps on layers {layers}")
    seed, pm = 7, 10
    inv_f = oracle.inv_freq(hd, 1e6)

    def rows(t, l, r0, n, dim):
        return oracle.synth(n, dim, seed, (t << 32) | l, row0=r0, tensor=t, per_mille=pm)

    K, V = {}, {}
    with _attn(3, ctx, nh, nkv, hd, 1e6) as attn:
        for l in layers:
            k0, v0 = rows(2, l, 0, n0, nkv * hd), rows(3, l, 0, n0, nkv * hd)
            attn.prefill(l, 0, rows(1, l, 0, n0, nh * hd), k0, v0)
            K[l] = np.zeros((n0 + steps, nkv * hd), np.float32)
            V[l] = np.zeros((n0 + steps, nkv * hd), np.float32)
            K[l][:n0], V[l][:n0] = oracle.rope_rows(k0, np.arange(n0), nkv, hd, inv_f), v0
            kg, vg = attn.read_kv(l, 0, n0)
            np.testing.assert_array_equal(kg, K[l][:n0])
            np.testing.assert_array_equal(vg, V[l][:n0])
        worst = 0.0
        for step in range(steps):
            pos = n0 + step
            for l in layers:
                q, k, v = rows(1, l, pos, 1, nh * hd)[0], rows(2, l, pos, 1, nkv * hd)[0], rows(3, l, pos, 1, nkv * hd)[0]
                out = attn.decode(l, pos, q, k, v)
                K[l][pos] = oracle.rope_rows(k[None], [pos], nkv, hd, inv_f)[0]
                V[l][pos] = v
                qr = oracle.rope_rows(q[None], [pos], nh, hd, inv_f)[0]
                ref = oracle.attn_decode(qr, K[l][:pos + 1], V[l][:pos + 1], pos, nh, nkv, hd)
                _close(out, ref, f"7b decode layer {l} pos {pos}")
                ref64 = np.asarray(ref, np.float64)
                worst = max(worst, float(np.max(np.abs(out - ref64)) / np.max(np.abs(ref64))))
        _say(f"decode 7b ctx4096 outliers: max rel err {worst:.3e}")
        for l in layers:
            kg, vg = attn.read_kv(l, n0, steps)
            np.testing.assert_array_equal(kg, K[l][n0:])
            np.testing.assert_array_equal(vg, V[l][n0:])
        # layer 1 untouched (zero-initialised like kore.cpp:1344)
        k_l1, v_l1 = attn.read_kv(1, 0, n0 + steps)
        assert not k_l1.any() and not v_l1.any()


def test_decode_3b_long_context():
    """Qwen2.5-3B shape, decode at position 32767 over a full cache, on two
    layers with different inputs: every cache row bit for bit, the outputs
    against the oracle."""
    nh, nkv, hd, ctx, nl = 16, 2, 128, 32768, 2
    n0 = ctx - 1
    seed = 9
    inv_f = oracle.inv_freq(hd, 1e6)
    with _attn(nl, ctx, nh, nkv, hd, 1e6) as attn:
        for l in range(nl):
            _say(f"decode 3b pos 32767 layer {l}")
            sq, sk, sv = (1 << 32) | l, (2 << 32) | l, (3 << 32) | l
            q0 = oracle.synth(n0, nh * hd, seed, sq)
            k0 = oracle.synth(n0, nkv * hd, seed, sk)
            v0 = oracle.synth(n0, nkv * hd, seed, sv)
            for p0 in range(0, n0, 8192):       # chunked prefill fills the cache
                n = min(8192, n0 - p0)
                attn.prefill(l, p0, q0[p0:p0 + n], k0[p0:p0 + n], v0[p0:p0 + n])
            del q0
            q = oracle.synth(1, nh * hd, seed, sq, row0=n0)[0]
            k = oracle.synth(1, nkv * hd, seed, sk, row0=n0)[0]
            v = oracle.synth(1, nkv * hd, seed, sv, row0=n0)[0]
            out = attn.decode(l, n0, q, k, v)
            kg, vg = attn.read_kv(l, 0, ctx)
            K = oracle.rope_rows(np.concatenate([k0, k[None]]), np.arange(ctx), nkv, hd, inv_f)
            V = np.concatenate([v0, v[None]])
            np.testing.assert_array_equal(kg, K)
            np.testing.assert_array_equal(vg, V)
            qr = oracle.rope_rows(q[None], [n0], nh, hd, inv_f)[0]
            _close(out, oracle.attn_decode(qr, K, V, n0, nh, nkv, hd), f"3b decode pos 32767 layer {l}")


@pytest.mark.parametrize("nh,nkv,hd,n0", [(40, 8, 128, 2600), (40, 8, 128, 2700), (20, 4, 64, 5200)])
def test_decode_extra_rows_and_multiblock_waves(nh, nkv, hd, n0):
    """Row counts where a split has more 16-row blocks than waves (a wave
    prefetches its second block) with and without extra rows past the last
    block, on 256 CUs: kv-heads 8 give 32 splits (2600 rows -> 82-row splits
    = 5 blocks + 2 extra rows, 2700 -> 96 = 6 blocks); kv-heads 4 give 64
    (5200 -> 82 = 5 blocks + 2 extra rows)."""
    _say(f"decode extra rows / multi-block {nh}/{nkv}/{hd} at {n0}")
    seed = 13
    q0 = oracle.synth(n0, nh * hd, seed, 1 << 32)
    k0 = oracle.synth(n0, nkv * hd, seed, 2 << 32)
    v0 = oracle.synth(n0, nkv * hd, seed, 3 << 32)
    inv_f = oracle.inv_freq(hd, 1e6)
    ctx = n0 + 4
    K = np.zeros((ctx, nkv * hd), np.float32)
    V = np.zeros((ctx, nkv * hd), np.float32)
    K[:n0] = oracle.rope_rows(k0, np.arange(n0), nkv, hd, inv_f)
    V[:n0] = v0
    with _attn(1, ctx, nh, nkv, hd, 1e6) as attn:
        attn.prefill(0, 0, q0, k0, v0)
        for pos in range(n0, n0 + 3):
            q = oracle.synth(1, nh * hd, seed, 1 << 32, row0=pos)[0]
            k = oracle.synth(1, nkv * hd, seed, 2 << 32, row0=pos)[0]
            v = oracle.synth(1, nkv * hd, seed, 3 << 32, row0=pos)[0]
            out = attn.decode(0, pos, q, k, v)
            K[pos] = oracle.rope_rows(k[None], [pos], nkv, hd, inv_f)[0]
            V[pos] = v
            qr = oracle.rope_rows(q[None], [pos], nh, hd, inv_f)[0]
            _close(out, oracle.attn_decode(qr, K, V, pos, nh, nkv, hd), f"pos {pos}")
        kg, vg = attn.read_kv(0, 0, n0 + 3)
    np.testing.assert_array_equal(kg, K[:n0 + 3])
    np.testing.assert_array_equal(vg, V[:n0 + 3])


@pytest.mark.parametrize("nh,nkv,hd,W", [(12, 2, 128, 260), (14, 2, 64, 130)])
def test_window_decode_stale_slot_on_extra_row(nh, nkv, hd, W):
    """Wrapped ring whose splits end in an extra row (W = 260: 16 splits of
    17 rows; W = 130: 8 of 17): over a full turn of the ring the stale copy of
    the new slot falls on every slot, extra rows included, and is masked."""
    _say(f"window {W} stale slot on extra rows {nh}/{nkv}/{hd}")
    kv = oracle.KV(1, W, nh, nkv, hd, 1e6, window=W)
    rng = np.random.default_rng(W + hd)
    with _attn(1, W, nh, nkv, hd, 1e6, window=W) as attn:
        q = rng.standard_normal((W, nh * hd)).astype(np.float32)
        k = rng.standard_normal((W, nkv * hd)).astype(np.float32)
        v = rng.standard_normal((W, nkv * hd)).astype(np.float32)
        _close(attn.prefill(0, 0, q, k, v), kv.prefill(0, 0, q, k, v), "window prefill")
        for p in range(W, 2 * W + 3):
            q = rng.standard_normal(nh * hd).astype(np.float32)
            k = rng.standard_normal(nkv * hd).astype(np.float32)
            v = rng.standard_normal(nkv * hd).astype(np.float32)
            _close(attn.decode(0, p, q, k, v), kv.decode(0, p, q, k, v), f"window pos {p}")
        kg, vg = attn.read_kv(0, W + 3, W)
    slots = np.arange(W + 3, 2 * W + 3) % W
    np.testing.assert_array_equal(kg, kv.kcache()[0, slots])
    np.testing.assert_array_equal(vg, kv.vcache()[0, slots])


def test_decode_deterministic():
    nh, nkv, hd, ctx = 28, 4, 128, 2048
    _say("decode determinism")
    outs = []
    for _ in range(2):
        with _attn(1, ctx, nh, nkv, hd, 1e6) as attn:
            rng = np.random.default_rng(5)
            attn.prefill(0, 0, rng.standard_normal((1500, nh * hd), np.float32),
                         rng.standard_normal((1500, nkv * hd), np.float32),
                         rng.standard_normal((1500, nkv * hd), np.float32))
            o = attn.decode(0, 1500, rng.standard_normal(nh * hd, np.float32),
                            rng.standard_normal(nkv * hd, np.float32),
                            rng.standard_normal(nkv * hd, np.float32))
            outs.append(o)
    np.testing.assert_array_equal(outs[0], outs[1])


def test_window_decode():
    """Sliding-window extension: ring of W slots, decode past W attends the
    last W positions."""
    nh, nkv, hd, W = 12, 2, 128, 256
    _say("window decode")
    kv = oracle.KV(1, W, nh, nkv, hd, 1e6, window=W)
    rng = np.random.default_rng(11)
    with _attn(1, W, nh, nkv, hd, 1e6, window=W) as attn:
        q = rng.standard_normal((200, nh * hd)).astype(np.float32)
        k = rng.standard_normal((200, nkv * hd)).astype(np.float32)
        v = rng.standard_normal((200, nkv * hd)).astype(np.float32)
        _close(attn.prefill(0, 0, q, k, v), kv.prefill(0, 0, q, k, v), "window prefill")
        for p in range(200, 700):
            q = rng.standard_normal(nh * hd).astype(np.float32)
            k = rng.standard_normal(nkv * hd).astype(np.float32)
            v = rng.standard_normal(nkv * hd).astype(np.float32)
            out = attn.decode(0, p, q, k, v)
            ref = kv.decode(0, p, q, k, v)
            if p % 50 == 0 or p in (255, 256, 257, 511, 512, 699):
                _close(out, ref, f"window pos {p}")
        kg, vg = attn.read_kv(0, 699 - W + 1, W)
    slots = np.arange(699 - W + 1, 700) % W
    np.testing.assert_array_equal(kg, kv.kcache()[0, slots])
    np.testing.assert_array_equal(vg, kv.vcache()[0, slots])


# ------------------------------------------------------------- prefill

PREFILL_CASES = [
    # nh, nkv, hd, [(pos0, n), ...]
    (28, 4, 128, [(0, 1), (1, 31), (32, 33), (65, 100), (165, 300)]),
    (14, 2, 64, [(0, 64), (64, 1), (65, 257)]),
    (12, 2, 128, [(0, 7), (7, 512)]),
    (16, 2, 128, [(0, 96), (96, 5)]),
    (8, 8, 128, [(0, 40), (40, 90)]),
    (40, 8, 128, [(0, 70)]),
    # short chunks over a longer cache: the key range is split into segments
    (28, 4, 128, [(0, 700), (700, 45)]),
    (14, 2, 64, [(0, 900), (900, 40)]),
    # between one and two workgroups per CU (256 CUs): the longest items run
    # as two key halves merged afterwards; 33 items per kv-head with the last
    # one half empty, and a chunk at an offset on head_dim 64
    (40, 8, 128, [(0, 830)]),
    (32, 8, 64, [(0, 300), (300, 1000)]),
]


@pytest.mark.parametrize("nh,nkv,hd,chunks", PREFILL_CASES)
def test_prefill_chunks(nh, nkv, hd, chunks):
    """Causal prefill chunks of ragged sizes and offsets against kore's AVX2
    batched attention; K/V rows bitwise."""
    ctx = sum(n for _, n in chunks)
    _say(f"prefill {nh}/{nkv}/{hd} chunks {chunks}")
    kv = oracle.KV(1, ctx, nh, nkv, hd, 1e6)
    rng = np.random.default_rng(nh + 7 * hd)
    with _attn(1, ctx, nh, nkv, hd, 1e6) as attn:
        for pos0, n in chunks:
            q = rng.standard_normal((n, nh * hd)).astype(np.float32)
            k = rng.standard_normal((n, nkv * hd)).astype(np.float32)
            v = rng.standard_normal((n, nkv * hd)).astype(np.float32)
            _close(attn.prefill(0, pos0, q, k, v), kv.prefill(0, pos0, q, k, v),
                   f"chunk {pos0}+{n}")
        kg, vg = attn.read_kv(0, 0, ctx)
    np.testing.assert_array_equal(kg, kv.kcache()[0])
    np.testing.assert_array_equal(vg, kv.vcache()[0])


def test_prefill_7b_2048_rows_vs_brute_force():
    """The 2048-token 7B prefill: sampled rows against the double brute
    force, every row against the oracle (kore's AVX2 batched attention), the
    cache rows bit for bit."""
    nh, nkv, hd, n = 28, 4, 128, 2048
    _say("prefill 7b 2048")
    seed = 3
    q = oracle.synth(n, nh * hd, seed, 1 << 32)
    k = oracle.synth(n, nkv * hd, seed, 2 << 32)
    v = oracle.synth(n, nkv * hd, seed, 3 << 32)
    inv_f = oracle.inv_freq(hd, 1e6)
    with _attn(1, n, nh, nkv, hd, 1e6) as attn:
        out = attn.prefill(0, 0, q, k, v)
        kg, vg = attn.read_kv(0, 0, n)
    K = oracle.rope_rows(k, np.arange(n), nkv, hd, inv_f)
    np.testing.assert_array_equal(kg, K)
    np.testing.assert_array_equal(vg, v)
    qr = oracle.rope_rows(q, np.arange(n), nh, hd, inv_f)
    for z in (0, 1, 31, 32, 500, 1023, 1024, 2047):
        ref = oracle.attn_ref64(qr[z], K, v, np.arange(z + 1), nh, nkv, hd)
        _close(out[z], ref, f"row {z}")
    # every row against kore's own arithmetic (the oracle's AVX2 batched
    # attention, kore.cpp:1542-1563): kore's 64-row chunks give each row the
    # same result as one 2048-row call
    kv = oracle.KV(1, n, nh, nkv, hd, 1e6)
    ref_all = kv.prefill(0, 0, q, k, v, avx2=True)
    kv.close()
    for z0 in range(0, n, 64):
        _close(out[z0:z0 + 64], ref_all[z0:z0 + 64], f"rows {z0}..{z0 + 63}")


def test_prefill_chunk_then_window_decode_1p5b():
    """Qwen2.5-1.5B shape: 1024-row chunk at 7168 onto a cache holding 7168
    positions, every row against the oracle's batched attention (kore's AVX2
    hd_dot / hd_fma arithmetic, kore.cpp:1542-1563) and every K/V row bit for
    bit; then all 256 decode steps sliding the window at 8192 (positions
    8192..8447) against the oracle's window decode, the ring's rows bit for bit
    after the last step."""
    from concurrent.futures import ThreadPoolExecutor
    nh, nkv, hd, W = 12, 2, 128, 8192
    _say("1.5b chunk at 7168 then sliding decode")
    seed = 5
    kv = oracle.KV(1, W, nh, nkv, hd, 1e6, window=W)
    with _attn(1, W, nh, nkv, hd, 1e6, window=W) as attn:
        q = oracle.synth(8192, nh * hd, seed, 1 << 32)
        k = oracle.synth(8192, nkv * hd, seed, 2 << 32)
        v = oracle.synth(8192, nkv * hd, seed, 3 << 32)
        attn.prefill(0, 0, q[:7168], k[:7168], v[:7168])
        kv_k, kv_v = kv.kcache(), kv.vcache()
        inv_f = oracle.inv_freq(hd, 1e6)
        out = attn.prefill(0, 7168, q[7168:], k[7168:], v[7168:])
        K = oracle.rope_rows(k, np.arange(8192), nkv, hd, inv_f)
        kg, vg = attn.read_kv(0, 0, 8192)
        np.testing.assert_array_equal(kg, K)
        np.testing.assert_array_equal(vg, v)
        kv_k[0] = K
        kv_v[0] = v
        qr = oracle.rope_rows(q[7168:], np.arange(7168, 8192), nh, hd, inv_f)

        def piece(z0):
            return oracle.attn_batch(qr[z0:z0 + 64], 7168 + z0, K[:7168 + z0 + 64], v[:7168 + z0 + 64], nh, nkv, hd,
                                     avx2=True)

        with ThreadPoolExecutor(max_workers=8) as ex:
            refs = list(ex.map(piece, range(0, 1024, 64)))
        for z0, ref in zip(range(0, 1024, 64), refs):
            _close(out[z0:z0 + 64], ref, f"chunk rows {z0}..{z0 + 63}")
        for p in range(8192, 8192 + 256):
            qd = oracle.synth(1, nh * hd, seed, 1 << 32, row0=p)[0]
            kd = oracle.synth(1, nkv * hd, seed, 2 << 32, row0=p)[0]
            vd = oracle.synth(1, nkv * hd, seed, 3 << 32, row0=p)[0]
            _close(attn.decode(0, p, qd, kd, vd), kv.decode(0, p, qd, kd, vd), f"decode {p}")
        kg, vg = attn.read_kv(0, 0, W)
        np.testing.assert_array_equal(kg, kv.kcache()[0])
        np.testing.assert_array_equal(vg, kv.vcache()[0])
    kv.close()


# --------------------------------------------------------- errors, misc

def test_error_codes():
    import kore_amd as ka
    _say("error codes")
    z = np.zeros(28 * 128, np.float32)
    zk = np.zeros(4 * 128, np.float32)
    with _attn(2, 64, 28, 4, 128) as attn:
        with pytest.raises(ka.KoreAttnError) as e:
            attn.decode(0, 64, z, zk, zk)                       # kore.cpp:1400
        assert e.value.code == ka.KORE_ATTN_E_RANGE
        with pytest.raises(ka.KoreAttnError) as e:
            attn.decode(0, -1, z, zk, zk)
        assert e.value.code == ka.KORE_ATTN_E_RANGE
        with pytest.raises(ka.KoreAttnError) as e:
            attn.decode(2, 0, z, zk, zk)
        assert e.value.code == ka.KORE_ATTN_E_INVALID
        with pytest.raises(ka.KoreAttnError) as e:
            attn.prefill(0, 60, np.zeros((5, 28 * 128), np.float32), np.zeros((5, 512), np.float32),
                         np.zeros((5, 512), np.float32))        # kore.cpp:1490
        assert e.value.code == ka.KORE_ATTN_E_RANGE
        rc = ka._lib.lib().kore_attn_decode(attn.handle, 0, 0, 28, 2, 128, z.ctypes.data,
                                            zk.ctypes.data, zk.ctypes.data, z.ctypes.data)
        assert rc == ka.KORE_ATTN_E_INVALID                     # geometry mismatch
        # a failed call leaves the handle usable
        out = attn.decode(0, 0, np.ones(28 * 128, np.float32), np.ones(512, np.float32),
                          np.full(512, 2.0, np.float32))
        np.testing.assert_array_equal(out, np.full(28 * 128, 2.0, np.float32))


def test_synth_kernel_matches_cpu_generator():
    from kore_amd import hip, synth_dev
    _say("synth kernel")
    rows, dim = 37, 3584
    buf = hip.DeviceBuffer(rows * dim)
    synth_dev(buf.ptr, rows, dim, 1234, (1 << 32) | 3, row0=11, tensor=1, per_mille=10)
    hip.synchronize()
    got = buf.download().reshape(rows, dim)
    np.testing.assert_array_equal(got, oracle.synth(rows, dim, 1234, (1 << 32) | 3, row0=11,
                                                    tensor=1, per_mille=10))


def test_device_api_matches_host_api():
    from kore_amd import hip
    nh, nkv, hd, ctx = 28, 4, 128, 512
    _say("device api")
    rng = np.random.default_rng(2)
    q = rng.standard_normal((300, nh * hd)).astype(np.float32)
    k = rng.standard_normal((300, nkv * hd)).astype(np.float32)
    v = rng.standard_normal((300, nkv * hd)).astype(np.float32)
    with _attn(1, ctx, nh, nkv, hd) as a, _attn(1, ctx, nh, nkv, hd) as b:
        ref_p = a.prefill(0, 0, q[:299], k[:299], v[:299])
        ref_d = a.decode(0, 299, q[299], k[299], v[299])
        dq, dk, dv = (hip.DeviceBuffer.from_array(x) for x in (q, k, v))
        dout = hip.DeviceBuffer(300 * nh * hd)
        b.prefill_dev(0, 0, 299, dq.ptr, dk.ptr, dv.ptr, dout.ptr)
        b.decode_dev(0, 299, dq.at(299 * nh * hd), dk.at(299 * nkv * hd), dv.at(299 * nkv * hd),
                     dout.at(299 * nh * hd))
        b.sync()
        got = dout.download().reshape(300, nh * hd)
        np.testing.assert_array_equal(got[:299], ref_p)
        np.testing.assert_array_equal(got[299], ref_d)
        np.testing.assert_array_equal(a.read_kv(0, 0, 300)[0], b.read_kv(0, 0, 300)[0])


def test_append_dev_matches_prefill_cache_rows():
    """kore_attn_append_dev writes the same cache rows as kore_attn_prefill
    (kore.cpp:1535-1538), and keeps kore's range rule (kore.cpp:1490)."""
    import kore_amd as ka
    from kore_amd import hip
    nh, nkv, hd, ctx = 12, 2, 128, 300
    _say("append_dev")
    rng = np.random.default_rng(21)
    q = rng.standard_normal((ctx, nh * hd)).astype(np.float32)
    k = rng.standard_normal((ctx, nkv * hd)).astype(np.float32)
    v = rng.standard_normal((ctx, nkv * hd)).astype(np.float32)
    with _attn(2, ctx, nh, nkv, hd) as a, _attn(2, ctx, nh, nkv, hd) as b:
        a.prefill(1, 0, q[:170], k[:170], v[:170])
        a.prefill(1, 170, q[170:], k[170:], v[170:])
        dk, dv = hip.DeviceBuffer.from_array(k), hip.DeviceBuffer.from_array(v)
        b.append_dev(1, 0, 170, dk.ptr, dv.ptr)
        b.append_dev(1, 170, ctx - 170, dk.at(170 * nkv * hd), dv.at(170 * nkv * hd))
        b.sync()
        for x, y in zip(a.read_kv(1, 0, ctx), b.read_kv(1, 0, ctx)):
            np.testing.assert_array_equal(x, y)
        with pytest.raises(ka.KoreAttnError) as e:
            b.append_dev(1, ctx - 5, 6, dk.ptr, dv.ptr)
        assert e.value.code == ka.KORE_ATTN_E_RANGE
        # a decode over appended rows equals a decode over prefilled rows
        np.testing.assert_array_equal(a.decode(1, ctx - 1, q[-1], k[-1], v[-1]),
                                      b.decode(1, ctx - 1, q[-1], k[-1], v[-1]))


def test_condense_reprefill_over_a_filled_cache():
    """kore's condense (kore.cpp:1786-1796) re-prefills a shorter sequence
    from position 0 over a cache that holds a longer one; attention reads only
    positions <= pos (kore.cpp:1437, 1549), so the stale rows past the new end
    must never be read.  The stale rows are overwritten with NaN (through the
    append path) before the decode and the next chunk: outputs must match the
    oracle's fresh run of the condensed sequence, hold no NaN, and the rows up
    to the new end must be bit-identical."""
    from kore_amd import hip
    nh, nkv, hd, ctx, nl = 28, 4, 128, 512, 2
    old_n, new_n, dec, tail = 400, 150, 20, 64
    E, kvd = nh * hd, nkv * hd
    _say(f"condense: {old_n} rows, re-prefill {new_n} from 0, NaN rows {new_n}..{old_n - 1}, decode and a chunk")
    rng = np.random.default_rng(77)

    def rows(n, d):
        return rng.standard_normal((n, d)).astype(np.float32)

    kv = oracle.KV(nl, ctx, nh, nkv, hd, 1e6)
    with _attn(nl, ctx, nh, nkv, hd, 1e6) as attn:
        for l in range(nl):   # the old conversation, in kore's 64-row chunks
            qo, ko, vo = rows(old_n, E), rows(old_n, kvd), rows(old_n, kvd)
            for z0 in range(0, old_n, 64):
                attn.prefill(l, z0, qo[z0:z0 + 64], ko[z0:z0 + 64], vo[z0:z0 + 64])
        # condense: a new, shorter sequence from position 0
        new = [(rows(new_n, E), rows(new_n, kvd), rows(new_n, kvd)) for _ in range(nl)]
        for l in range(nl):
            qn, kn, vn = new[l]
            for z0 in range(0, new_n, 64):
                out = attn.prefill(l, z0, qn[z0:z0 + 64], kn[z0:z0 + 64], vn[z0:z0 + 64])
                ref = kv.prefill(l, z0, qn[z0:z0 + 64], kn[z0:z0 + 64], vn[z0:z0 + 64], avx2=True)
                _close(out, ref, f"re-prefill layer {l} rows {z0}..")
        # poison the stale rows of the old conversation
        nan = np.full((old_n - new_n, kvd), np.nan, np.float32)
        dn = hip.DeviceBuffer.from_array(nan)
        for l in range(nl):
            attn.append_dev(l, new_n, old_n - new_n, dn.ptr, dn.ptr)
        attn.sync()
        dn.free()
        for st in range(dec):
            pos = new_n + st
            for l in range(nl):
                q, k, v = rows(1, E)[0], rows(1, kvd)[0], rows(1, kvd)[0]
                out = attn.decode(l, pos, q, k, v)
                assert np.all(np.isfinite(out)), f"stale row read at decode pos {pos} layer {l}"
                _close(out, kv.decode(l, pos, q, k, v), f"decode layer {l} pos {pos}")
        p0 = new_n + dec
        for l in range(nl):
            qc, kc_, vc_ = rows(tail, E), rows(tail, kvd), rows(tail, kvd)
            out = attn.prefill(l, p0, qc, kc_, vc_)
            assert np.all(np.isfinite(out)), f"stale row read by the chunk at {p0} layer {l}"
            _close(out, kv.prefill(l, p0, qc, kc_, vc_, avx2=True), f"chunk layer {l}")
        end = p0 + tail
        for l in range(nl):
            kg, vg = attn.read_kv(l, 0, end)
            np.testing.assert_array_equal(kg, kv.kcache()[l, :end])
            np.testing.assert_array_equal(vg, kv.vcache()[l, :end])
            ks, _ = attn.read_kv(l, end, old_n - end)   # rows past the new end stay stale
            assert np.isnan(ks).all()
    kv.close()
