"""GPU parity of the steps fused around the matvecs and of a whole forward()
layer (include/kore_layer.h) against the oracle and against kore's own
forward() (tests/golden/layer_2x256).

Bit for bit: rmsnorm + Q8_K quantisation + q/k/v matvecs + biases (one launch),
the residual add into x (Wo), and therefore layer 0's K/V cache rows (which
depend only on those and on RoPE).  To kore's tolerance (max|d| <= 1e-4 max|ref|,
kore_kernels.cpp:742): SwiGLU (exp), attention's softmax, and what follows them.
"""
import os
import sys

import numpy as np
import pytest

import oracle

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from test_oracle_layer import load_layer_fixture  # noqa: E402

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-layer] {msg}", flush=True)


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def _close(out, ref, what, tol=1e-4):
    out, ref = np.asarray(out, np.float64), np.asarray(ref, np.float64)
    err = float(np.max(np.abs(out - ref)))
    bound = tol * float(np.max(np.abs(ref)))
    assert err <= bound, f"{what}: max|d| {err:.3e} > {bound:.3e}"


def _synth(wtype, rows, cols, seed):
    """Synthetic GGUF blocks on the device (hashed bytes, finite scales) and their bytes on the host."""
    from kore_amd import hip, qmv
    nbytes = rows * cols // 256 * oracle.BLOCK_BYTES[wtype]
    raw = hip.DeviceBuffer((nbytes + 3) // 4)
    qmv.synth_dev(wtype, rows, cols, seed, raw.ptr)
    hip.synchronize()
    w = np.zeros(nbytes, np.uint8)
    hip.check(hip.lib().hipMemcpy(w.ctypes.data, raw.ptr, nbytes, hip.D2H), "download")
    m = qmv.QMat(wtype, rows, cols, device_ptr=raw.ptr)
    raw.free()
    return m, w


def _x(n, rng):
    x = rng.standard_normal(n).astype(np.float32)
    x[rng.random(n) < 0.01] *= 20.0
    return x


@pytest.mark.parametrize("avx2", [True, False])
@pytest.mark.parametrize("case", ["random", "midpoint"])
def test_rmsnorm_quant_qkv_bias_bitwise(avx2, case):
    """7B attention width: q (3584), k, v (512) with attn_norm and biases in one launch."""
    from kore_amd import hip, qmv
    E, KVD = 3584, 512
    _say(f"rmsnorm + q/k/v + bias, E {E}, {case}, avx2 {avx2}")
    rng = np.random.default_rng(5)
    if case == "random":
        x = _x(E, rng)
        eps = np.float32(1e-6)
    else:
        # (1 + 2^-12)^2 = 1 + 2^-11 + 2^-24 lies exactly between two floats: the
        # parallel sum cannot settle the rounding and kore's own loop runs
        x = np.full(E, 1 + 2.0 ** -12, np.float32)
        x[::7] *= -1
        eps = np.float32(0.0)
    nw = (1 + 0.1 * rng.standard_normal(E)).astype(np.float32)
    biases = [(0.5 * rng.standard_normal(r)).astype(np.float32) for r in (E, KVD, KVD)]
    mats, ws = zip(*[_synth(t, r, E, 900 + k) for k, (t, r) in
                     enumerate([(oracle.TYPE_Q4K, E), (oracle.TYPE_Q4K, KVD), (oracle.TYPE_Q6K, KVD)])])
    try:
        dx, dn = hip.DeviceBuffer.from_array(x), hip.DeviceBuffer.from_array(nw)
        db = [hip.DeviceBuffer.from_array(b) for b in biases]
        outs = [hip.DeviceBuffer(r) for r in (E, KVD, KVD)]
        qmv.mv_group_ex_dev(list(mats), dx.ptr, [o.ptr for o in outs], norm_w=dn.ptr, norm_eps=float(eps),
                            bias=[b.ptr for b in db], avx2=avx2)
        hip.synchronize()
        xq = oracle.quantize_q8K(oracle.rmsnorm(x, nw, float(eps)))
        for k, (m, w, b, o) in enumerate(zip(mats, ws, biases, outs)):
            ref = oracle.qmatvec(m.type, w, m.rows, E, xq, avx2=avx2) + b
            assert np.array_equal(_bits(o.download()), _bits(ref)), f"matrix {k}"
        for b in [dx, dn] + db + outs:
            b.free()
    finally:
        for m in mats:
            m.close()


@pytest.mark.parametrize("avx2", [True, False])
def test_residual_add_bitwise(avx2):
    """Wo: x += Wo . quant(att), the add in the matvec's store."""
    from kore_amd import hip, qmv
    E = 3584
    _say(f"Wo + residual, E {E}, avx2 {avx2}")
    rng = np.random.default_rng(6)
    att, x = _x(E, rng), _x(E, rng)
    m, w = _synth(oracle.TYPE_Q4K, E, E, 77)
    try:
        da, dx = hip.DeviceBuffer.from_array(att), hip.DeviceBuffer.from_array(x)
        qmv.mv_group_ex_dev([m], da.ptr, [dx.ptr], accumulate=True, avx2=avx2)
        hip.synchronize()
        ref = x + oracle.qmatvec(oracle.TYPE_Q4K, w, E, E, oracle.quantize_q8K(att), avx2=avx2)
        assert np.array_equal(_bits(dx.download()), _bits(ref))
        da.free()
        dx.free()
    finally:
        m.close()


def test_swiglu_down_residual():
    """down: x += W_down . quant(gate / (1 + exp(-gate)) * up), 7B width 18944."""
    from kore_amd import hip, qmv
    E, FF = 3584, 18944
    _say(f"SwiGLU + down + residual, {E} x {FF}")
    rng = np.random.default_rng(7)
    gate, up, x = _x(FF, rng), _x(FF, rng), _x(E, rng)
    m, w = _synth(oracle.TYPE_Q6K, E, FF, 78)
    try:
        dg, du, dx = (hip.DeviceBuffer.from_array(a) for a in (gate, up, x))
        qmv.mv_group_ex_dev([m], dg.ptr, [dx.ptr], up=du.ptr, accumulate=True)
        hip.synchronize()
        ref = x + oracle.qmatvec(oracle.TYPE_Q6K, w, E, FF, oracle.quantize_q8K(oracle.swiglu(gate, up)))
        got = dx.download()
        _close(got, ref, "x after down")
        _say(f"outputs bitwise equal to the oracle: {int(np.sum(_bits(got) == _bits(ref)))} of {E}")
        for b in (dg, du, dx):
            b.free()
    finally:
        m.close()


@pytest.mark.parametrize("tag,avx2", [("avx2", True), ("ref", False)])
def test_layers_against_kore_forward(tag, avx2):
    """Two layers, five steps on kore's fixture: layer 0's K/V rows bit for bit,
    the residual after both layers within kore's tolerance."""
    from kore_amd import KoreAttn, hip
    from kore_amd.layer import Layer, LayerWeights
    man, z, lws = load_layer_fixture()
    E, FF = man["n_head"] * man["head_dim"], man["n_ff"]
    kvd = man["n_head_kv"] * man["head_dim"]
    _say(f"kore fixture layer_2x256, order {tag}")
    ws = [LayerWeights.upload(lw.types, lw.mats, lw.attn_norm, lw.ffn_norm, lw.bq, lw.bk, lw.bv, E, FF, kvd)
          for lw in lws]
    try:
        with KoreAttn(man["n_layer"], man["ctx"], man["n_head"], man["n_head_kv"], man["head_dim"],
                      man["rope_base"]) as attn, Layer(E, FF, man["n_head"], man["n_head_kv"], man["rms_eps"]) as L:
            dx = hip.DeviceBuffer(E)
            emb = np.ascontiguousarray(z["emb"], np.float32)   # held: hipMemcpy reads it after the call starts
            for st in range(man["steps"]):
                row = np.ascontiguousarray(emb[st])
                hip.check(hip.lib().hipMemcpy(dx.ptr, row.ctypes.data, E * 4, hip.H2D), "H2D")
                for l in range(man["n_layer"]):
                    L.decode_dev(ws[l], attn, l, st, dx.ptr, avx2=avx2)
                L.sync()
                _close(dx.download(), z[f"x_{tag}"][st], f"x after step {st}")
            k, v = attn.read_kv(0, 0, man["steps"])
            assert np.array_equal(_bits(k), _bits(z[f"kcache_{tag}"][0, :man["steps"]])), "layer 0 K rows"
            assert np.array_equal(_bits(v), _bits(z[f"vcache_{tag}"][0, :man["steps"]])), "layer 0 V rows"
            k1, v1 = attn.read_kv(1, 0, man["steps"])
            _close(k1, z[f"kcache_{tag}"][1, :man["steps"]], "layer 1 K rows")
            _close(v1, z[f"vcache_{tag}"][1, :man["steps"]], "layer 1 V rows")
            dx.free()
    finally:
        for w in ws:
            w.close()


def test_layer_7b_geometry_against_oracle():
    """One 7B-shape layer (E 3584, n_ff 18944, 28/4 heads), three steps, against
    the oracle's composition, with synthetic weights."""
    from kore_amd import KoreAttn, hip, qmv
    from kore_amd.layer import Layer, LayerWeights
    E, FF, NH, NKV, HD = 3584, 18944, 28, 4, 128
    KVD = NKV * HD
    _say("7B geometry layer, 3 steps")
    rng = np.random.default_rng(8)
    types = [oracle.TYPE_Q4K, oracle.TYPE_Q4K, oracle.TYPE_Q6K, oracle.TYPE_Q4K, oracle.TYPE_Q4K,
             oracle.TYPE_Q4K, oracle.TYPE_Q6K]
    shapes = [(E, E), (KVD, E), (KVD, E), (E, E), (FF, E), (FF, E), (E, FF)]
    host = []
    w = LayerWeights()
    for j, (t, (r, c)) in enumerate(zip(types, shapes)):
        m, b = _synth(t, r, c, 4000 + j)
        w.mats.append(m)
        host.append(b)
    norms = [(1 + 0.1 * rng.standard_normal(E)).astype(np.float32) for _ in range(2)]
    biases = [(0.2 * rng.standard_normal(n)).astype(np.float32) for n in (E, KVD, KVD)]
    for name, a in zip(("attn_norm", "ffn_norm", "bq", "bk", "bv"), norms + biases):
        w.bufs[name] = hip.DeviceBuffer.from_array(a)
    lw = oracle.LayerWeights(types, host, norms[0], norms[1], *biases)
    kv = oracle.KV(1, 8, NH, NKV, HD, 1e6)
    try:
        with KoreAttn(1, 8, NH, NKV, HD, 1e6) as attn, Layer(E, FF, NH, NKV, 1e-6) as L:
            dx = hip.DeviceBuffer(E)
            for st in range(3):
                x0 = _x(E, rng)
                hip.check(hip.lib().hipMemcpy(dx.ptr, x0.ctypes.data, E * 4, hip.H2D), "H2D")
                L.decode_dev(w, attn, 0, st, dx.ptr)
                L.sync()
                ref = oracle.layer_forward(kv, 0, st, x0, lw, FF, 1e-6)
                _close(dx.download(), ref, f"7B layer step {st}")
            k, _ = attn.read_kv(0, 0, 3)
            assert np.array_equal(_bits(k), _bits(kv.kcache()[0, :3])), "K rows"
            dx.free()
    finally:
        w.close()


def test_layer_rejections():
    from kore_amd import KoreAttn, hip
    from kore_amd.layer import Layer, LayerError, LayerWeights
    with pytest.raises(LayerError):
        Layer(300, 512, 2, 1, 1e-6)                     # n_embd not a multiple of 256
    man, z, lws = load_layer_fixture()
    E, FF = 256, 512
    lw = lws[0]
    w = LayerWeights.upload(lw.types, lw.mats, lw.attn_norm, lw.ffn_norm, lw.bq, lw.bk, lw.bv, E, FF, 128)
    try:
        with KoreAttn(1, 8, 4, 1, 64) as attn, Layer(E, FF, 2, 1, 1e-6) as L:    # head_dim 64 != 128
            dx = hip.DeviceBuffer(E)
            with pytest.raises(LayerError) as e:
                L.decode_dev(w, attn, 0, 0, dx.ptr)
            assert e.value.code == 1
            dx.free()
    finally:
        w.close()
