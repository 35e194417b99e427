"""GPU parity of kore's forward_batch() (kore.cpp:1486-1598) built from the
batched matmul: the row-wise rmsnorm bit for bit, SwiGLU and the matmul's bias
and residual epilogues against the same kernel without them, one layer
(include/kore_layer.h kore_layer_prefill_dev) against the oracle's
composition, and the whole engine (include/kore_model.h kore_model_prefill_dev)
against kore's own forward_batch() on a GGUF file
(tests/golden/gguf_tiny_qwen2_forward_batch.json).

Tolerance where the matmul, softmax or exp enter: kore's max|d| <= 1e-4 *
max|ref| (kore_kernels.cpp:742); the matmul sums in another order than kore's
single FMA chain per output.
"""
import json
import os
import sys

import numpy as np
import pytest

import oracle

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from test_gguf import oracle_engine_batch  # noqa: E402
from test_gpu_layer import _bits, _close, _synth, _x  # noqa: E402
from test_oracle_layer import load_layer_fixture  # noqa: E402

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _say(msg):
    print(f"[gpu-prefill] {msg}", flush=True)


def _up(a):
    from kore_amd import hip
    return hip.DeviceBuffer.from_array(np.ascontiguousarray(a, np.float32).reshape(-1))


@pytest.mark.parametrize("E", [3584, 4096, 4097, 5120, 7, 17])
def test_rmsnorm_rows_bitwise(E):
    """Rows of the 7B width, random and the midpoint case that needs kore's own
    loop; also the widths around the kernel's register path (up to 4096
    values) and its two-pass path for wider rows (a width that is not a
    multiple of its load batch), and short odd rows, in place and not."""
    from kore_amd import qmv
    _say(f"rmsnorm rows, E {E}")
    rng = np.random.default_rng(21)
    x = np.stack([_x(E, rng) for _ in range(6)] + [np.full(E, 1 + 2.0 ** -12, np.float32)])
    w = (1 + 0.1 * rng.standard_normal(E)).astype(np.float32)
    for eps in (np.float32(1e-6), np.float32(0.0)):
        dx, dw, do = _up(x), _up(w), _up(np.zeros_like(x))
        qmv.rmsnorm_rows_dev(dx.ptr, dw.ptr, E, x.shape[0], float(eps), do.ptr)
        got = do.download().reshape(x.shape)
        for r in range(x.shape[0]):
            assert np.array_equal(_bits(got[r]), _bits(oracle.rmsnorm(x[r], w, eps))), f"row {r} eps {eps}"
        # in place
        qmv.rmsnorm_rows_dev(dx.ptr, dw.ptr, E, x.shape[0], float(eps), dx.ptr)
        assert np.array_equal(_bits(dx.download().reshape(x.shape)), _bits(got))
        for b in (dx, dw, do):
            b.free()


def test_swiglu_rows():
    from kore_amd import qmv
    _say("swiglu 64 x 18944")
    rng = np.random.default_rng(22)
    g = (4 * rng.standard_normal(64 * 18944)).astype(np.float32)
    u = rng.standard_normal(g.size).astype(np.float32)
    dg, du = _up(g), _up(u)
    qmv.swiglu_dev(dg.ptr, du.ptr, g.size)
    got, ref = dg.download(), oracle.swiglu(g, u)
    _close(got, ref, "swiglu", tol=1e-6)
    assert np.mean(_bits(got) == _bits(ref)) > 0.999
    dg.free()
    du.free()


@pytest.mark.parametrize("B,E", [(1, 3584), (33, 3584), (64, 3584), (7, 512), (64, 4096)])
def test_rmsnorm_split_then_matmul_is_bitwise_the_plain_pair(B, E):
    """kore_qmv_rmsnorm_rows_split_dev + kore_qmv_matmul_batch_group_split_dev
    (the rmsnorm writes the matmul's fp16 split, no pre-pass) against
    kore_qmv_rmsnorm_rows_dev + kore_qmv_matmul_batch_group_ex_dev: the
    normalised rows and every output bit for bit, biases included."""
    from kore_amd import hip, qmv
    KVD = 512
    if qmv.split_bytes(E) == 0:
        pytest.skip("the split needs the fp16 matmul path")
    _say(f"rmsnorm split + matmul, B {B}, width {E}")
    rng = np.random.default_rng(41 + B)
    mats = [_synth(t, r, E, 900 + k)[0] for k, (t, r) in
            enumerate([(oracle.TYPE_Q4K, E), (oracle.TYPE_Q4K, KVD), (oracle.TYPE_Q6K, KVD)])]
    x = np.stack([_x(E, rng) for _ in range(B)])
    x[0] *= 1e-3
    nw = (1.0 + 0.1 * rng.standard_normal(E)).astype(np.float32)
    biases = [(0.5 * rng.standard_normal(m.rows)).astype(np.float32) for m in mats]
    dx, dw = _up(x), _up(nw)
    xn_a, xn_b = _up(np.zeros((B, E))), _up(np.zeros((B, E)))
    x16 = hip.DeviceBuffer(qmv.split_bytes(E) // 4)
    out_a = [_up(np.zeros((B, m.rows))) for m in mats]
    out_b = [_up(np.zeros((B, m.rows))) for m in mats]
    db = [_up(b) for b in biases]
    try:
        qmv.rmsnorm_rows_dev(dx.ptr, dw.ptr, E, B, 1e-6, xn_a.ptr)
        qmv.matmul_batch_group_ex_dev(mats, xn_a.ptr, B, [o.ptr for o in out_a], bias=[b.ptr for b in db])
        qmv.rmsnorm_rows_split_dev(dx.ptr, dw.ptr, E, B, 1e-6, xn_b.ptr, x16.ptr)
        qmv.matmul_batch_group_split_dev(mats, x16.ptr, B, [o.ptr for o in out_b], bias=[b.ptr for b in db])
        hip.synchronize()
        assert np.array_equal(_bits(xn_a.download()), _bits(xn_b.download())), "normalised rows"
        for k in range(3):
            assert np.array_equal(_bits(out_a[k].download()), _bits(out_b[k].download())), f"matrix {k}"
        with pytest.raises(qmv.QmvError):       # widths above 4096 have no split
            qmv.rmsnorm_rows_split_dev(dx.ptr, dw.ptr, 4352, 1, 1e-6, xn_b.ptr, x16.ptr)
    finally:
        for b in [dx, dw, xn_a, xn_b, x16] + out_a + out_b + db:
            b.free()
        for m in mats:
            m.close()


@pytest.mark.parametrize("B,rows,E", [(64, 18944, 3584), (1, 18944, 3584), (37, 700, 2048), (5, 512, 512)])
def test_glu_matmul_is_bitwise_matmul_then_swiglu(B, rows, E):
    """kore_qmv_matmul_batch_glu_split_dev (gate/up with the SwiGLU applied where
    the split tiles are summed) against kore_qmv_matmul_batch_group_split_dev +
    kore_qmv_swiglu_dev: every output bit for bit.  Shapes: the 7B gate/up, a
    ragged last tile, and tiles that one worker runs whole (no partials)."""
    from kore_amd import hip, qmv
    if qmv.split_bytes(E) == 0:
        pytest.skip("the split needs the fp16 matmul path")
    _say(f"glu matmul, B {B}, {rows} x {E}")
    rng = np.random.default_rng(71 + B)
    gate, up = (_synth(oracle.TYPE_Q4K, rows, E, 1300 + k)[0] for k in range(2))
    x = np.stack([_x(E, rng) for _ in range(B)])
    nw = (1.0 + 0.1 * rng.standard_normal(E)).astype(np.float32)
    dx, dw, xn = _up(x), _up(nw), _up(np.zeros((B, E)))
    x16 = hip.DeviceBuffer(qmv.split_bytes(E) // 4)
    g_a, u_a, g_b, tmp = (_up(np.zeros((B, rows))) for _ in range(4))
    try:
        qmv.rmsnorm_rows_split_dev(dx.ptr, dw.ptr, E, B, 1e-6, xn.ptr, x16.ptr)
        qmv.matmul_batch_group_split_dev([gate, up], x16.ptr, B, [g_a.ptr, u_a.ptr])
        qmv.swiglu_dev(g_a.ptr, u_a.ptr, B * rows)
        qmv.matmul_batch_glu_split_dev(gate, up, x16.ptr, B, g_b.ptr, tmp.ptr)
        hip.synchronize()
        a, b = g_a.download(), g_b.download()
        assert np.all(np.isfinite(a))
        assert np.array_equal(_bits(a), _bits(b)), f"{int(np.sum(_bits(a) != _bits(b)))} values differ"
    finally:
        for buf in [dx, dw, xn, x16, g_a, u_a, g_b, tmp]:
            buf.free()
        gate.close()
        up.close()


@pytest.mark.parametrize("B", [1, 13, 64])
def test_matmul_epilogues(B):
    """bias and accumulate: the stores of the same launch without them, then
    one float add each (kore.cpp:1530-1532, 1567-1570)."""
    from kore_amd import hip, qmv
    E, KVD = 3584, 512
    _say(f"matmul epilogues, B {B}")
    rng = np.random.default_rng(23 + B)
    mats = [_synth(t, r, E, 700 + k)[0] for k, (t, r) in
            enumerate([(oracle.TYPE_Q4K, E), (oracle.TYPE_Q4K, KVD), (oracle.TYPE_Q6K, KVD)])]
    x = np.stack([_x(E, rng) for _ in range(B)])
    biases = [(0.5 * rng.standard_normal(m.rows)).astype(np.float32) for m in mats]
    res = [rng.standard_normal((B, m.rows)).astype(np.float32) for m in mats]
    dx = _up(x)
    plain = [_up(np.zeros((B, m.rows))) for m in mats]
    withb = [_up(np.zeros((B, m.rows))) for m in mats]
    acc = [_up(r) for r in res]
    db = [_up(b) for b in biases]
    try:
        qmv.matmul_batch_group_dev(mats, dx.ptr, B, [p.ptr for p in plain])
        qmv.matmul_batch_group_ex_dev(mats, dx.ptr, B, [p.ptr for p in withb], bias=[b.ptr for b in db])
        qmv.matmul_batch_group_ex_dev(mats, dx.ptr, B, [p.ptr for p in acc], accumulate=True)
        hip.synchronize()
        for k in range(3):
            p = plain[k].download().reshape(B, -1)
            assert np.array_equal(_bits(withb[k].download().reshape(B, -1)), _bits(p + biases[k])), f"bias {k}"
            assert np.array_equal(_bits(acc[k].download().reshape(B, -1)), _bits(res[k] + p)), f"accumulate {k}"
        with pytest.raises(qmv.QmvError):       # norm_w is the matvec's, not the matmul's
            o = qmv.MvOpts()
            o.norm_w = db[0].ptr
            hs = (qmv.C.c_void_p * 1)(mats[0].handle.value)
            outs = (qmv.C.c_void_p * 1)(plain[0].ptr)
            qmv._check(qmv.lib().kore_qmv_matmul_batch_group_ex_dev(1, hs, dx.ptr, B, qmv.C.byref(o), outs, None))
    finally:
        for b in [dx] + plain + withb + acc + db:
            b.free()
        for m in mats:
            m.close()


def test_layer_prefill_against_oracle_kore_fixture_weights():
    """kore's two fixture layers (E 256), rows 0..4 then 5..7, against the oracle's forward_batch."""
    from kore_amd import KoreAttn
    from kore_amd.layer import Layer, LayerWeights
    man, z, lws = load_layer_fixture()
    E, FF, NH, NKV, HD = man["n_head"] * man["head_dim"], man["n_ff"], man["n_head"], man["n_head_kv"], man["head_dim"]
    kvd = NKV * HD
    _say("layer_2x256 weights, prefill 5 + 3 rows")
    rng = np.random.default_rng(24)
    ws = [LayerWeights.upload(lw.types, lw.mats, lw.attn_norm, lw.ffn_norm, lw.bq, lw.bk, lw.bv, E, FF, kvd)
          for lw in lws]
    kv = oracle.KV(man["n_layer"], 16, NH, NKV, HD, man["rope_base"])
    try:
        with KoreAttn(man["n_layer"], 16, NH, NKV, HD, man["rope_base"]) as attn, \
                Layer(E, FF, NH, NKV, man["rms_eps"]) as L:
            for pos0, n in ((0, 5), (5, 3)):
                x0 = np.stack([_x(E, rng) for _ in range(n)])
                dx = _up(x0)
                ref = x0
                for l in range(man["n_layer"]):
                    L.prefill_dev(ws[l], attn, l, pos0, n, dx.ptr)
                    ref = oracle.layer_forward_batch(kv, l, pos0, ref, lws[l], FF, man["rms_eps"])
                L.sync()
                _close(dx.download().reshape(n, E), ref, f"rows at {pos0}")
                dx.free()
            for l in range(man["n_layer"]):
                k, v = attn.read_kv(l, 0, 8)
                _close(k, kv.kcache()[l, :8], f"layer {l} K rows")
                _close(v, kv.vcache()[l, :8], f"layer {l} V rows")
    finally:
        for w in ws:
            w.close()


def test_layer_prefill_7b_geometry_against_oracle():
    """One 7B-shape layer (E 3584, n_ff 18944, 28/4 heads): 8 rows at 0, then 4 at 8."""
    from kore_amd import KoreAttn, hip
    from kore_amd.layer import Layer, LayerWeights
    E, FF, NH, NKV, HD = 3584, 18944, 28, 4, 128
    KVD = NKV * HD
    _say("7B geometry layer, prefill 8 + 4 rows")
    rng = np.random.default_rng(25)
    types = [oracle.TYPE_Q4K, oracle.TYPE_Q4K, oracle.TYPE_Q6K, oracle.TYPE_Q4K, oracle.TYPE_Q4K,
             oracle.TYPE_Q4K, oracle.TYPE_Q6K]
    shapes = [(E, E), (KVD, E), (KVD, E), (E, E), (FF, E), (FF, E), (E, FF)]
    host = []
    w = LayerWeights()
    for j, (t, (r, c)) in enumerate(zip(types, shapes)):
        m, b = _synth(t, r, c, 5000 + j)
        w.mats.append(m)
        host.append(b)
    norms = [(1 + 0.1 * rng.standard_normal(E)).astype(np.float32) for _ in range(2)]
    biases = [(0.2 * rng.standard_normal(n)).astype(np.float32) for n in (E, KVD, KVD)]
    for name, a in zip(("attn_norm", "ffn_norm", "bq", "bk", "bv"), norms + biases):
        w.bufs[name] = hip.DeviceBuffer.from_array(a)
    lw = oracle.LayerWeights(types, host, norms[0], norms[1], *biases)
    kv = oracle.KV(1, 16, NH, NKV, HD, 1e6)
    try:
        with KoreAttn(1, 16, NH, NKV, HD, 1e6) as attn, Layer(E, FF, NH, NKV, 1e-6) as L:
            for pos0, n in ((0, 8), (8, 4)):
                x0 = np.stack([_x(E, rng) for _ in range(n)])
                dx = _up(x0)
                L.prefill_dev(w, attn, 0, pos0, n, dx.ptr)
                L.sync()
                ref = oracle.layer_forward_batch(kv, 0, pos0, x0, lw, FF, 1e-6)
                _close(dx.download().reshape(n, E), ref, f"7B rows at {pos0}")
                dx.free()
            k, _ = attn.read_kv(0, 0, 12)
            _close(k, kv.kcache()[0, :12], "K rows")
    finally:
        w.close()


def test_layer_prefill_rejections():
    from kore_amd import KoreAttn
    from kore_amd.layer import Layer, LayerError, LayerWeights
    man, z, lws = load_layer_fixture()
    E, FF = 256, 512
    lw = lws[0]
    w = LayerWeights.upload(lw.types, lw.mats, lw.attn_norm, lw.ffn_norm, lw.bq, lw.bk, lw.bv, E, FF, 128)
    try:
        with KoreAttn(1, 8, 2, 1, 128) as attn, Layer(E, FF, 2, 1, 1e-6) as L:
            dx = _up(np.zeros((65, E)))
            for pos0, n, code in ((0, 0, 1), (0, 65, 1), (4, 5, 3), (-1, 2, 3)):   # E_INVALID, E_STEP (range)
                with pytest.raises(LayerError) as e:
                    L.prefill_dev(w, attn, 0, pos0, n, dx.ptr)
                assert e.value.code == code, (pos0, n)
            dx.free()
    finally:
        w.close()


def test_model_prefill_against_kore_forward_batch():
    """kore's forward_batch() on the tiny GGUF: tokens 0..4 at 0, 5..8 at 5 with logits."""
    from kore_amd.model import KORE_MODEL_E_RANGE, Model, ModelError
    man = json.load(open(os.path.join(GOLD, "gguf_tiny_qwen2_forward_batch.json")))
    path, kore = os.path.join(GOLD, man["file"]), man["kore"]
    toks, split = man["tokens"], man["split"]
    hexes = lambda a: np.array([int(h, 16) for h in a], np.uint32).view(np.float32)   # noqa: E731
    _say("tiny_qwen2 engine, forward_batch 5 + 4 tokens")
    with Model(path, man["ctx_max"]) as m:
        m.prefill(toks[:split], 0, want_logits=False)
        rows, logits = m.prefill(toks[split:], split)
        _close(rows, hexes(kore["x"]).reshape(rows.shape), "rows")
        _close(logits, hexes(kore["logits"]), "logits")
        k, v = m.read_kv(0, 0, len(toks))
        for pos0, n, t in ((0, 65, 0), (60, 5, 0), (-1, 1, 0), (0, 1, 12), (0, 1, -1)):
            with pytest.raises(ModelError) as e:
                m.prefill([t] * n, pos0)
            assert e.value.code == KORE_MODEL_E_RANGE, (pos0, n, t)
    _, _, _, kv = oracle_engine_batch(path, toks, split, man["ctx_max"])
    _close(k, kv.kcache()[0, :len(toks)], "layer 0 K rows")
    _close(v, kv.vcache()[0, :len(toks)], "layer 0 V rows")
