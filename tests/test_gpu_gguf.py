"""GPU side of the GGUF loader: tensors of tests/golden/gguf_tiny_qwen2.gguf
copied to the device through include/kore_gguf.h, a matvec on each quantised
matrix bit for bit against the oracle on the file's own bytes, the F32 arrays
verbatim, and one forward() layer built from the file against the oracle's
composition (kore's tolerance)."""
import os

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
PATH = os.path.join(GOLD, "gguf_tiny_qwen2.gguf")
MATS = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_quantised_tensors_and_f32_arrays():
    from kore_amd import hip, qmv
    from kore_amd.gguf import GGUF
    print("[gpu-gguf] matvecs of every quantised tensor of the tiny model", flush=True)
    rng = np.random.default_rng(2)
    with GGUF(PATH) as g:
        for name in [f"blk.0.{m}.weight" for m in MATS] + ["output.weight", "token_embd.weight"]:
            t = g.find(name)
            rows, cols = int(t.dims[1]), int(t.dims[0])
            m = g.to_qmv(name)
            x = rng.standard_normal(cols).astype(np.float32)
            got = m.mv(x, avx2=True)
            ref = oracle.qmatvec(t.type, np.frombuffer(t.bytes(), np.uint8), rows, cols, oracle.quantize_q8K(x))
            assert np.array_equal(_bits(got), _bits(ref)), name
            m.close()
        for name in ("blk.0.attn_norm.weight", "blk.0.attn_q.bias", "output_norm.weight"):
            t = g.find(name)
            d = g.to_device_f32(name)
            out = np.empty(int(t.nbytes // 4), np.float32)
            hip.check(hip.lib().hipMemcpy(out.ctypes.data, d.ptr, int(t.nbytes), hip.D2H), "D2H")
            assert np.array_equal(out, np.frombuffer(t.bytes(), np.float32)), name
            d.free()


def test_layer_from_gguf():
    from kore_amd import KoreAttn, hip
    from kore_amd.gguf import GGUF
    from kore_amd.layer import Layer, LayerWeights
    print("[gpu-gguf] one forward() layer built from the file, 3 steps", flush=True)
    with GGUF(PATH) as g:
        hp = g.hparams()
        E, FF, NH, NKV = hp.n_embd, hp.n_ff, hp.n_head, hp.n_head_kv
        HD = E // NH
        w = LayerWeights()
        host = []
        for m in MATS:
            t = g.find(f"blk.0.{m}.weight")
            w.mats.append(g.to_qmv(f"blk.0.{m}.weight"))
            host.append((t.type, np.frombuffer(t.bytes(), np.uint8).copy()))
        f32 = {}
        for key, name in (("attn_norm", "attn_norm.weight"), ("ffn_norm", "ffn_norm.weight"), ("bq", "attn_q.bias"),
                          ("bk", "attn_k.bias"), ("bv", "attn_v.bias")):
            t = g.find(f"blk.0.{name}")
            f32[key] = np.frombuffer(t.bytes(), np.float32).copy()
            w.bufs[key] = hip.DeviceBuffer.from_array(f32[key])
        lw = oracle.LayerWeights([t for t, _ in host], [b for _, b in host], f32["attn_norm"], f32["ffn_norm"],
                                 f32["bq"], f32["bk"], f32["bv"])
        kv = oracle.KV(1, 8, NH, NKV, HD, float(hp.rope_base))
        rng = np.random.default_rng(3)
        try:
            with KoreAttn(1, 8, NH, NKV, HD, float(hp.rope_base)) as attn, \
                    Layer(E, FF, NH, NKV, float(hp.rms_eps)) as L:
                dx = hip.DeviceBuffer(E)
                for st in range(3):
                    x0 = rng.standard_normal(E).astype(np.float32)
                    hip.check(hip.lib().hipMemcpy(dx.ptr, x0.ctypes.data, E * 4, hip.H2D), "H2D")
                    L.decode_dev(w, attn, 0, st, dx.ptr)
                    L.sync()
                    ref = oracle.layer_forward(kv, 0, st, x0, lw, FF, float(hp.rms_eps))
                    got = dx.download().astype(np.float64)
                    assert np.max(np.abs(got - ref)) <= 1e-4 * np.max(np.abs(ref)), f"step {st}"
                k, _ = attn.read_kv(0, 0, 3)
                assert np.array_equal(_bits(k), _bits(kv.kcache()[0, :3]))
                dx.free()
        finally:
            w.close()
