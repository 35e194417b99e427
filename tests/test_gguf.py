"""kore's GGUF parse (load_model, kore.cpp:188-285): the oracle's restatement
and the library's parser (include/kore_gguf.h, host code: no GPU needed)
against kore's own parse of the fixture files tests/golden/gguf_*, written by
tests/golden/make_golden_gguf.py and parsed there by kore.cpp itself."""
import json
import os

import numpy as np
import pytest

import oracle.gguf as ogguf

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASES = sorted(f[5:-5] for f in os.listdir(GOLD)
               if f.startswith("gguf_") and f.endswith(".json") and "_forward" not in f)


def _case(name):
    man = json.load(open(os.path.join(GOLD, f"gguf_{name}.json")))
    data = open(os.path.join(GOLD, man["file"]), "rb").read()
    return man, data


def _hp_equal(hp, kore_hp):
    for k in ("n_layer", "n_embd", "n_ff", "n_head", "n_head_kv", "n_ctx", "n_vocab"):
        assert hp[k] == kore_hp[k], k
    for k in ("rope_base", "rms_eps"):                 # kore prints %.9g of the float
        assert np.float32(hp[k]) == np.float32(kore_hp[k]), k


def test_fixture_set():
    assert {"tiny_qwen2", "align64_v2", "bad_magic", "truncated", "five_dims", "bad_array",
            "short_header"} <= set(CASES)
    man, _ = _case("tiny_qwen2")
    names = [t["name"] for t in man["kore"]["tensors"]]
    assert "test.unknown_type" in names and names.count("blk.0.attn_q.weight") == 1


@pytest.mark.parametrize("name", CASES)
def test_oracle_parse_matches_kore(name):
    man, data = _case(name)
    got, kore = ogguf.parse(data), man["kore"]
    assert got["ok"] == kore["ok"]
    if kore["ok"]:
        _hp_equal(got["hp"], kore["hp"])
        assert got["data_start"] == kore["data_start"]
        assert got["tensors"] == kore["tensors"]


@pytest.mark.parametrize("name", CASES)
def test_library_parse_matches_kore(name):
    from kore_amd.gguf import GGUF, KORE_GGUF_E_FORMAT, GGUFError
    man, _ = _case(name)
    kore, path = man["kore"], os.path.join(GOLD, man["file"])
    if not kore["ok"]:
        with pytest.raises(GGUFError) as e:
            GGUF(path)
        assert e.value.code == KORE_GGUF_E_FORMAT
        return
    with GGUF(path) as g:
        hp = g.hparams()
        _hp_equal({k: getattr(hp, k) for k in kore["hp"]}, kore["hp"])
        assert hp.data_start == kore["data_start"] and hp.file_size == man["bytes"]
        got = sorted(({"name": t.name.decode(), "type": t.type, "n_dims": t.n_dims, "dims": list(t.dims),
                       "nbytes": t.nbytes, "has_data": bool(t.data), "fnv": ogguf.fnv1a64(t.bytes())}
                      for t in g.tensors()), key=lambda d: d["name"])
        assert got == kore["tensors"]
        # file order of first appearances, and lookups by name
        assert g.tensors()[0].name.decode() == "token_embd.weight" or name != "tiny_qwen2"
        for t in kore["tensors"]:
            assert g.find(t["name"]).nbytes == t["nbytes"]


def test_library_errors():
    from kore_amd.gguf import GGUF, KORE_GGUF_E_IO, KORE_GGUF_E_NOT_FOUND, KORE_GGUF_E_TYPE, GGUFError
    with pytest.raises(GGUFError) as e:
        GGUF(os.path.join(GOLD, "no_such_file.gguf"))
    assert e.value.code == KORE_GGUF_E_IO
    with GGUF(os.path.join(GOLD, "gguf_tiny_qwen2.gguf")) as g:
        with pytest.raises(GGUFError) as e:
            g.find("blk.9.attn_q.weight")
        assert e.value.code == KORE_GGUF_E_NOT_FOUND
        with pytest.raises(GGUFError) as e:
            g.to_qmv("blk.0.attn_norm.weight")             # F32, not Q4_K / Q6_K
        assert e.value.code == KORE_GGUF_E_TYPE
        with pytest.raises(GGUFError) as e:
            g.to_device_f32("blk.0.attn_q.weight")         # Q4_K, not F32
        assert e.value.code == KORE_GGUF_E_TYPE


def test_oracle_rejects_what_breaks_the_rules():
    # independently of kore's fixtures: each rule on a minimal file
    good = open(os.path.join(GOLD, "gguf_align64_v2.gguf"), "rb").read()
    assert ogguf.parse(good)["ok"]
    assert not ogguf.parse(b"GGUF")["ok"]                   # header cut short
    assert not ogguf.parse(b"XGUF" + good[4:])["ok"]        # magic
    assert not ogguf.parse(good[:-1])["ok"]                 # last tensor leaves the file by one byte


def _oracle_engine(path, ctx_max):
    """engine_init's tensors (kore.cpp:1274-1334) from the oracle's parse:
    (hp, ctx, layers, f32, embedding row, output head (type, rows, bytes), kv)."""
    import oracle
    data = open(path, "rb").read()
    p = ogguf.parse(data)
    hp, start = p["hp"], p["data_start"]
    # tensor bytes by name, from the parse's offsets (first of a repeated name)
    r = ogguf._R(data)
    r.take(4), r.u32()
    n_t, n_kv = r.u64(), r.u64()
    for _ in range(n_kv):
        r.str()
        r.skip_value(r.u32())
    tens = {}
    for _ in range(n_t):
        name, nd = r.str().decode(), r.u32()
        dims = [r.u64() for _ in range(nd)] + [1] * (4 - nd)
        t, off = r.u32(), r.u64()
        if name not in tens:
            nb = next(x["nbytes"] for x in p["tensors"] if x["name"] == name)
            tens[name] = (t, dims, np.frombuffer(data[start + off:start + off + nb], np.uint8))
    E, FF, NH, NKV = hp["n_embd"], hp["n_ff"], hp["n_head"], hp["n_head_kv"]
    ctx = min(hp["n_ctx"], ctx_max) if hp["n_ctx"] else ctx_max
    f32 = lambda n: tens[n][2].view(np.float32)                     # noqa: E731
    layers = []
    for l in range(hp["n_layer"]):
        b = f"blk.{l}."
        names = ["attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"]
        layers.append(oracle.LayerWeights([tens[b + n + ".weight"][0] for n in names],
                                          [tens[b + n + ".weight"][2] for n in names],
                                          f32(b + "attn_norm.weight"), f32(b + "ffn_norm.weight"),
                                          f32(b + "attn_q.bias"), f32(b + "attn_k.bias"), f32(b + "attn_v.bias")))
    kv = oracle.KV(hp["n_layer"], ctx, NH, NKV, E // NH, hp["rope_base"])
    et, edims, eb = tens["token_embd.weight"]
    row_bytes = len(eb) // edims[1]

    def emb(tok):
        r = eb[tok * row_bytes:(tok + 1) * row_bytes]
        return oracle.dequant_row(et, r, E) if et in (12, 14) else r.view(np.float32).copy()

    ot, odims, ob = tens["output.weight"]
    return hp, ctx, layers, f32, emb, (ot, odims[1], ob), kv


def _oracle_logits(hp, f32, head, x, avx2=True):
    """forward()'s logits (kore.cpp:1474-1478)."""
    import oracle
    ot, rows, ob = head
    xq = oracle.quantize_q8K(oracle.rmsnorm(x, f32("output_norm.weight"), hp["rms_eps"]))
    return oracle.qmatvec(ot, ob, rows, hp["n_embd"], xq, avx2=avx2)


def oracle_engine_logits(path, tokens, ctx_max=64, avx2=True):
    """The oracle's kore engine over a GGUF file: engine_init, then per token
    get_row (kore.cpp:384-407), every forward() layer and the logits; avx2 is
    kore's e.avx2 (the matvecs' summation order)."""
    import oracle
    hp, ctx, layers, f32, emb, head, kv = _oracle_engine(path, ctx_max)
    out = []
    for pos, tok in enumerate(tokens):
        x = emb(tok)
        for l, lw in enumerate(layers):
            x = oracle.layer_forward(kv, l, pos, x, lw, hp["n_ff"], hp["rms_eps"], avx2=avx2)
        out.append(_oracle_logits(hp, f32, head, x, avx2))
    return ctx, np.stack(out), kv


def oracle_engine_batch(path, tokens, split, ctx_max=64):
    """The oracle's forward_batch() (kore.cpp:1486-1600) over the tokens in two
    chunks, [0, split) at position 0 and the rest at `split`: the second
    chunk's residual rows and the logits of its last row."""
    import oracle
    hp, ctx, layers, f32, emb, head, kv = _oracle_engine(path, ctx_max)
    for pos0, chunk in ((0, tokens[:split]), (split, tokens[split:])):
        x = np.stack([emb(t) for t in chunk])
        for l, lw in enumerate(layers):
            x = oracle.layer_forward_batch(kv, l, pos0, x, lw, hp["n_ff"], hp["rms_eps"], avx2=True)
    return ctx, x, _oracle_logits(hp, f32, head, x[-1]), kv


def test_oracle_engine_matches_kore_logits():
    man = json.load(open(os.path.join(GOLD, "gguf_tiny_qwen2_forward.json")))
    kore = man["kore"]
    ctx, logits, _ = oracle_engine_logits(os.path.join(GOLD, man["file"]), man["tokens"], man["ctx_max"])
    assert kore["ok"] and kore["avx2"] == 1 and ctx == kore["ctx"]
    want = np.array([[int(h, 16) for h in row] for row in kore["logits"]], np.uint32)
    assert np.array_equal(logits.astype(np.float32).view(np.uint32), want)


def test_oracle_forward_batch_matches_kore():
    man = json.load(open(os.path.join(GOLD, "gguf_tiny_qwen2_forward_batch.json")))
    kore = man["kore"]
    ctx, x, logits, _ = oracle_engine_batch(os.path.join(GOLD, man["file"]), man["tokens"], man["split"],
                                            man["ctx_max"])
    assert kore["ok"] and kore["avx2"] == 1 and ctx == kore["ctx"]
    hexes = lambda a: np.array([int(h, 16) for h in a], np.uint32)   # noqa: E731
    assert np.array_equal(x.astype(np.float32).reshape(-1).view(np.uint32), hexes(kore["x"]))
    assert np.array_equal(logits.astype(np.float32).view(np.uint32), hexes(kore["logits"]))
    # the batch and the token-at-a-time paths differ (matmul in float vs Q8_K matvec)
    _, dec, _ = oracle_engine_logits(os.path.join(GOLD, man["file"]), man["tokens"], man["ctx_max"])
    assert not np.array_equal(dec[-1].astype(np.float32), logits.astype(np.float32))



@pytest.mark.parametrize("change,fragment", [
    ({"output.weight": [128, 12]}, "output.weight has the wrong shape"),
    ({"output.weight": [256, 12, 2]}, "output.weight has the wrong shape"),
    ({"blk.0.attn_norm.weight": [128]}, "blk.0.attn_norm.weight does not hold 256 floats"),
    ({"output_norm.weight": [255]}, "output_norm.weight does not hold 256 floats"),
    ({"blk.0.attn_k.bias": [256]}, "blk.0.attn_k.bias does not hold 128 floats"),
    ({"blk.0.attn_q.bias": [128]}, "blk.0.attn_q.bias does not hold 256 floats"),
    ({"blk.0.ffn_down.weight": [256, 512]}, "blk.0.ffn_down.weight has the wrong shape"),
])
def test_model_refuses_malformed_shapes_before_the_device(tmp_path, change, fragment):
    """kore_model_load checks the shape of every tensor the forward pass reads
    and refuses a parseable file with a short norm or bias, or a head of the
    wrong width, with KORE_MODEL_E_LOAD before anything is copied to a GPU
    (runs on a host without one)."""
    import sys
    sys.path.insert(0, os.path.join(GOLD))
    import make_golden_gguf as mg
    from kore_amd.model import KORE_MODEL_E_LOAD, Model, ModelError
    rng = np.random.default_rng(3)
    E, FF, V = 256, 256, 12
    meta = [("general.architecture", mg.STR, "qwen2"), ("qwen2.block_count", mg.U32, 1),
            ("qwen2.context_length", mg.U32, 64), ("qwen2.embedding_length", mg.U32, E),
            ("qwen2.feed_forward_length", mg.U32, FF), ("qwen2.attention.head_count", mg.U32, 2),
            ("qwen2.attention.head_count_kv", mg.U32, 1), ("qwen2.rope.freq_base", mg.F32, 1e6),
            ("qwen2.attention.layer_norm_rms_epsilon", mg.F32, 1e-6)]
    shapes = {"token_embd.weight": ([E, V], 12), "blk.0.attn_q.weight": ([E, E], 12),
              "blk.0.attn_k.weight": ([E, 128], 12), "blk.0.attn_v.weight": ([E, 128], 14),
              "blk.0.attn_q.bias": ([E], 0), "blk.0.attn_k.bias": ([128], 0), "blk.0.attn_v.bias": ([128], 0),
              "blk.0.attn_output.weight": ([E, E], 12), "blk.0.ffn_gate.weight": ([E, FF], 12),
              "blk.0.ffn_up.weight": ([E, FF], 12), "blk.0.ffn_down.weight": ([FF, E], 14),
              "blk.0.attn_norm.weight": ([E], 0), "blk.0.ffn_norm.weight": ([E], 0),
              "output_norm.weight": ([E], 0), "output.weight": ([E, V], 14)}
    for name, dims in change.items():
        shapes[name] = (dims, shapes[name][1])
    tensors = [(n, d, t, mg.tensor_bytes(t, d, rng)) for n, (d, t) in shapes.items()]
    path = tmp_path / "bad.gguf"
    path.write_bytes(mg.gguf(meta, tensors))
    with pytest.raises(ModelError) as e:
        Model(str(path), 64)
    assert e.value.code == KORE_MODEL_E_LOAD and fragment in str(e.value)
