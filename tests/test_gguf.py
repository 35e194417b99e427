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
CASES = sorted(f[5:-5] for f in os.listdir(GOLD) if f.startswith("gguf_") and f.endswith(".json"))


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
