"""kore itself with the attention drop-in linked in.

oracle/_ref/kore_layer_gpu is kore.cpp with INTEGRATION.md's binding applied
(oracle/make_kore_gpu.py: AttnHandle in Engine, kore_attn_create in
engine_init, kore_attn_decode in forward(), kore_attn_prefill in
forward_batch()), linked to libkore_attn.so and driven by
oracle/ref_layer_harness.cpp, built where kore's sources are (oracle/Makefile,
target ref-gpu) and carried to the GPU box with the tree.  It loads the tiny
Qwen2 GGUF file with kore's own load_model and engine_init and runs kore's own
forward() and forward_batch(); the results are held to kore's CPU results on
the same file (the committed fixtures written by the unpatched kore) within
kore's tolerance, max|d| <= 1e-4 * max|ref| (kore_kernels.cpp:742): the
attention is the only step computed differently, and it feeds the next
steps through kore's own quantisation."""
import json
import os
import subprocess

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = os.path.join(ROOT, "tests", "golden")
BIN = os.path.join(ROOT, "oracle", "_ref", "kore_layer_gpu")

needs_bin = pytest.mark.skipif(not os.path.exists(BIN),
                               reason="oracle/_ref/kore_layer_gpu is built only where kore's sources are")


def _run(args):
    print(f"[gpu-kore] kore_layer_gpu {' '.join(args[:2])} ...", flush=True)
    p = subprocess.run([BIN] + args, capture_output=True, text=True, timeout=120)
    assert p.returncode == 0, p.stderr[-2000:]
    return json.loads(p.stdout.strip().splitlines()[-1])


def _floats(hexes):
    return np.array([int(h, 16) for h in hexes], np.uint32).view(np.float32).astype(np.float64)


def _close(got, ref, what):
    err = float(np.max(np.abs(got - ref)))
    bound = 1e-4 * float(np.max(np.abs(ref)))
    assert err <= bound, f"{what}: max|d| {err:.3e} > {bound:.3e}"


@needs_bin
def test_kore_forward_with_gpu_attention():
    """kore's forward() per token with kore_attn_decode in its layer loop:
    four tokens' logits against kore's own."""
    man = json.load(open(os.path.join(GOLD, "gguf_tiny_qwen2_forward.json")))
    got = _run(["--gguf-forward", os.path.join(GOLD, man["file"]), str(man["ctx_max"])] +
               [str(t) for t in man["tokens"]])
    kore = man["kore"]
    assert got["ok"] and got["ctx"] == kore["ctx"] and got["n_vocab"] == kore["n_vocab"]
    assert len(got["logits"]) == len(kore["logits"])
    for pos, (g, r) in enumerate(zip(got["logits"], kore["logits"])):
        _close(_floats(g), _floats(r), f"token {pos}")


@needs_bin
def test_kore_forward_batch_with_gpu_attention():
    """kore's forward_batch() with kore_attn_prefill in its layer loop: two
    chunks (the second attends the first's cache rows on the GPU), the second
    chunk's residual rows and its last row's logits against kore's own."""
    man = json.load(open(os.path.join(GOLD, "gguf_tiny_qwen2_forward_batch.json")))
    got = _run(["--gguf-forward-batch", os.path.join(GOLD, man["file"]), str(man["ctx_max"]), str(man["split"])] +
               [str(t) for t in man["tokens"]])
    kore = man["kore"]
    assert got["ok"] and got["ctx"] == kore["ctx"]
    _close(_floats(got["x"]), _floats(kore["x"]), "residual rows")
    _close(_floats(got["logits"]), _floats(kore["logits"]), "logits")
