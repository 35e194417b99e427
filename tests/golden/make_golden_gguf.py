#!/usr/bin/env python3
"""Write small GGUF files and kore's own parse of each: tests/golden/gguf_*.gguf
and gguf_*.json; and kore's whole engine on the tiny model's file
(gguf_tiny_qwen2_forward.json: logits of four decode tokens;
gguf_tiny_qwen2_forward_batch.json: forward_batch() of two chunks).

The files are written here from the GGUF layout (magic, version, tensor and
metadata counts, typed key/value pairs, the tensor table, data aligned to
general.alignment); kore's load_model (kore.cpp:188-285), run through
oracle/_ref/kore_qmv_ref --gguf, records what it makes of each: the Qwen2
hyper-parameters, data_start, and per tensor its type, dims, byte size and a
hash of the bytes it points to - or that it rejects the file.  Cases: a tiny
Qwen2 model with metadata of every kind kore skips (strings, string and number
arrays, bools, 64-bit values), an F16 tensor, a tensor of a type kore does not
know, a repeated tensor name; a version-2 file with 64-byte alignment; and five
malformed files (bad magic, a tensor past the end, five dimensions, an array of
an unknown element type, a header cut short).
"""
from __future__ import annotations

import json
import os
import struct
import subprocess
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
          I64: "<q", F64: "<d"}
BLOCK = {0: (1, 4), 1: (1, 2), 12: (256, 144), 14: (256, 210)}   # type: (values per block, bytes per block)


def s_(v: str) -> bytes:
    b = v.encode()
    return struct.pack("<Q", len(b)) + b


def value(t: int, v) -> bytes:
    if t == STR:
        return s_(v)
    if t == ARR:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        return out + b"".join(s_(x) if et == STR else struct.pack(SCALAR[et], x) for x in items)
    return struct.pack(SCALAR[t], v)


def gguf(meta, tensors, alignment=32, version=3, magic=b"GGUF", n_dims_override=None, cut=None):
    """meta: [(key, type, value)]; tensors: [(name, dims, type, bytes)]."""
    head = magic + struct.pack("<IQQ", version, len(tensors), len(meta))
    head += b"".join(s_(k) + struct.pack("<I", t) + value(t, v) for k, t, v in meta)
    offs, off = [], 0
    for name, dims, t, data in tensors:
        offs.append(off)
        off += (len(data) + alignment - 1) // alignment * alignment
    for (name, dims, t, data), o in zip(tensors, offs):
        nd = n_dims_override.get(name, len(dims)) if n_dims_override else len(dims)
        head += s_(name) + struct.pack("<I", nd) + b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", t, o)
    start = (len(head) + alignment - 1) // alignment * alignment
    body = bytearray(head + bytes(start - len(head)))
    for (name, dims, t, data), o in zip(tensors, offs):
        body += bytes(start + o - len(body))
        body += data
    body = bytes(body)
    return body[:cut] if cut is not None else body


def tensor_bytes(t: int, dims, rng) -> bytes:
    n = int(np.prod(dims))
    per, bb = BLOCK.get(t, (1, 1))
    raw = rng.integers(0, 256, size=n // per * bb, dtype=np.uint8)
    if t == 12:
        raw.reshape(-1, 144)[:, 0:4] = np.frombuffer(np.array([3e-4, 1e-4], np.float16).tobytes(), np.uint8)
    if t == 14:
        raw.reshape(-1, 210)[:, 208:210] = np.frombuffer(np.float16(5e-5).tobytes(), np.uint8)
    if t == 0:
        raw = rng.standard_normal(n).astype(np.float32).view(np.uint8)
    return raw.tobytes()


def cases():
    rng = np.random.default_rng(41)
    E, FF, V = 256, 256, 12
    meta = [("general.architecture", STR, "qwen2"), ("general.name", STR, "tiny"),
            ("qwen2.block_count", U32, 1), ("qwen2.context_length", U32, 4096), ("qwen2.embedding_length", U32, E),
            ("qwen2.feed_forward_length", U32, FF), ("qwen2.attention.head_count", U32, 2),
            ("qwen2.attention.head_count_kv", U32, 1), ("qwen2.rope.freq_base", F32, 1000000.0),
            ("qwen2.attention.layer_norm_rms_epsilon", F32, 1e-6), ("general.file_type", U32, 15),
            ("tokenizer.ggml.model", STR, "gpt2"), ("tokenizer.ggml.tokens", ARR, (STR, [f"t{i}" for i in range(V)])),
            ("tokenizer.ggml.token_type", ARR, (I32, [1] * V)), ("tokenizer.ggml.merges", ARR, (STR, ["a b", "c d"])),
            ("tokenizer.ggml.add_bos_token", BOOL, False), ("tokenizer.ggml.eos_token_id", U32, 3),
            ("general.quantization_version", U32, 2), ("test.u64", U64, 1 << 40), ("test.f64", F64, 0.5),
            ("test.i16", I16, -3), ("test.u8arr", ARR, (U8, [1, 2, 3]))]
    shapes = [("token_embd.weight", [E, V], 12), ("blk.0.attn_q.weight", [E, E], 12),
              ("blk.0.attn_k.weight", [E, 128], 12), ("blk.0.attn_v.weight", [E, 128], 14),
              ("blk.0.attn_q.bias", [E], 0), ("blk.0.attn_k.bias", [128], 0), ("blk.0.attn_v.bias", [128], 0),
              ("blk.0.attn_output.weight", [E, E], 12), ("blk.0.ffn_gate.weight", [E, FF], 12),
              ("blk.0.ffn_up.weight", [E, FF], 12), ("blk.0.ffn_down.weight", [FF, E], 14),
              ("blk.0.attn_norm.weight", [E], 0), ("blk.0.ffn_norm.weight", [E], 0), ("output_norm.weight", [E], 0),
              ("output.weight", [E, V], 14), ("test.f16", [64, 2], 1), ("test.unknown_type", [32], 99),
              ("blk.0.attn_q.weight", [E, 2], 0)]        # a repeated name: kore keeps the first
    tensors = [(n, d, t, tensor_bytes(t, d, rng)) for n, d, t in shapes]
    tensors[16] = (tensors[16][0], tensors[16][1], 99, bytes(40))
    small = tensors[4:7]
    yield "tiny_qwen2", gguf(meta, tensors)
    yield "align64_v2", gguf([("general.alignment", U32, 64)] + meta[2:10], small, alignment=64, version=2)
    yield "bad_magic", gguf(meta[:3], small, magic=b"GGUX")
    yield "truncated", gguf(meta[:3], small)[:-100]
    yield "five_dims", gguf(meta[:3], [("x", [1, 1, 1, 1], 0, bytes(4))], n_dims_override={"x": 5})
    yield "bad_array", gguf([("bad", ARR, (77, []))], small)          # element type 77: kore's "array invalido"
    yield "short_header", gguf(meta, small, cut=60)


def main():
    if not os.path.exists(oracle.REF_QMV_BIN):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "ref"], check=True)
    for name, data in cases():
        path = os.path.join(HERE, f"gguf_{name}.gguf")
        with open(path, "wb") as f:
            f.write(data)
        r = subprocess.run([oracle.REF_QMV_BIN, "--gguf", path], capture_output=True, text=True, check=True)
        kore = json.loads(r.stdout)
        with open(os.path.join(HERE, f"gguf_{name}.json"), "w") as f:
            json.dump({"file": f"gguf_{name}.gguf", "bytes": len(data), "kore": kore,
                       "kore_stderr": r.stderr.strip()}, f, indent=1)
        print(name, len(data), "ok" if kore["ok"] else "rejected", r.stderr.strip()[:60])
    # kore's whole engine on the tiny model: engine_init (ctx_max 64) and
    # forward() with logits for four tokens at positions 0..3
    if not os.path.exists(oracle.REF_LAYER_BIN):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "ref"], check=True)
    tokens = [3, 7, 0, 11]
    r = subprocess.run([oracle.REF_LAYER_BIN, "--gguf-forward", os.path.join(HERE, "gguf_tiny_qwen2.gguf"), "64"] +
                       [str(t) for t in tokens], capture_output=True, text=True, check=True)
    fwd = json.loads(r.stdout)
    with open(os.path.join(HERE, "gguf_tiny_qwen2_forward.json"), "w") as f:
        json.dump({"file": "gguf_tiny_qwen2.gguf", "ctx_max": 64, "tokens": tokens,
                   "source": "kore.cpp load_model + engine_init + forward(logits) via oracle/_ref/kore_layer_ref",
                   "kore": fwd}, f, indent=1)
    print("forward:", fwd["ok"], fwd["ctx"], fwd["n_vocab"])
    # kore's forward_batch() on the same model: tokens 0..4 at position 0, then
    # 5..8 at position 5 with logits (the residual rows of the second chunk)
    tokens, split = [3, 7, 0, 11, 5, 2, 9, 10, 1], 5
    r = subprocess.run([oracle.REF_LAYER_BIN, "--gguf-forward-batch", os.path.join(HERE, "gguf_tiny_qwen2.gguf"),
                        "64", str(split)] + [str(t) for t in tokens], capture_output=True, text=True, check=True)
    fwd = json.loads(r.stdout)
    with open(os.path.join(HERE, "gguf_tiny_qwen2_forward_batch.json"), "w") as f:
        json.dump({"file": "gguf_tiny_qwen2.gguf", "ctx_max": 64, "tokens": tokens, "split": split,
                   "source": "kore.cpp load_model + engine_init + forward_batch x2 via oracle/_ref/kore_layer_ref",
                   "kore": fwd}, f, indent=1)
    print("forward_batch:", fwd["ok"], fwd["ctx"], fwd["bsz"], len(fwd["x"]))


if __name__ == "__main__":
    main()
