"""The oracle's restatement of kore's GGUF parse (load_model, kore.cpp:188-285),
in pure Python over the file's bytes.  TEST INFRASTRUCTURE ONLY.

parse(data) returns what oracle/_ref/kore_qmv_ref --gguf prints for the same
file: {"ok": False} when kore's load_model would return false, else the Qwen2
hyper-parameters, data_start and the tensors (first of a repeated name, sorted
by name) with type, dims, byte size, whether kore gives them data, and the
64-bit FNV-1a hash of their bytes.
"""
from __future__ import annotations

import struct

import numpy as np

# ggml types kore knows: values per block, bytes per block (kore.cpp:141-158)
BLOCKS = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 10: (256, 84),
          11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 15: (256, 292), 30: (1, 2)}
SCALAR = {0: 1, 1: 1, 7: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 10: 8, 11: 8, 12: 8}   # gguf value type: bytes
STR, ARR, U32, F32 = 8, 9, 4, 6
U32_KEYS = {"qwen2.block_count": "n_layer", "qwen2.embedding_length": "n_embd",
            "qwen2.feed_forward_length": "n_ff", "qwen2.attention.head_count": "n_head",
            "qwen2.attention.head_count_kv": "n_head_kv", "qwen2.context_length": "n_ctx"}


class _Bad(Exception):
    pass


class _R:
    """kore's Reader (kore.cpp:46-100): every read past the end is an error."""

    def __init__(self, b: bytes):
        self.b, self.pos = b, 0

    def take(self, n: int) -> bytes:
        if n > len(self.b) - self.pos:
            raise _Bad("read past the end")
        v = self.b[self.pos:self.pos + n]
        self.pos += n
        return v

    def u32(self):
        return struct.unpack("<I", self.take(4))[0]

    def u64(self):
        return struct.unpack("<Q", self.take(8))[0]

    def f32(self):
        return struct.unpack("<f", self.take(4))[0]

    def str(self) -> bytes:
        return self.take(self.u64())

    def skip_value(self, t: int):                   # kore.cpp:113-134
        if t == STR:
            self.str()
        elif t == ARR:
            et, n = self.u32(), self.u64()
            if et == STR:
                for _ in range(n):
                    self.str()
            elif et in SCALAR and n <= (len(self.b) - self.pos) // SCALAR[et]:
                self.take(n * SCALAR[et])
            else:
                raise _Bad("array")
        elif t in SCALAR:
            self.take(SCALAR[t])
        else:
            raise _Bad("metadata type")


def fnv1a64(b: bytes) -> str:
    h = 0xcbf29ce484222325
    for c in b:
        h = ((h ^ c) * 0x100000001b3) & 0xFFFFFFFFFFFFFFFF
    return f"{h:016x}"


def parse(data: bytes) -> dict:
    r = _R(data)
    try:
        if r.take(4) != b"GGUF":
            return {"ok": False}
    except _Bad:
        return {"ok": False}
    hp = {k: 0 for k in ("n_layer", "n_embd", "n_ff", "n_head", "n_head_kv", "n_ctx", "n_vocab")}
    hp["rope_base"] = hp["rms_eps"] = 0.0
    alignment = 32
    try:
        r.u32()                                     # version: kore only warns outside 2..3
        n_tensors, n_kv = r.u64(), r.u64()
        for _ in range(n_kv):
            key, t = r.str().decode(errors="replace"), r.u32()
            if key == "general.alignment" and t == U32:
                a = r.u32()
                alignment = a or alignment
            elif key in U32_KEYS and t == U32:
                hp[U32_KEYS[key]] = r.u32()
            elif key == "qwen2.rope.freq_base" and t == F32:
                hp["rope_base"] = r.f32()
            elif key == "qwen2.attention.layer_norm_rms_epsilon" and t == F32:
                hp["rms_eps"] = r.f32()
            elif key == "tokenizer.ggml.tokens" and t == ARR and len(data) - r.pos >= 12:
                hp["n_vocab"] = struct.unpack_from("<Q", data, r.pos + 4)[0] & 0xFFFFFFFF
                r.skip_value(t)
            else:
                r.skip_value(t)
        infos = []
        for _ in range(n_tensors):
            name, nd = r.str().decode(errors="replace"), r.u32()
            if nd == 0 or nd > 4:
                return {"ok": False}
            dims = [r.u64() for _ in range(nd)] + [1] * (4 - nd)
            t, off = r.u32(), r.u64()
            nel = int(np.prod(np.array(dims, dtype=object)))
            per, bb = BLOCKS.get(t, (0, 0))
            nbytes = nel // per * bb if per and nel % per == 0 else 0
            infos.append((name, t, nd, dims, nbytes, off))
    except _Bad:
        return {"ok": False}
    start = (r.pos + alignment - 1) // alignment * alignment
    if start > len(data):
        return {"ok": False}
    avail = len(data) - start
    tensors = {}
    for name, t, nd, dims, nbytes, off in infos:
        if nbytes and (off > avail or nbytes > avail - off):
            return {"ok": False}
        if name not in tensors:
            b = data[start + off:start + off + nbytes] if nbytes else b""
            tensors[name] = {"name": name, "type": t, "n_dims": nd, "dims": dims, "nbytes": nbytes,
                             "has_data": bool(nbytes), "fnv": fnv1a64(b)}
    return {"ok": True, "hp": hp, "data_start": start, "tensors": [tensors[k] for k in sorted(tensors)]}
