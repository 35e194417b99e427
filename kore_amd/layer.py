"""ctypes binding of include/kore_layer.h (kore_amd/libkore_layer.so): one layer
of kore's forward() (kore.cpp:1415-1472) on the GPU over a device-resident
residual stream, chaining libkore_qmv's fused matvec launches and
libkore_attn's decode on one stream.

    L = Layer(n_embd, n_ff, n_head, n_head_kv, rms_eps)
    w = LayerWeights.upload(types, mats, attn_norm, ffn_norm, bq, bk, bv, n_embd, n_ff, kv_dim)
    L.decode_dev(w, attn, layer, pos, x_ptr)       # x (device) updated in place

No CPU fallback: without the built library or a GPU every call raises.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import _lib as _attn_lib
from . import hip, qmv

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkore_layer.so")

KORE_LAYER_OK = 0
KORE_LAYER_E_INVALID = 1
KORE_LAYER_E_HIP = 2
KORE_LAYER_E_STEP = 3

_vp, _i, _f = C.c_void_p, C.c_int, C.c_float


class _Weights(C.Structure):
    _fields_ = [(n, _vp) for n in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down",
                                   "attn_norm", "ffn_norm", "bq", "bk", "bv")]


SYMBOLS = [
    ("kore_layer_create", _i, [C.POINTER(_vp), _i, _i, _i, _i, _f]),
    ("kore_layer_destroy", None, [_vp]),
    ("kore_layer_decode_dev", _i, [_vp, C.POINTER(_Weights), _vp, _i, _i, _vp, _i, _vp]),
    ("kore_layer_prefill_dev", _i, [_vp, C.POINTER(_Weights), _vp, _i, _i, _i, _vp, _vp]),
    ("kore_layer_sync", _i, [_vp]),
    ("kore_layer_last_error", C.c_char_p, [_vp]),
]

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise _attn_lib.LibraryMissing(f"{LIB_PATH} is not built; run `make -C kore_amd/csrc`")
        _attn_lib.lib()
        qmv.lib()
        L = C.CDLL(LIB_PATH)
        for name, res, args in SYMBOLS:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


class LayerError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"kore_layer error {code}: {message}")
        self.code = code


class LayerWeights:
    """Device copies of one layer's weights: libkore_qmv tensors for the seven
    matrices, device arrays for the norms and biases (kore's Layer,
    kore.cpp:1246-1250)."""

    def __init__(self):
        self.mats, self.bufs = [], {}

    @classmethod
    def upload(cls, types, mats, attn_norm, ffn_norm, bq, bk, bv, n_embd: int, n_ff: int, kv_dim: int):
        shapes = [(n_embd, n_embd), (kv_dim, n_embd), (kv_dim, n_embd), (n_embd, n_embd), (n_ff, n_embd),
                  (n_ff, n_embd), (n_embd, n_ff)]
        w = cls()
        for t, m, (r, c) in zip(types, mats, shapes):
            w.mats.append(qmv.QMat(t, r, c, np.ascontiguousarray(m, np.uint8)))
        for name, a in (("attn_norm", attn_norm), ("ffn_norm", ffn_norm), ("bq", bq), ("bk", bk), ("bv", bv)):
            w.bufs[name] = None if a is None else hip.DeviceBuffer.from_array(np.asarray(a, np.float32))
        return w

    def struct(self) -> _Weights:
        s = _Weights()
        for name, m in zip(("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"), self.mats):
            setattr(s, name, m.handle.value)
        for name, b in self.bufs.items():
            setattr(s, name, b.ptr if b is not None else None)
        return s

    def close(self):
        for m in self.mats:
            m.close()
        for b in self.bufs.values():
            if b is not None:
                b.free()
        self.mats, self.bufs = [], {}


class Layer:
    """kore_layer_t: geometry and device scratch of a forward() layer step."""

    def __init__(self, n_embd: int, n_ff: int, n_head: int, n_head_kv: int, rms_eps: float):
        h = _vp()
        rc = lib().kore_layer_create(C.byref(h), n_embd, n_ff, n_head, n_head_kv, rms_eps)
        if rc != KORE_LAYER_OK:
            raise LayerError(rc, lib().kore_layer_last_error(None).decode())
        self._h = h

    def _check(self, rc: int):
        if rc != KORE_LAYER_OK:
            raise LayerError(rc, lib().kore_layer_last_error(self._h).decode())

    def decode_dev(self, w: LayerWeights, attn, layer: int, pos: int, x_ptr: int, avx2: bool = True,
                   stream=None) -> None:
        """kore's forward() body for `layer` at `pos`: x (device) updated in place."""
        s = w.struct()
        self._check(lib().kore_layer_decode_dev(self._h, C.byref(s), attn.handle, layer, pos, x_ptr, int(avx2),
                                                stream))

    def prefill_dev(self, w: LayerWeights, attn, layer: int, pos0: int, n_tok: int, x_ptr: int,
                    stream=None) -> None:
        """kore's forward_batch() body for `layer` over n_tok rows at pos0..:
        x (device, [n_tok][n_embd]) updated in place."""
        s = w.struct()
        self._check(lib().kore_layer_prefill_dev(self._h, C.byref(s), attn.handle, layer, pos0, n_tok, x_ptr, stream))

    def sync(self):
        self._check(lib().kore_layer_sync(self._h))

    def close(self):
        if self._h:
            lib().kore_layer_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
