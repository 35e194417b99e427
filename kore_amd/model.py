"""ctypes binding of include/kore_model.h (in kore_amd/libkore_layer.so): kore's
engine over a GGUF file with every tensor in HBM, and forward() for one token
on the GPU (embedding row, every layer, logits).

    with Model(path, ctx_max=4096) as m:
        logits = m.decode(token, pos)            # kore's e.logits after forward(token, pos, true)
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from .gguf import Hparams
from .layer import lib as _layer_lib

KORE_MODEL_OK, KORE_MODEL_E_LOAD, KORE_MODEL_E_RANGE, KORE_MODEL_E_DEVICE = range(4)


class Info(C.Structure):
    _fields_ = [("hp", Hparams), ("ctx", C.c_int), ("n_vocab", C.c_int), ("head_dim", C.c_int), ("kv_dim", C.c_int),
                ("weight_bytes", C.c_size_t), ("avx2", C.c_int)]


_done = False


def lib() -> C.CDLL:
    global _done
    L = _layer_lib()
    if not _done:
        vp = C.c_void_p
        for name, res, args in (("kore_model_load", C.c_int, [C.c_char_p, C.c_int, C.POINTER(vp)]),
                                ("kore_model_load_ex", C.c_int, [C.c_char_p, C.c_int, C.c_int, C.POINTER(vp)]),
                                ("kore_model_destroy", None, [vp]),
                                ("kore_model_get_info", C.c_int, [vp, C.POINTER(Info)]),
                                ("kore_model_decode_dev", C.c_int, [vp, C.c_int, C.c_int, C.c_int, vp]),
                                ("kore_model_logits_dev", vp, [vp]),
                                ("kore_model_prefill_dev", C.c_int, [vp, vp, C.c_int, C.c_int, C.c_int, vp]),
                                ("kore_model_rows_dev", vp, [vp]),
                                ("kore_model_sync", C.c_int, [vp]),
                                ("kore_model_decode", C.c_int, [vp, C.c_int, C.c_int, vp]),
                                ("kore_model_attn", vp, [vp]),
                                ("kore_model_last_error", C.c_char_p, [vp])):
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _done = True
    return L


class ModelError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"kore_model error {code}: {message}")
        self.code = code


class Model:
    """avx2: the matvecs' summation order, kore's e.avx2 (kore.cpp:1293): None
    picks it as kore's engine_init does on this host, True / False force
    kore's AVX2 / scalar order."""

    def __init__(self, path: str, ctx_max: int = 4096, avx2: bool | None = None):
        h = C.c_void_p()
        rc = lib().kore_model_load_ex(path.encode(), ctx_max, -1 if avx2 is None else int(bool(avx2)), C.byref(h))
        if rc != KORE_MODEL_OK:
            raise ModelError(rc, lib().kore_model_last_error(None).decode())
        self._h = h
        self.info = Info()
        self._check(lib().kore_model_get_info(self._h, C.byref(self.info)))

    def _check(self, rc):
        if rc != KORE_MODEL_OK:
            raise ModelError(rc, lib().kore_model_last_error(self._h).decode())

    def decode(self, token: int, pos: int, want_logits: bool = True):
        """kore's forward(token, pos, want_logits): the logits (host copy) or None."""
        out = np.zeros(self.info.n_vocab, np.float32) if want_logits else None
        self._check(lib().kore_model_decode(self._h, token, pos, out.ctypes.data if want_logits else None))
        return out

    def prefill(self, tokens, pos0: int, want_logits: bool = True):
        """kore's forward_batch(tokens, pos0, want_logits): (rows [n][n_embd],
        logits of the last row or None), host copies."""
        from . import hip
        t = np.ascontiguousarray(tokens, np.int32).reshape(-1)
        self._check(lib().kore_model_prefill_dev(self._h, t.ctypes.data, t.size, pos0, int(want_logits), None))
        self._check(lib().kore_model_sync(self._h))
        rows = np.zeros((t.size, self.info.hp.n_embd), np.float32)
        hip.check(hip.lib().hipMemcpy(rows.ctypes.data, lib().kore_model_rows_dev(self._h), rows.nbytes, hip.D2H),
                  "rows")
        logits = None
        if want_logits:
            logits = np.zeros(self.info.n_vocab, np.float32)
            hip.check(hip.lib().hipMemcpy(logits.ctypes.data, lib().kore_model_logits_dev(self._h), logits.nbytes,
                                          hip.D2H), "logits")
        return rows, logits

    def read_kv(self, layer: int, pos0: int, n: int):
        from . import _lib
        kvd = self.info.kv_dim
        k, v = np.zeros((n, kvd), np.float32), np.zeros((n, kvd), np.float32)
        rc = _lib.lib().kore_attn_read_kv(lib().kore_model_attn(self._h), layer, pos0, n, k.ctypes.data,
                                          v.ctypes.data)
        if rc != 0:
            raise ModelError(KORE_MODEL_E_DEVICE, _lib.lib().kore_attn_last_error(None).decode())
        return k, v

    def close(self):
        if self._h:
            lib().kore_model_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
