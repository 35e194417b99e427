"""ctypes binding of include/kore_gguf.h (in kore_amd/libkore_layer.so): kore's
GGUF parse (load_model, kore.cpp:188-285) and the copies of its tensors into
HBM.

    with GGUF(path) as g:
        hp = g.hparams()                 # kore's Hparams
        t = g.find("blk.0.attn_q.weight")
        wq = g.to_qmv("blk.0.attn_q.weight")        # a qmv.QMat on the device
        norm = g.to_device_f32("blk.0.attn_norm.weight")
"""
from __future__ import annotations

import ctypes as C

from . import qmv
from .layer import lib as _layer_lib

KORE_GGUF_OK, KORE_GGUF_E_IO, KORE_GGUF_E_FORMAT, KORE_GGUF_E_NOT_FOUND, KORE_GGUF_E_TYPE, KORE_GGUF_E_DEVICE = range(6)


class Hparams(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("n_layer", "n_embd", "n_ff", "n_head", "n_head_kv", "n_ctx", "n_vocab")] + \
               [("rope_base", C.c_float), ("rms_eps", C.c_float), ("version", C.c_uint32),
                ("alignment", C.c_uint64), ("data_start", C.c_uint64), ("file_size", C.c_uint64)]


class Tensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("type", C.c_uint32), ("n_dims", C.c_uint32), ("dims", C.c_uint64 * 4),
                ("nbytes", C.c_uint64), ("data", C.c_void_p)]

    def bytes(self) -> bytes:
        return C.string_at(self.data, self.nbytes) if self.data else b""


_done = False


def lib() -> C.CDLL:
    global _done
    L = _layer_lib()
    if not _done:
        vp = C.c_void_p
        for name, res, args in (("kore_gguf_open", C.c_int, [C.c_char_p, C.POINTER(vp)]),
                                ("kore_gguf_close", None, [vp]),
                                ("kore_gguf_get_hparams", C.c_int, [vp, C.POINTER(Hparams)]),
                                ("kore_gguf_tensor_count", C.c_int64, [vp]),
                                ("kore_gguf_tensor_at", C.c_int, [vp, C.c_int64, C.POINTER(Tensor)]),
                                ("kore_gguf_find", C.c_int, [vp, C.c_char_p, C.POINTER(Tensor)]),
                                ("kore_gguf_to_qmv", C.c_int, [vp, C.c_char_p, C.POINTER(vp)]),
                                ("kore_gguf_to_device_f32", C.c_int, [vp, C.c_char_p, C.POINTER(vp)]),
                                ("kore_gguf_free_device", None, [vp]),
                                ("kore_gguf_last_error", C.c_char_p, [vp])):
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _done = True
    return L


class GGUFError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"kore_gguf error {code}: {message}")
        self.code = code


class DeviceArray:
    """A device copy of an F32 tensor (kore_gguf_to_device_f32)."""

    def __init__(self, ptr: int, n: int):
        self.ptr, self.n = ptr, n

    def free(self):
        if self.ptr:
            lib().kore_gguf_free_device(self.ptr)
            self.ptr = None


class GGUF:
    def __init__(self, path: str):
        h = C.c_void_p()
        rc = lib().kore_gguf_open(path.encode(), C.byref(h))
        if rc != KORE_GGUF_OK:
            raise GGUFError(rc, lib().kore_gguf_last_error(None).decode())
        self._h = h

    def _check(self, rc):
        if rc != KORE_GGUF_OK:
            raise GGUFError(rc, lib().kore_gguf_last_error(self._h).decode())

    def hparams(self) -> Hparams:
        hp = Hparams()
        self._check(lib().kore_gguf_get_hparams(self._h, C.byref(hp)))
        return hp

    def tensors(self):
        out = []
        for i in range(lib().kore_gguf_tensor_count(self._h)):
            t = Tensor()
            self._check(lib().kore_gguf_tensor_at(self._h, i, C.byref(t)))
            out.append(t)
        return out

    def find(self, name: str) -> Tensor:
        t = Tensor()
        self._check(lib().kore_gguf_find(self._h, name.encode(), C.byref(t)))
        return t

    def to_qmv(self, name: str) -> "qmv.QMat":
        t = self.find(name)
        h = C.c_void_p()
        self._check(lib().kore_gguf_to_qmv(self._h, name.encode(), C.byref(h)))
        return qmv.QMat.adopt(h, t.type, t.dims[1] * t.dims[2] * t.dims[3], t.dims[0])

    def to_device_f32(self, name: str) -> DeviceArray:
        t = self.find(name)
        p = C.c_void_p()
        self._check(lib().kore_gguf_to_device_f32(self._h, name.encode(), C.byref(p)))
        return DeviceArray(p.value, t.nbytes // 4)

    def close(self):
        if self._h:
            lib().kore_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
