"""Loader of libkore_attn.so (built in-tree by kore_amd/csrc/Makefile).

There is no fallback: if the library is missing or does not load, every entry
point raises.  The exported symbols are exactly those declared in
include/kore_attn.h and include/kore_attn_synth.h.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkore_attn.so")

# (name, restype, argtypes) of every exported function.
_vp, _fp, _i, _f = C.c_void_p, C.POINTER(C.c_float), C.c_int, C.c_float


class AttnInfo(C.Structure):
    _fields_ = [("n_layer", C.c_int), ("ctx", C.c_int), ("n_head", C.c_int),
                ("n_head_kv", C.c_int), ("head_dim", C.c_int), ("window", C.c_int),
                ("device", C.c_int), ("num_cu", C.c_int), ("kv_bytes", C.c_size_t),
                ("stream", C.c_void_p)]


SYMBOLS = [
    ("kore_attn_create", _i, [C.POINTER(_vp), _i, _i, _i, _i, _i, _f, _i]),
    ("kore_attn_destroy", None, [_vp]),
    ("kore_attn_decode", _i, [_vp, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp]),
    ("kore_attn_prefill", _i, [_vp, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp]),
    ("kore_attn_read_kv", _i, [_vp, _i, _i, _i, _vp, _vp]),
    ("kore_attn_last_error", C.c_char_p, [_vp]),
    ("kore_attn_decode_dev", _i, [_vp, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp]),
    ("kore_attn_decode_noalloc_dev", _i, [_vp, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp]),
    ("kore_attn_prefill_dev", _i, [_vp, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp]),
    ("kore_attn_append_dev", _i, [_vp, _i, _i, _i, _vp, _vp, _vp]),
    ("kore_attn_sync", _i, [_vp]),
    ("kore_attn_get_info", _i, [_vp, C.POINTER(AttnInfo)]),
    ("kore_attn_synth_dev", _i, [_vp, _i, _i, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64,
                                 C.c_uint32, _f, _vp]),
]

_lib = None


class LibraryMissing(RuntimeError):
    pass


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise LibraryMissing(
                f"{LIB_PATH} is not built; run `make -C kore_amd/csrc` (or __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        for name, res, args in SYMBOLS:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib
