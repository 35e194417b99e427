"""Quantised matrix-vector product of kore on the MI355X (libkore_qmv.so).

Mirrors kore's ``quant()`` / ``mv()`` pair (kore.cpp:1387-1394): activations
are quantised to Q8_K blocks (``quantize_row_q8_K``, kore.cpp:422-446) and
every row of a Q4_K or Q6_K weight matrix is dotted with them
(``matvec_mt``, kore.cpp:649-682).  Results are kore's, bit for bit, in its
AVX2 summation order (``avx2=True``, what kore runs on an AVX2/FMA CPU) or its
scalar reference order (``avx2=False``)::

    w = QMat(KORE_QMV_Q4_K, rows, cols, gguf_block_bytes)
    xq = quantize(x)                 # kore's BlockQ8K records (Q8K_DTYPE)
    out = w.matvec(xq)               # kore's matvec_mt(t, xq, out, avx2, nth)
    out = w.mv(x)                    # quant() + mv()

There is no CPU fallback: without the built library or a GPU every call raises.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkore_qmv.so")

KORE_QMV_Q4_K, KORE_QMV_Q6_K = 12, 14
BLOCK_BYTES = {KORE_QMV_Q4_K: 144, KORE_QMV_Q6_K: 210}
KORE_QMV_OK, KORE_QMV_E_INVALID, KORE_QMV_E_UNSUPPORTED, KORE_QMV_E_HIP, KORE_QMV_E_NOMEM = 0, -1, -3, -4, -5

# kore's BlockQ8K (kore.cpp:415-420)
Q8K_DTYPE = np.dtype([("d", "<f4"), ("qs", "i1", (256,)), ("bsums", "<i2", (16,))])
assert Q8K_DTYPE.itemsize == 292

_vp, _i, _i64 = C.c_void_p, C.c_int, C.c_int64


class QmvInfo(C.Structure):
    _fields_ = [("type", C.c_int), ("device", C.c_int), ("rows", C.c_int64), ("cols", C.c_int64),
                ("weight_bytes", C.c_size_t), ("rows_per_wave", C.c_int)]


SYMBOLS = [
    ("kore_qmv_tensor_create", _i, [C.POINTER(_vp), _i, _i64, _i64, _vp, _i]),
    ("kore_qmv_tensor_destroy", None, [_vp]),
    ("kore_qmv_quantize", _i, [_vp, _i64, _vp]),
    ("kore_qmv_quantize_dev", _i, [_vp, _i64, _vp, _vp]),
    ("kore_qmv_matvec", _i, [_vp, _vp, _vp, _i]),
    ("kore_qmv_matvec_dev", _i, [_vp, _vp, _vp, _i, _vp]),
    ("kore_qmv_mv", _i, [_vp, _vp, _vp, _i]),
    ("kore_qmv_mv_dev", _i, [_vp, _vp, _vp, _i, _vp]),
    ("kore_qmv_mv_group_dev", _i, [_i, _vp, _vp, _vp, _i, _vp]),
    ("kore_qmv_matmul_batch", _i, [_vp, _vp, _i, _vp]),
    ("kore_qmv_matmul_batch_dev", _i, [_vp, _vp, _i, _vp, _vp]),
    ("kore_qmv_matmul_batch_group_dev", _i, [_i, _vp, _vp, _i, _vp, _vp]),
    ("kore_qmv_mv_group_ex_dev", _i, [_i, _vp, _vp, _vp, _vp, _i, _vp]),
    ("kore_qmv_get_row_dev", _i, [_i, _vp, _i64, _i64, _vp, _vp]),
    ("kore_qmv_matmul_batch_group_ex_dev", _i, [_i, _vp, _vp, _i, _vp, _vp, _vp]),
    ("kore_qmv_rmsnorm_rows_dev", _i, [_vp, _vp, _i64, _i, C.c_float, _vp, _vp]),
    ("kore_qmv_split_bytes", C.c_size_t, [_i64]),
    ("kore_qmv_rmsnorm_rows_split_dev", _i, [_vp, _vp, _i64, _i, C.c_float, _vp, _vp, _vp]),
    ("kore_qmv_matmul_batch_group_split_dev", _i, [_i, _vp, _vp, _i, _vp, _vp, _vp]),
    ("kore_qmv_swiglu_dev", _i, [_vp, _vp, _i64, _vp]),
    ("kore_qmv_matmul_batch_glu_split_dev", _i, [_vp, _vp, _i, _vp, _vp, _vp]),
    ("kore_qmv_last_error", C.c_char_p, [_vp]),
    ("kore_qmv_get_info", _i, [_vp, C.POINTER(QmvInfo)]),
    ("kore_qmv_synth_dev", _i, [_i, _i64, _i64, C.c_uint64, _vp, _vp]),
]

_lib = None


class QmvError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            from ._lib import LibraryMissing
            raise LibraryMissing(f"{LIB_PATH} is not built; run `make -C kore_amd/csrc` (or __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        for name, res, args in SYMBOLS:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _check(rc: int, t=None):
    if rc != KORE_QMV_OK:
        raise QmvError(rc, lib().kore_qmv_last_error(t).decode())


def _u8(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a).view(np.uint8) if np.asarray(a).dtype != np.uint8 else a,
                                np.uint8).reshape(-1)


def quantize(x) -> np.ndarray:
    """kore's quantize_row_q8_K on the GPU: x (n floats, n % 256 == 0) ->
    n/256 BlockQ8K records."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.zeros(max(x.size // 256, 1), Q8K_DTYPE)
    _check(lib().kore_qmv_quantize(x.ctypes.data, x.size, out.ctypes.data))
    return out[:x.size // 256]


def quantize_dev(x_ptr: int, n: int, xq_ptr: int, stream=None) -> None:
    _check(lib().kore_qmv_quantize_dev(x_ptr, n, xq_ptr, stream))


def synth_dev(wtype: int, rows: int, cols: int, seed: int, dst_ptr: int, stream=None) -> None:
    """Synthetic GGUF blocks straight into device memory (include/kore_qmv_synth.h)."""
    _check(lib().kore_qmv_synth_dev(wtype, rows, cols, seed, dst_ptr, stream))


class QMat:
    """A device-resident Q4_K / Q6_K weight matrix (kore's Tensor)."""

    def __init__(self, wtype: int, rows: int, cols: int, data=None, *, device_ptr: int | None = None):
        self.handle = C.c_void_p()
        self.type, self.rows, self.cols = wtype, rows, cols
        if device_ptr is not None:
            _check(lib().kore_qmv_tensor_create(C.byref(self.handle), wtype, rows, cols, device_ptr, 1))
        else:
            w = _u8(data)
            bb = BLOCK_BYTES.get(wtype)
            if bb is not None and cols % 256 == 0 and w.size != rows * (cols // 256) * bb:
                raise ValueError(f"expected {rows * (cols // 256) * bb} weight bytes, got {w.size}")
            _check(lib().kore_qmv_tensor_create(C.byref(self.handle), wtype, rows, cols, w.ctypes.data, 0))

    @classmethod
    def adopt(cls, handle: C.c_void_p, wtype: int, rows: int, cols: int) -> "QMat":
        """Wrap a tensor another library created (kore_gguf_to_qmv); it is destroyed on close."""
        m = cls.__new__(cls)
        m.handle, m.type, m.rows, m.cols = handle, wtype, int(rows), int(cols)
        return m

    def close(self):
        if self.handle:
            lib().kore_qmv_tensor_destroy(self.handle)
            self.handle = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def info(self) -> QmvInfo:
        inf = QmvInfo()
        _check(lib().kore_qmv_get_info(self.handle, C.byref(inf)), self.handle)
        return inf

    def matvec(self, xq: np.ndarray, avx2: bool = True) -> np.ndarray:
        xq = np.ascontiguousarray(xq, Q8K_DTYPE)
        if xq.size != self.cols // 256:
            raise ValueError(f"xq must hold {self.cols // 256} blocks")
        out = np.zeros(self.rows, np.float32)
        _check(lib().kore_qmv_matvec(self.handle, xq.ctypes.data, out.ctypes.data, int(avx2)), self.handle)
        return out

    def mv(self, x, avx2: bool = True) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        if x.size != self.cols:
            raise ValueError(f"x must hold {self.cols} floats")
        out = np.zeros(self.rows, np.float32)
        _check(lib().kore_qmv_mv(self.handle, x.ctypes.data, out.ctypes.data, int(avx2)), self.handle)
        return out

    def matmul_batch(self, x) -> np.ndarray:
        """kore's matmul_batch_float: x [nb][cols] (nb <= 64) -> [nb][rows]."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.cols)
        out = np.zeros((x.shape[0], self.rows), np.float32)
        _check(lib().kore_qmv_matmul_batch(self.handle, x.ctypes.data, x.shape[0], out.ctypes.data), self.handle)
        return out

    def matmul_batch_dev(self, x_ptr: int, nb: int, out_ptr: int, stream=None) -> None:
        _check(lib().kore_qmv_matmul_batch_dev(self.handle, x_ptr, nb, out_ptr, stream), self.handle)

    def matvec_dev(self, xq_ptr: int, out_ptr: int, avx2: bool = True, stream=None) -> None:
        _check(lib().kore_qmv_matvec_dev(self.handle, xq_ptr, out_ptr, int(avx2), stream), self.handle)

    def mv_dev(self, x_ptr: int, out_ptr: int, avx2: bool = True, stream=None) -> None:
        _check(lib().kore_qmv_mv_dev(self.handle, x_ptr, out_ptr, int(avx2), stream), self.handle)


def mv_group_dev(mats, x_ptr: int, out_ptrs, avx2: bool = True, stream=None) -> None:
    """One launch of up to 4 matrices sharing the input x (device pointers)."""
    n = len(mats)
    hs = (C.c_void_p * n)(*[m.handle.value for m in mats])
    outs = (C.c_void_p * n)(*out_ptrs)
    _check(lib().kore_qmv_mv_group_dev(n, hs, x_ptr, outs, int(avx2), stream))


def matmul_batch_group_dev(mats, x_ptr: int, nb: int, out_ptrs, stream=None) -> None:
    """One batched-matmul launch of up to 4 matrices of equal cols sharing x
    [nb][cols] (device pointers); out_ptrs[k] receives [nb][rows_k]."""
    n = len(mats)
    hs = (C.c_void_p * n)(*[m.handle.value for m in mats])
    outs = (C.c_void_p * n)(*out_ptrs)
    _check(lib().kore_qmv_matmul_batch_group_dev(n, hs, x_ptr, nb, outs, stream))


class MvOpts(C.Structure):
    """kore_qmv_mv_opts: the steps fused around a matvec launch."""
    _fields_ = [("norm_w", C.c_void_p), ("norm_eps", C.c_float), ("up", C.c_void_p), ("bias", C.c_void_p * 4),
                ("accumulate", C.c_int)]


def mv_group_ex_dev(mats, x_ptr: int, out_ptrs, norm_w: int = None, norm_eps: float = 0.0, up: int = None,
                    bias=None, accumulate: bool = False, avx2: bool = True, stream=None) -> None:
    """kore_qmv_mv_group_ex_dev: rmsnorm (norm_w) or SwiGLU (up) on x before
    the quantisation, bias per matrix and/or out += in the store (device
    pointers)."""
    n = len(mats)
    o = MvOpts()
    o.norm_w, o.norm_eps, o.up, o.accumulate = norm_w, norm_eps, up, int(accumulate)
    for k, b in enumerate(bias or ()):
        o.bias[k] = b
    hs = (C.c_void_p * n)(*[m.handle.value for m in mats])
    outs = (C.c_void_p * n)(*out_ptrs)
    _check(lib().kore_qmv_mv_group_ex_dev(n, hs, x_ptr, C.byref(o), outs, int(avx2), stream))


def matmul_batch_group_ex_dev(mats, x_ptr: int, nb: int, out_ptrs, bias=None, accumulate: bool = False,
                              stream=None) -> None:
    """kore_qmv_matmul_batch_group_ex_dev: the batched matmul with bias per
    matrix and/or out += in the final store (device pointers)."""
    n = len(mats)
    o = MvOpts()
    o.accumulate = int(accumulate)
    for k, b in enumerate(bias or ()):
        o.bias[k] = b
    hs = (C.c_void_p * n)(*[m.handle.value for m in mats])
    outs = (C.c_void_p * n)(*out_ptrs)
    _check(lib().kore_qmv_matmul_batch_group_ex_dev(n, hs, x_ptr, nb, C.byref(o), outs, stream))


def rmsnorm_rows_dev(x_ptr: int, w_ptr: int, n: int, rows: int, eps: float, out_ptr: int, stream=None) -> None:
    """kore's rmsnorm of `rows` rows of n floats (device pointers)."""
    _check(lib().kore_qmv_rmsnorm_rows_dev(x_ptr, w_ptr, n, rows, eps, out_ptr, stream))


def split_bytes(cols: int) -> int:
    """kore_qmv_split_bytes: bytes of the fp16 activation split of up to 64
    rows of cols values (0: not available, use the plain calls)."""
    return int(lib().kore_qmv_split_bytes(cols))


def rmsnorm_rows_split_dev(x_ptr: int, w_ptr: int, n: int, rows: int, eps: float, out_ptr: int, x16_ptr: int,
                           stream=None) -> None:
    """kore_qmv_rmsnorm_rows_split_dev: rmsnorm_rows_dev, also writing the
    rows' fp16 split into x16 (device, split_bytes(n) bytes)."""
    _check(lib().kore_qmv_rmsnorm_rows_split_dev(x_ptr, w_ptr, n, rows, eps, out_ptr, x16_ptr, stream))


def matmul_batch_group_split_dev(mats, x16_ptr: int, nb: int, out_ptrs, bias=None, accumulate: bool = False,
                                 stream=None) -> None:
    """kore_qmv_matmul_batch_group_split_dev: matmul_batch_group_ex_dev on the
    split written by rmsnorm_rows_split_dev."""
    n = len(mats)
    o = MvOpts()
    o.accumulate = int(accumulate)
    for k, b in enumerate(bias or ()):
        o.bias[k] = b
    hs = (C.c_void_p * n)(*[m.handle.value for m in mats])
    outs = (C.c_void_p * n)(*out_ptrs)
    _check(lib().kore_qmv_matmul_batch_group_split_dev(n, hs, x16_ptr, nb, C.byref(o), outs, stream))


def matmul_batch_glu_split_dev(gate, up, x16_ptr: int, nb: int, out_ptr: int, tmp_ptr: int, stream=None) -> None:
    """kore_qmv_matmul_batch_glu_split_dev: SwiGLU(gate . x, up . x) of the nb
    activations split in x16 into out (tmp: nb * rows floats of scratch)."""
    hs = (C.c_void_p * 2)(gate.handle.value, up.handle.value)
    _check(lib().kore_qmv_matmul_batch_glu_split_dev(hs, x16_ptr, nb, out_ptr, tmp_ptr, stream))


def swiglu_dev(g_ptr: int, u_ptr: int, n: int, stream=None) -> None:
    """kore's batched SwiGLU in place over n floats (device pointers)."""
    _check(lib().kore_qmv_swiglu_dev(g_ptr, u_ptr, n, stream))
