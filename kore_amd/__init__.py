"""kore_amd - MI355X (gfx950) attention path of kore: RoPE-NEOX, fp32 KV-cache
append and GQA softmax attention for single-token decode and batched causal
prefill, as hand-written HIP kernels behind the C ABI of include/kore_attn.h.

``KoreAttn`` mirrors kore's per-layer attention step (the inline blocks of
``forward()`` kore.cpp:1405-1455 and ``forward_batch()`` kore.cpp:1503-1563)
over a device-resident KV cache:

    attn = KoreAttn(n_layer=28, ctx=8192, n_head=28, n_head_kv=4, head_dim=128)
    out = attn.decode(layer, pos, q, k, v)          # kore's e.att
    out = attn.prefill(layer, pos0, q, k, v)        # kore's e.batt
    k_rows, v_rows = attn.read_kv(layer, pos0, n)   # kore's cache layout

Calls kore rejects (``forward()``/``forward_batch()`` returning false,
kore.cpp:1400, 1490) raise ``KoreAttnError`` with ``code ==
KORE_ATTN_E_RANGE``.  There is no CPU fallback: without the built library or
a GPU every call raises.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib

KORE_ATTN_OK = 0
KORE_ATTN_E_INVALID = -1
KORE_ATTN_E_RANGE = -2
KORE_ATTN_E_UNSUPPORTED = -3
KORE_ATTN_E_HIP = -4
KORE_ATTN_E_NOMEM = -5


class KoreAttnError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


def _f32(a, shape) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    if a.size != int(np.prod(shape)):
        raise ValueError(f"expected {shape} floats, got array of shape {a.shape}")
    return a


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


class KoreAttn:
    """One KV-cache handle (``kore_attn_t``) on the current HIP device."""

    def __init__(self, n_layer: int, ctx: int, n_head: int, n_head_kv: int, head_dim: int,
                 rope_base: float = 1e6, window: int = 0):
        self._h = None
        L = _lib.lib()
        h = C.c_void_p()
        rc = L.kore_attn_create(C.byref(h), n_layer, ctx, n_head, n_head_kv, head_dim,
                                rope_base, window)
        if rc != 0:
            raise KoreAttnError(rc, L.kore_attn_last_error(None).decode())
        self._h = h
        self.n_layer, self.ctx, self.n_head, self.n_head_kv = n_layer, ctx, n_head, n_head_kv
        self.head_dim, self.rope_base, self.window = head_dim, rope_base, window
        self.E = n_head * head_dim
        self.kv_dim = n_head_kv * head_dim

    # -- plumbing
    def _check(self, rc: int) -> None:
        if rc != 0:
            raise KoreAttnError(rc, _lib.lib().kore_attn_last_error(self._h).decode())

    @property
    def handle(self):
        return self._h

    def info(self) -> "_lib.AttnInfo":
        inf = _lib.AttnInfo()
        self._check(_lib.lib().kore_attn_get_info(self._h, C.byref(inf)))
        return inf

    @property
    def stream(self) -> int:
        return self.info().stream

    def close(self) -> None:
        if self._h:
            _lib.lib().kore_attn_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- kore's per-layer calls (host buffers, synchronous)
    def decode(self, layer: int, pos: int, q, k, v) -> np.ndarray:
        q = _f32(q, (self.E,))
        k = _f32(k, (self.kv_dim,))
        v = _f32(v, (self.kv_dim,))
        out = np.empty(self.E, np.float32)
        self._check(_lib.lib().kore_attn_decode(self._h, layer, pos, self.n_head, self.n_head_kv,
                                                self.head_dim, _ptr(q), _ptr(k), _ptr(v), _ptr(out)))
        return out

    def prefill(self, layer: int, pos0: int, q, k, v) -> np.ndarray:
        q = np.ascontiguousarray(q, np.float32).reshape(-1, self.E)
        n = q.shape[0]
        k = _f32(k, (n, self.kv_dim))
        v = _f32(v, (n, self.kv_dim))
        out = np.empty((n, self.E), np.float32)
        self._check(_lib.lib().kore_attn_prefill(self._h, layer, pos0, n, self.n_head, self.n_head_kv,
                                                 self.head_dim, _ptr(q), _ptr(k), _ptr(v), _ptr(out)))
        return out

    def read_kv(self, layer: int, pos0: int, n: int):
        k = np.empty((n, self.kv_dim), np.float32)
        v = np.empty((n, self.kv_dim), np.float32)
        self._check(_lib.lib().kore_attn_read_kv(self._h, layer, pos0, n, _ptr(k), _ptr(v)))
        return k, v

    # -- device-pointer variants (asynchronous on `stream`, None = own stream)
    def decode_dev(self, layer: int, pos: int, q: int, k: int, v: int, out: int, stream=None) -> None:
        self._check(_lib.lib().kore_attn_decode_dev(self._h, layer, pos, self.n_head, self.n_head_kv,
                                                    self.head_dim, q, k, v, out, stream))

    def decode_noalloc_dev(self, layer: int, pos: int, q: int, k: int, v: int, out: int, stream=None) -> None:
        """decode_dev with the split partials in the library's fixed device array
        (allocates nothing; overlapping calls on one GPU race)."""
        self._check(_lib.lib().kore_attn_decode_noalloc_dev(self._h, layer, pos, self.n_head, self.n_head_kv,
                                                            self.head_dim, q, k, v, out, stream))

    def prefill_dev(self, layer: int, pos0: int, n_tok: int, q: int, k: int, v: int, out: int,
                    stream=None) -> None:
        self._check(_lib.lib().kore_attn_prefill_dev(self._h, layer, pos0, n_tok, self.n_head,
                                                     self.n_head_kv, self.head_dim, q, k, v, out,
                                                     stream))

    def append_dev(self, layer: int, pos0: int, n_tok: int, k: int, v: int, stream=None) -> None:
        """RoPE + append of n_tok device rows without attention (cache fill)."""
        self._check(_lib.lib().kore_attn_append_dev(self._h, layer, pos0, n_tok, k, v, stream))

    def sync(self) -> None:
        self._check(_lib.lib().kore_attn_sync(self._h))


def synth_dev(dst: int, rows: int, dim: int, seed: int, stream_id: int, row0: int = 0,
              tensor: int = 0, per_mille: int = 0, outlier_scale: float = 20.0,
              stream=None) -> None:
    """Fill device memory with the counter-based synthetic inputs (same bits
    as the CPU oracle's generator)."""
    rc = _lib.lib().kore_attn_synth_dev(dst, rows, dim, seed, stream_id, row0, tensor, per_mille,
                                        outlier_scale, stream)
    if rc != 0:
        raise KoreAttnError(rc, _lib.lib().kore_attn_last_error(None).decode())


__all__ = ["KoreAttn", "KoreAttnError", "synth_dev", "KORE_ATTN_OK", "KORE_ATTN_E_INVALID",
           "KORE_ATTN_E_RANGE", "KORE_ATTN_E_UNSUPPORTED", "KORE_ATTN_E_HIP", "KORE_ATTN_E_NOMEM"]
