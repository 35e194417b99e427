"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: the parity checker and the timed CPU baseline.
Only tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
import this module, and only to check or time against; the product path
(``kore_amd``) never imports it.

The C functions restate kore.cpp's RoPE / KV-append / attention arithmetic in
kore's operation order (citations in oracle/kore_oracle.c).  The KV store
``KV`` mirrors kore's ``Engine::kcache/vcache`` layout ``[layer][pos][kv_dim]``
(kore.cpp:1260).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_BIN = os.path.join(HERE, "_ref", "kore_ref")
REF_QMV_BIN = os.path.join(HERE, "_ref", "kore_qmv_ref")
REF_LAYER_BIN = os.path.join(HERE, "_ref", "kore_layer_ref")
# kore.cpp with the attention binding of INTEGRATION.md applied, linked to the GPU library
REF_LAYER_GPU_BIN = os.path.join(HERE, "_ref", "kore_layer_gpu")

# kore's BlockQ8K (kore.cpp:415-420): d, 256 int8 values, 16 int16 sums of 16
Q8K_DTYPE = np.dtype([("d", "<f4"), ("qs", "i1", (256,)), ("bsums", "<i2", (16,))])
assert Q8K_DTYPE.itemsize == 292
TYPE_Q4K, TYPE_Q6K = 12, 14
BLOCK_BYTES = {TYPE_Q4K: 144, TYPE_Q6K: 210}

_F = C.POINTER(C.c_float)
_D = C.POINTER(C.c_double)
_I = C.POINTER(C.c_int)


class _KV(C.Structure):
    _fields_ = [
        ("n_layer", C.c_int), ("ctx", C.c_int), ("n_head", C.c_int), ("n_head_kv", C.c_int),
        ("head_dim", C.c_int), ("window", C.c_int), ("rope_base", C.c_float),
        ("kcache", _F), ("vcache", _F), ("inv_freq", _F), ("scores", _F),
    ]


def build() -> None:
    """Compile liboracle.so (gcc) and, when the kore sources are present,
    kore's own harnesses under oracle/_ref/ (kore_ref, kore_qmv_ref,
    kore_layer_ref) and kore with the attention binding linked to the GPU
    library (kore_layer_gpu, once kore_amd/libkore_attn.so is built)."""
    subprocess.run(["make", "-s", "-C", HERE, "-B", "all"], check=True)
    if os.path.exists(os.path.join(os.environ.get("KORE_SRC", "/root/reference"), "kore.cpp")):
        subprocess.run(["make", "-s", "-C", HERE, "-B", "ref"], check=True)
        if os.path.exists(os.path.join(os.path.dirname(HERE.rstrip("/")), "kore_amd", "libkore_attn.so")):
            subprocess.run(["make", "-s", "-C", HERE, "-B", "ref-gpu"], check=True)


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)
        L = C.CDLL(LIB_PATH)
        L.ko_inv_freq.argtypes = [C.c_int, C.c_float, _F]
        L.ko_rope_cs.argtypes = [C.c_int, C.c_int, _F, _F, _F]
        L.ko_inv_sqrt.argtypes = [C.c_int]
        L.ko_inv_sqrt.restype = C.c_float
        L.ko_rope_neox.argtypes = [_F, C.c_int, C.c_int, _F, _F]
        L.ko_rope_rows.argtypes = [_F, C.c_int, C.c_int, C.c_int, _I, _F]
        L.ko_attn_decode.argtypes = [_F, _F, _F, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, _F, _F]
        L.ko_hd_dot.argtypes = [_F, _F, C.c_int, C.c_int]
        L.ko_hd_dot.restype = C.c_float
        L.ko_hd_fma.argtypes = [_F, _F, C.c_float, C.c_int, C.c_int]
        L.ko_attn_batch.argtypes = [_F, C.c_int, C.c_int, _F, _F, C.c_int, C.c_int, C.c_int,
                                    C.c_float, C.c_int, _F, _F]
        L.ko_kv_init.argtypes = [C.POINTER(_KV), C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                 C.c_float, C.c_int]
        L.ko_kv_free.argtypes = [C.POINTER(_KV)]
        L.ko_decode.argtypes = [C.POINTER(_KV), C.c_int, C.c_int, _F, _F, _F, _F]
        L.ko_prefill.argtypes = [C.POINTER(_KV), C.c_int, C.c_int, C.c_int, _F, _F, _F, _F, C.c_int]
        L.ko_attn_ref64.argtypes = [_F, _F, _F, _I, C.c_int, C.c_int, C.c_int, C.c_int, _D]
        L.ko_splitmix64.argtypes = [C.c_uint64]
        L.ko_splitmix64.restype = C.c_uint64
        L.ko_synth_value.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64]
        L.ko_synth_value.restype = C.c_float
        L.ko_synth_is_outlier.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint32]
        L.ko_synth_fill.argtypes = [_F, C.c_int, C.c_int, C.c_uint64, C.c_uint64, C.c_uint64,
                                    C.c_uint64, C.c_uint32, C.c_float]
        L.ko_cpu_has_fma.restype = C.c_int
        _u8 = C.c_void_p
        L.ko_f16.argtypes = [C.c_uint16]
        L.ko_f16.restype = C.c_float
        L.ko_quantize_q8K.argtypes = [_F, C.c_int64, _u8]
        for name in ("ko_dot_q4K_ref", "ko_dot_q6K_ref", "ko_dot_q4K_avx2", "ko_dot_q6K_avx2"):
            getattr(L, name).argtypes = [C.c_int64, _u8, _u8]
            getattr(L, name).restype = C.c_float
        L.ko_dot_q6K_avx2_v.argtypes = [C.c_int64, _u8, _u8, C.c_int]
        L.ko_dot_q6K_avx2_v.restype = C.c_float
        L.ko_qmatvec.argtypes = [C.c_int, C.c_int64, C.c_int64, _u8, _u8, _F, C.c_int]
        L.ko_dequant_row.argtypes = [C.c_int, C.c_int64, _u8, _F]
        L.ko_matmul_batch.argtypes = [C.c_int, C.c_int64, C.c_int64, _u8, _F, C.c_int, _F, C.c_int]
        L.ko_rmsnorm.argtypes = [_F, _F, _F, C.c_int, C.c_float]
        L.ko_swiglu.argtypes = [_F, _F, C.c_int]
        _lib = L
    return _lib


def fptr(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_F)


def dptr(a: np.ndarray):
    assert a.dtype == np.float64 and a.flags.c_contiguous
    return a.ctypes.data_as(_D)


# ---------------------------------------------------------------- functions

def inv_freq(head_dim: int, rope_base: float) -> np.ndarray:
    out = np.zeros(head_dim // 2, np.float32)
    lib().ko_inv_freq(head_dim, rope_base, fptr(out))
    return out


def rope_cs(pos: int, head_dim: int, inv_f: np.ndarray):
    c = np.zeros(head_dim // 2, np.float32)
    s = np.zeros(head_dim // 2, np.float32)
    lib().ko_rope_cs(pos, head_dim, fptr(np.ascontiguousarray(inv_f, np.float32)), fptr(c), fptr(s))
    return c, s


def inv_sqrt(head_dim: int) -> float:
    return float(lib().ko_inv_sqrt(head_dim))


def rope_neox(vec: np.ndarray, n_heads: int, head_dim: int, c: np.ndarray, s: np.ndarray) -> np.ndarray:
    out = np.array(vec, np.float32, copy=True, order="C")
    lib().ko_rope_neox(fptr(out), n_heads, head_dim, fptr(c), fptr(s))
    return out


def rope_rows(x: np.ndarray, positions, n_heads: int, head_dim: int, inv_f: np.ndarray) -> np.ndarray:
    """Rows ``x[r]`` rotated at ``positions[r]`` (kore's per-row RoPE)."""
    out = np.array(x, np.float32, copy=True, order="C").reshape(len(positions), n_heads * head_dim)
    pos = np.ascontiguousarray(np.asarray(positions, np.int32))
    lib().ko_rope_rows(fptr(out), out.shape[0], n_heads, head_dim, pos.ctypes.data_as(_I),
                       fptr(np.ascontiguousarray(inv_f, np.float32)))
    return out


def attn_decode(q_roped: np.ndarray, kc: np.ndarray, vc: np.ndarray, pos: int, n_head: int,
                n_head_kv: int, head_dim: int) -> np.ndarray:
    """kore's decode attention block (kore.cpp:1432-1455) over cache rows
    0..pos in kore layout ``[row][kv_dim]``."""
    out = np.zeros(n_head * head_dim, np.float32)
    sc = np.zeros(pos + 1, np.float32)
    kc = np.ascontiguousarray(kc, np.float32)
    vc = np.ascontiguousarray(vc, np.float32)
    lib().ko_attn_decode(fptr(np.ascontiguousarray(q_roped, np.float32)), fptr(kc), fptr(vc), pos,
                         n_head, n_head_kv, head_dim, inv_sqrt(head_dim), fptr(sc), fptr(out))
    return out


def attn_batch(bq_roped: np.ndarray, pos0: int, kc: np.ndarray, vc: np.ndarray, n_head: int,
               n_head_kv: int, head_dim: int, avx2: bool = True) -> np.ndarray:
    """kore's batched causal attention block (kore.cpp:1542-1563)."""
    bq = np.ascontiguousarray(bq_roped, np.float32).reshape(-1, n_head * head_dim)
    nb = bq.shape[0]
    out = np.zeros_like(bq)
    sc = np.zeros(pos0 + nb, np.float32)
    kc = np.ascontiguousarray(kc, np.float32)
    vc = np.ascontiguousarray(vc, np.float32)
    lib().ko_attn_batch(fptr(bq), nb, pos0, fptr(kc), fptr(vc), n_head, n_head_kv, head_dim,
                        inv_sqrt(head_dim), int(avx2), fptr(sc), fptr(out))
    return out


def hd_dot(a: np.ndarray, b: np.ndarray, avx2: bool = True) -> float:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return float(lib().ko_hd_dot(fptr(a), fptr(b), a.size, int(avx2)))


def hd_fma(o: np.ndarray, v: np.ndarray, p: float, avx2: bool = True) -> np.ndarray:
    o = np.array(o, np.float32, copy=True)
    v = np.ascontiguousarray(v, np.float32)
    lib().ko_hd_fma(fptr(o), fptr(v), p, o.size, int(avx2))
    return o


def attn_ref64(q_roped: np.ndarray, kc: np.ndarray, vc: np.ndarray, rows, n_head: int,
               n_head_kv: int, head_dim: int) -> np.ndarray:
    """Double-precision attention of one query over the given cache rows
    (kore layout ``[row][kv_dim]``)."""
    rows = np.ascontiguousarray(np.asarray(rows, np.int32))
    out = np.zeros(n_head * head_dim, np.float64)
    lib().ko_attn_ref64(fptr(np.ascontiguousarray(q_roped, np.float32)),
                        fptr(np.ascontiguousarray(kc, np.float32)),
                        fptr(np.ascontiguousarray(vc, np.float32)),
                        rows.ctypes.data_as(_I), rows.size, n_head, n_head_kv, head_dim, dptr(out))
    return out


def splitmix64(x: int) -> int:
    return int(lib().ko_splitmix64(x & 0xFFFFFFFFFFFFFFFF))


def synth(rows: int, dim: int, seed: int, stream: int, row0: int = 0, tensor: int = 0,
          per_mille: int = 0, outlier_scale: float = 20.0) -> np.ndarray:
    """Counter-based approximately N(0,1) fp32 inputs, ``[rows][dim]``."""
    out = np.zeros((rows, dim), np.float32)
    lib().ko_synth_fill(fptr(out), rows, dim, seed, stream, row0, tensor, per_mille, outlier_scale)
    return out


def cpu_has_fma() -> bool:
    return bool(lib().ko_cpu_has_fma())


# ------------------------------------------------- Q8_K / Q4_K / Q6_K matvec

def f16(h: int) -> float:
    return float(lib().ko_f16(h & 0xFFFF))


def quantize_q8K(x: np.ndarray) -> np.ndarray:
    """kore's quantize_row_q8_K (kore.cpp:422-446): ``x`` of n floats (n a
    multiple of 256) to n/256 BlockQ8K records (``Q8K_DTYPE``)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    if x.size % 256:
        raise ValueError("length must be a multiple of 256")
    out = np.zeros(x.size // 256, Q8K_DTYPE)
    lib().ko_quantize_q8K(fptr(x), x.size, out.ctypes.data)
    return out


def _w(weights: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(weights, np.uint8).reshape(-1)


def dot(wtype: int, wrow: np.ndarray, xq: np.ndarray, avx2: bool = True,
        q6k_fused_bias: int | None = None) -> float:
    """One row's Q4_K/Q6_K x Q8_K dot product (kore.cpp:450-506, 535-632)."""
    w = _w(wrow)
    xq = np.ascontiguousarray(xq, Q8K_DTYPE)
    n = 256 * xq.size
    L = lib()
    if wtype == TYPE_Q6K and avx2 and q6k_fused_bias is not None:
        return float(L.ko_dot_q6K_avx2_v(n, w.ctypes.data, xq.ctypes.data, int(q6k_fused_bias)))
    name = {(TYPE_Q4K, False): "ko_dot_q4K_ref", (TYPE_Q4K, True): "ko_dot_q4K_avx2",
            (TYPE_Q6K, False): "ko_dot_q6K_ref", (TYPE_Q6K, True): "ko_dot_q6K_avx2"}[(wtype, bool(avx2))]
    return float(getattr(L, name)(n, w.ctypes.data, xq.ctypes.data))


def qmatvec(wtype: int, weights: np.ndarray, rows: int, cols: int, xq: np.ndarray,
            avx2: bool = True) -> np.ndarray:
    """kore's matvec_rows over all rows (kore.cpp:649-660): out[r] = row r . xq."""
    w = _w(weights)
    if w.size != rows * (cols // 256) * BLOCK_BYTES[wtype]:
        raise ValueError("weights size does not match rows x cols")
    xq = np.ascontiguousarray(xq, Q8K_DTYPE)
    if xq.size != cols // 256:
        raise ValueError("xq must hold cols/256 blocks")
    out = np.zeros(rows, np.float32)
    rc = lib().ko_qmatvec(wtype, rows, cols, w.ctypes.data, xq.ctypes.data, fptr(out), int(avx2))
    if rc != 0:
        raise ValueError("ko_qmatvec rejected the type or cols")
    return out


def dequant_row(wtype: int, wrow: np.ndarray, cols: int) -> np.ndarray:
    """kore's dequant_block_q4_K / _q6_K over one row (kore.cpp:337-381)."""
    out = np.zeros(cols, np.float32)
    lib().ko_dequant_row(wtype, cols, _w(wrow).ctypes.data, fptr(out))
    return out


def matmul_batch(wtype: int, weights: np.ndarray, rows: int, cols: int, x: np.ndarray,
                 avx2: bool = True) -> np.ndarray:
    """kore's matmul_batch_float (kore.cpp:783-845): x [B][cols] -> out [B][rows]."""
    w = _w(weights)
    x = np.ascontiguousarray(x, np.float32).reshape(-1, cols)
    out = np.zeros((x.shape[0], rows), np.float32)
    rc = lib().ko_matmul_batch(wtype, rows, cols, w.ctypes.data, fptr(x), x.shape[0], fptr(out), int(avx2))
    if rc != 0:
        raise ValueError("ko_matmul_batch rejected the type, cols or B")
    return out


class KV:
    """kore-semantics KV store of the oracle (``[layer][pos][kv_dim]`` fp32,
    zero-initialised like kore.cpp:1344-1345)."""

    def __init__(self, n_layer: int, ctx: int, n_head: int, n_head_kv: int, head_dim: int,
                 rope_base: float = 1e6, window: int = 0):
        self._kv = _KV()
        rc = lib().ko_kv_init(C.byref(self._kv), n_layer, ctx, n_head, n_head_kv, head_dim,
                              rope_base, window)
        if rc != 0:
            raise ValueError(f"ko_kv_init failed ({rc})")
        self.n_layer, self.ctx, self.n_head, self.n_head_kv = n_layer, ctx, n_head, n_head_kv
        self.head_dim, self.window = head_dim, window
        self.kv_dim = n_head_kv * head_dim
        self.E = n_head * head_dim

    def close(self):
        if self._kv.kcache:
            lib().ko_kv_free(C.byref(self._kv))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def kcache(self) -> np.ndarray:
        n = self.n_layer * self.ctx * self.kv_dim
        return np.ctypeslib.as_array(self._kv.kcache, shape=(n,)).reshape(
            self.n_layer, self.ctx, self.kv_dim)

    def vcache(self) -> np.ndarray:
        n = self.n_layer * self.ctx * self.kv_dim
        return np.ctypeslib.as_array(self._kv.vcache, shape=(n,)).reshape(
            self.n_layer, self.ctx, self.kv_dim)

    def decode(self, layer: int, pos: int, q, k, v) -> np.ndarray:
        q = np.ascontiguousarray(q, np.float32).reshape(-1)
        k = np.ascontiguousarray(k, np.float32).reshape(-1)
        v = np.ascontiguousarray(v, np.float32).reshape(-1)
        out = np.zeros(self.E, np.float32)
        rc = lib().ko_decode(C.byref(self._kv), layer, pos, fptr(q), fptr(k), fptr(v), fptr(out))
        if rc != 0:
            raise ValueError(f"ko_decode rejected layer={layer} pos={pos} ({rc})")
        return out

    def prefill(self, layer: int, pos0: int, q, k, v, avx2: bool = True) -> np.ndarray:
        q = np.ascontiguousarray(q, np.float32).reshape(-1, self.E)
        k = np.ascontiguousarray(k, np.float32).reshape(-1, self.kv_dim)
        v = np.ascontiguousarray(v, np.float32).reshape(-1, self.kv_dim)
        n = q.shape[0]
        out = np.zeros((n, self.E), np.float32)
        rc = lib().ko_prefill(C.byref(self._kv), layer, pos0, n, fptr(q), fptr(k), fptr(v),
                              fptr(out), int(avx2))
        if rc != 0:
            raise ValueError(f"ko_prefill rejected layer={layer} pos0={pos0} n={n} ({rc})")
        return out


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """kore's rmsnorm (kore.cpp:1367-1372)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    w = np.ascontiguousarray(w, np.float32).reshape(-1)
    out = np.zeros_like(x)
    lib().ko_rmsnorm(fptr(out), fptr(x), fptr(w), x.size, eps)
    return out


def swiglu(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    """kore's SwiGLU (kore.cpp:1465-1468): g / (1 + exp(-g)) * u."""
    out = np.array(g, np.float32).reshape(-1)
    u = np.ascontiguousarray(u, np.float32).reshape(-1)
    lib().ko_swiglu(fptr(out), fptr(u), out.size)
    return out


class LayerWeights:
    """One layer's weights as kore holds them: the GGUF block bytes and types of
    wq, wk, wv, wo, w_gate, w_up, w_down, and the float norms and biases."""
    NAMES = ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")

    def __init__(self, types, mats, attn_norm, ffn_norm, bq, bk, bv):
        self.types, self.mats = list(types), [np.ascontiguousarray(m, np.uint8).reshape(-1) for m in mats]
        self.attn_norm, self.ffn_norm = np.asarray(attn_norm, np.float32), np.asarray(ffn_norm, np.float32)
        self.bq, self.bk, self.bv = (np.asarray(b, np.float32) for b in (bq, bk, bv))


def layer_forward(kv: "KV", layer: int, pos: int, x: np.ndarray, lw: LayerWeights, n_ff: int, eps: float,
                  avx2: bool = True) -> np.ndarray:
    """kore's forward() body for one layer on the quantised path
    (kore.cpp:1415-1472): returns the new residual x; the KV store gets the
    roped k and v at pos."""
    E, kvd = kv.E, kv.kv_dim
    x = np.array(x, np.float32).reshape(-1)
    shapes = [(E, E), (kvd, E), (kvd, E), (E, E), (n_ff, E), (n_ff, E), (E, n_ff)]

    def mv(j, xq):
        return qmatvec(lw.types[j], lw.mats[j], shapes[j][0], shapes[j][1], xq, avx2=avx2)

    xq = quantize_q8K(rmsnorm(x, lw.attn_norm, eps))
    q = mv(0, xq) + lw.bq
    k = mv(1, xq) + lw.bk
    v = mv(2, xq) + lw.bv
    att = kv.decode(layer, pos, q, k, v)
    x = x + mv(3, quantize_q8K(att))
    xq = quantize_q8K(rmsnorm(x, lw.ffn_norm, eps))
    g = swiglu(mv(4, xq), mv(5, xq))
    return x + mv(6, quantize_q8K(g))


def layer_forward_batch(kv: "KV", layer: int, pos0: int, x: np.ndarray, lw: LayerWeights, n_ff: int, eps: float,
                        avx2: bool = True) -> np.ndarray:
    """kore's forward_batch() body for one layer (kore.cpp:1518-1589) over the
    rows x [nb][E] at positions pos0..: returns the new residual rows; the KV
    store gets the roped k and v rows."""
    E, kvd = kv.E, kv.kv_dim
    x = np.array(x, np.float32).reshape(-1, E)
    shapes = [(E, E), (kvd, E), (kvd, E), (E, E), (n_ff, E), (n_ff, E), (E, n_ff)]

    def mm(j, a):
        return matmul_batch(lw.types[j], lw.mats[j], shapes[j][0], shapes[j][1], a, avx2=avx2)

    xb = np.stack([rmsnorm(r, lw.attn_norm, eps) for r in x])
    q = mm(0, xb) + lw.bq
    k = mm(1, xb) + lw.bk
    v = mm(2, xb) + lw.bv
    att = kv.prefill(layer, pos0, q, k, v, avx2=avx2)
    x = x + mm(3, att)
    xb = np.stack([rmsnorm(r, lw.ffn_norm, eps) for r in x])
    g = swiglu(mm(4, xb).reshape(-1), mm(5, xb).reshape(-1)).reshape(x.shape[0], n_ff)
    return x + mm(6, g)

