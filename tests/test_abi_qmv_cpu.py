"""CPU-side checks of the matvec C ABI (include/kore_qmv.h, kore_qmv_synth.h):
libkore_qmv.so loads, exports exactly what the headers declare, and rejects
bad arguments the way kore's matvec_rows() does (kore.cpp:650) before it
touches a GPU."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("kore_qmv.h", "kore_qmv_synth.h")]


def _declared():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= {m.group(1) for m in re.finditer(r"\b(kore_qmv_[a-z_]+)\s*\(", text)}
    return names


def _exported():
    from kore_amd import qmv
    out = subprocess.run(["nm", "-D", "--defined-only", qmv.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_headers_declare_the_abi():
    assert _declared() == {"kore_qmv_tensor_create", "kore_qmv_tensor_destroy", "kore_qmv_quantize",
                           "kore_qmv_quantize_dev", "kore_qmv_matvec", "kore_qmv_matvec_dev", "kore_qmv_mv",
                           "kore_qmv_mv_dev", "kore_qmv_mv_group_dev", "kore_qmv_mv_group_ex_dev", "kore_qmv_get_row_dev",
                           "kore_qmv_matmul_batch",
                           "kore_qmv_matmul_batch_dev", "kore_qmv_matmul_batch_group_dev",
                           "kore_qmv_matmul_batch_group_ex_dev", "kore_qmv_rmsnorm_rows_dev", "kore_qmv_swiglu_dev",
                           "kore_qmv_split_bytes", "kore_qmv_rmsnorm_rows_split_dev",
                           "kore_qmv_matmul_batch_group_split_dev", "kore_qmv_matmul_batch_glu_split_dev",
                           "kore_qmv_last_error", "kore_qmv_get_info", "kore_qmv_synth_dev"}


def test_library_exports_every_declared_symbol():
    from kore_amd import qmv
    L = qmv.lib()
    exported = _exported()
    for name in _declared():
        assert name in exported, f"{name} not exported"
        assert getattr(L, name)
    assert {n for n, _, _ in qmv.SYMBOLS} == _declared()
    ours = [f for f in exported if "kore" in f]
    assert ours and all(f.startswith("kore_qmv_") for f in ours), ours


def test_header_constants_match_binding():
    from kore_amd import qmv
    text = open(HEADERS[0]).read()
    assert re.search(r"KORE_QMV_Q4_K\s*=\s*12", text) and qmv.KORE_QMV_Q4_K == 12
    assert re.search(r"KORE_QMV_Q6_K\s*=\s*14", text) and qmv.KORE_QMV_Q6_K == 14
    assert re.search(r"KORE_QMV_Q8K_BYTES\s+292", text) and qmv.Q8K_DTYPE.itemsize == 292


@pytest.mark.parametrize("wtype,rows,cols,code,fragment", [
    (0, 4, 256, -3, "Q4_K"),           # F32: kore's matvec_rows returns false
    (1, 4, 256, -3, "Q4_K"),           # F16
    (30, 4, 256, -3, "Q4_K"),          # BF16
    (12, 4, 300, -1, "multiple of 256"),
    (12, 0, 256, -1, "rows"),
    (14, 4, 256 * 129, -3, "32768"),
])
def test_create_rejects_what_kore_rejects(wtype, rows, cols, code, fragment):
    from kore_amd import qmv
    h = C.c_void_p()
    buf = np.zeros(16, np.uint8)
    rc = qmv.lib().kore_qmv_tensor_create(C.byref(h), wtype, rows, cols, buf.ctypes.data, 0)
    assert rc == code and not h.value
    assert fragment in qmv.lib().kore_qmv_last_error(None).decode()


def test_calls_without_a_tensor_fail_cleanly():
    from kore_amd import qmv
    L = qmv.lib()
    assert L.kore_qmv_matvec(None, None, None, 1) == qmv.KORE_QMV_E_INVALID
    assert L.kore_qmv_matvec_dev(None, None, None, 1, None) == qmv.KORE_QMV_E_INVALID
    assert L.kore_qmv_mv(None, None, None, 0) == qmv.KORE_QMV_E_INVALID
    assert L.kore_qmv_mv_dev(None, None, None, 0, None) == qmv.KORE_QMV_E_INVALID
    assert L.kore_qmv_mv_group_dev(0, None, None, None, 0, None) == qmv.KORE_QMV_E_INVALID
    assert L.kore_qmv_mv_group_dev(5, None, None, None, 0, None) == qmv.KORE_QMV_E_INVALID
    assert L.kore_qmv_get_info(None, None) == qmv.KORE_QMV_E_INVALID
    assert L.kore_qmv_matmul_batch(None, None, 1, None) == qmv.KORE_QMV_E_INVALID
    assert L.kore_qmv_matmul_batch_dev(None, None, 1, None, None) == qmv.KORE_QMV_E_INVALID
    assert L.kore_qmv_matmul_batch_group_dev(0, None, None, 1, None, None) == qmv.KORE_QMV_E_INVALID
    assert L.kore_qmv_mv_group_ex_dev(0, None, None, None, None, 1, None) == qmv.KORE_QMV_E_INVALID
    assert L.kore_qmv_matmul_batch_group_dev(5, None, None, 1, None, None) == qmv.KORE_QMV_E_INVALID
    assert L.kore_qmv_rmsnorm_rows_split_dev(None, None, 256, 1, 1e-6, None, None, None) == qmv.KORE_QMV_E_INVALID
    assert L.kore_qmv_matmul_batch_group_split_dev(1, None, None, 1, None, None, None) == qmv.KORE_QMV_E_INVALID
    assert L.kore_qmv_matmul_batch_glu_split_dev(None, None, 1, None, None, None) == qmv.KORE_QMV_E_INVALID
    # the fp16 split: 256-column blocks of 67,840 bytes (64 activations: hi and lo fp16,
    # the sub-block sums and 1 / scale), widths up to 4096 only
    assert L.kore_qmv_split_bytes(3584) == 14 * 67840
    assert L.kore_qmv_split_bytes(300) == 0 and L.kore_qmv_split_bytes(8192) == 0
    assert L.kore_qmv_last_error(None) is not None
    L.kore_qmv_tensor_destroy(None)
    x = np.zeros(300, np.float32)
    assert L.kore_qmv_quantize(x.ctypes.data, 300, x.ctypes.data) == qmv.KORE_QMV_E_INVALID
    assert L.kore_qmv_quantize_dev(x.ctypes.data, 255, x.ctypes.data, None) == qmv.KORE_QMV_E_INVALID
    assert L.kore_qmv_synth_dev(0, 1, 256, 1, x.ctypes.data, None) == qmv.KORE_QMV_E_UNSUPPORTED
    assert L.kore_qmv_synth_dev(12, 1, 255, 1, x.ctypes.data, None) == qmv.KORE_QMV_E_INVALID
    with pytest.raises(qmv.QmvError):
        qmv.quantize(np.zeros(100, np.float32))


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is present")
def test_create_without_gpu_is_a_hip_error():
    from kore_amd import qmv
    h = C.c_void_p()
    buf = np.zeros(144, np.uint8)
    rc = qmv.lib().kore_qmv_tensor_create(C.byref(h), 12, 1, 256, buf.ctypes.data, 0)
    assert rc == qmv.KORE_QMV_E_HIP and not h.value
