"""CPU-side checks of the layer and loader C ABI (include/kore_layer.h,
kore_gguf.h): libkore_layer.so loads, exports exactly what the headers
declare, and rejects bad arguments before it touches a GPU."""
import os
import re
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("kore_layer.h", "kore_gguf.h", "kore_model.h")]


def _declared():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= {m.group(1) for m in re.finditer(r"\b(kore_(?:layer|gguf|model)_[a-z_0-9]+)\s*\(", text)}
    return names


def test_library_exports_exactly_the_declared_symbols():
    from kore_amd import layer
    layer.lib()
    out = subprocess.run(["nm", "-D", "--defined-only", layer.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert _declared() == exported
    assert {"kore_layer_decode_dev", "kore_layer_prefill_dev", "kore_model_prefill_dev", "kore_model_rows_dev",
            "kore_model_sync", "kore_gguf_open", "kore_gguf_to_qmv"} <= exported


def test_rejections_without_a_gpu():
    import ctypes as C

    from kore_amd import layer
    L = layer.lib()
    h = C.c_void_p()
    assert L.kore_layer_create(C.byref(h), 300, 512, 2, 1, 1e-6) == layer.KORE_LAYER_E_INVALID   # 300 % 256
    assert L.kore_layer_create(C.byref(h), 256, 512, 3, 2, 1e-6) == layer.KORE_LAYER_E_INVALID   # 3 % 2
    assert L.kore_layer_decode_dev(None, None, None, 0, 0, None, 1, None) == layer.KORE_LAYER_E_INVALID
    assert L.kore_layer_prefill_dev(None, None, None, 0, 0, 1, None, None) == layer.KORE_LAYER_E_INVALID
    assert b"NULL" in L.kore_layer_last_error(None)


def test_model_load_rejects_an_unknown_matvec_order():
    # kore's e.avx2 is 0 or 1; -1 asks for kore's own choice on this host
    import ctypes as C

    from kore_amd import model
    L = model.lib()
    h = C.c_void_p()
    path = os.path.join(ROOT, "tests", "golden", "gguf_tiny_qwen2.gguf").encode()
    for bad in (2, -2):
        assert L.kore_model_load_ex(path, 16, bad, C.byref(h)) == model.KORE_MODEL_E_LOAD and not h.value
        assert b"avx2" in L.kore_model_last_error(None)
