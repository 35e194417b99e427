"""CPU-side checks of the C ABI: the library loads, exports every function the
public headers declare, and rejects bad arguments with kore's error behaviour
before it touches a GPU."""
import ctypes as C
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("kore_attn.h", "kore_attn_synth.h")]


def _declared():
    names = set()
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(kore_attn_[a-z_]+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_headers_declare_the_abi():
    names = _declared()
    for fn in ("kore_attn_create", "kore_attn_destroy", "kore_attn_decode", "kore_attn_prefill",
               "kore_attn_read_kv", "kore_attn_last_error", "kore_attn_decode_dev",
               "kore_attn_prefill_dev", "kore_attn_append_dev", "kore_attn_sync", "kore_attn_get_info",
               "kore_attn_synth_dev", "kore_attn_decode_noalloc_dev"):
        assert fn in names


def test_library_exports_every_declared_symbol():
    from kore_amd import _lib
    L = _lib.lib()
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    for name in _declared():
        assert name in exported, f"{name} not exported"
        assert getattr(L, name)
    # the Python binding covers the same set
    assert {n for n, _, _ in _lib.SYMBOLS} == _declared()


def test_exports_are_c_abi_only():
    from kore_amd import _lib
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    funcs = [line.split()[-1] for line in out.splitlines() if " T " in line]
    ours = [f for f in funcs if "kore" in f]
    assert ours and all(f.startswith("kore_attn_") for f in ours), ours


def _create(*args):
    from kore_amd import _lib
    h = C.c_void_p()
    rc = _lib.lib().kore_attn_create(C.byref(h), *args)
    msg = _lib.lib().kore_attn_last_error(None).decode()
    return rc, h, msg


@pytest.mark.parametrize("args,fragment", [
    ((1, 16, 6, 4, 64, 1e6, 0), "multiple"),     # n_head % n_head_kv (kore.cpp:1278)
    ((1, 16, 4, 2, 63, 1e6, 0), "odd"),          # odd head_dim (kore.cpp:1288)
    ((0, 16, 4, 2, 64, 1e6, 0), "non-positive"),
    ((1, 0, 4, 2, 64, 1e6, 0), "non-positive"),
    ((1, 16, 4, 2, 64, 0.0, 0), "rope_base"),
    ((1, 16, 4, 2, 64, 1e6, 8), "window"),       # window must equal ctx
])
def test_create_rejects_bad_geometry(args, fragment):
    import kore_amd
    rc, h, msg = _create(*args)
    assert rc == kore_amd.KORE_ATTN_E_INVALID and not h.value
    assert fragment in msg


def test_create_reports_unsupported_geometry():
    """Every even head_dim up to 256 has a kernel; a larger one is refused
    before anything touches the device."""
    import kore_amd
    rc, h, msg = _create(1, 80, 4, 2, 258, 1e6, 0)
    assert rc == kore_amd.KORE_ATTN_E_UNSUPPORTED and "head_dim 258" in msg and not h.value


def test_null_handle_calls_fail_cleanly():
    import kore_amd
    from kore_amd import _lib
    L = _lib.lib()
    assert L.kore_attn_decode(None, 0, 0, 4, 2, 64, None, None, None, None) == kore_amd.KORE_ATTN_E_INVALID
    assert L.kore_attn_prefill(None, 0, 0, 1, 4, 2, 64, None, None, None, None) == kore_amd.KORE_ATTN_E_INVALID
    assert L.kore_attn_read_kv(None, 0, 0, 1, None, None) == kore_amd.KORE_ATTN_E_INVALID
    assert L.kore_attn_sync(None) == kore_amd.KORE_ATTN_E_INVALID
    assert L.kore_attn_append_dev(None, 0, 0, 1, None, None, None) == kore_amd.KORE_ATTN_E_INVALID
    assert L.kore_attn_last_error(None) is not None
    L.kore_attn_destroy(None)


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is present")
def test_create_without_gpu_is_a_hip_error():
    import kore_amd
    rc, h, msg = _create(1, 16, 4, 2, 64, 1e6, 0)
    assert rc == kore_amd.KORE_ATTN_E_HIP and not h.value and msg


def test_product_never_imports_the_oracle():
    """The product package has no reference to the test oracle."""
    pkg = os.path.join(ROOT, "kore_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert "import oracle" not in text and "liboracle" not in text, f
