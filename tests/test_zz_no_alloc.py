"""GPU test of kore_attn_decode_noalloc_dev (the decode whose split partials
live in the library's fixed device array): through the C ABI, on two calls in
a row (the second attends fewer rows, so it uses fewer splits and a smaller
part of the array), its outputs and appended K/V rows must equal those of
kore_attn_decode_dev on the same inputs bit for bit - the same kernels run,
only the partials' address differs."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("nh,nkv,hd,fill,positions", [
    (28, 4, 128, 3000, (3000, 77)),     # Qwen2.5-7B geometry: 64 splits, then 4
    (28, 4, 128, 8190, (8190, 6000)),   # 128 splits of 64 rows (two workgroups per CU), then 125 of 48
    (16, 2, 128, 12000, (12000, 9000)), # 250 splits of 48 rows: 520,000 floats of the array, then 250 of 36
    (16, 2, 128, 4200, (4200, 1500)),   # 3B geometry: 128 splits of 33 rows, then 93 splits
    (14, 2, 64, 600, (600, 16)),        # 0.5B geometry, head_dim 64
    (32, 8, 40, 2000, (2000, 50)),      # head_dim 40: the generic kernels (roped q in the array too)
    (24, 2, 128, 3000, (3000, 100)),    # 12 q-heads per kv-head: generic decode
])
def test_noalloc_decode_equals_decode_dev(nh, nkv, hd, fill, positions):
    from kore_amd import KoreAttn, hip
    ctx = fill + 8
    E, kvd = nh * hd, nkv * hd
    rng = np.random.default_rng(nh * 31 + fill)
    _say(f"noalloc decode {nh}/{nkv}/{hd} fill {fill} positions {positions}")
    K0 = rng.standard_normal((fill, kvd)).astype(np.float32)
    V0 = rng.standard_normal((fill, kvd)).astype(np.float32)
    with KoreAttn(1, ctx, nh, nkv, hd, 1e6) as A, KoreAttn(1, ctx, nh, nkv, hd, 1e6) as B:
        dk, dv = hip.DeviceBuffer.from_array(K0), hip.DeviceBuffer.from_array(V0)
        A.append_dev(0, 0, fill, dk.ptr, dv.ptr)
        B.append_dev(0, 0, fill, dk.ptr, dv.ptr)
        A.sync()
        B.sync()
        oa, ob = hip.DeviceBuffer(E), hip.DeviceBuffer(E)
        for pos in positions:
            q = rng.standard_normal(E).astype(np.float32) * 2
            k = rng.standard_normal(kvd).astype(np.float32)
            v = rng.standard_normal(kvd).astype(np.float32)
            dq, dk1, dv1 = (hip.DeviceBuffer.from_array(x) for x in (q, k, v))
            A.decode_dev(0, pos, dq.ptr, dk1.ptr, dv1.ptr, oa.ptr)
            B.decode_noalloc_dev(0, pos, dq.ptr, dk1.ptr, dv1.ptr, ob.ptr)
            A.sync()
            B.sync()
            ra, rb = oa.download(), ob.download()
            assert np.all(np.isfinite(ra))
            np.testing.assert_array_equal(ra.view(np.uint32), rb.view(np.uint32),
                                          err_msg=f"position {pos}: outputs differ")
            ka, va = A.read_kv(0, pos, 1)
            kb, vb = B.read_kv(0, pos, 1)
            np.testing.assert_array_equal(ka, kb)
            np.testing.assert_array_equal(va, vb)
            for b in (dq, dk1, dv1):
                b.free()
        for b in (dk, dv, oa, ob):
            b.free()
