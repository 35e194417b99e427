"""GPU tests of the decode over the split counts it uses (1 .. 256 splits per
kv-head; the single-block split kernel at one and two workgroups per CU and
the multi-block split kernel; head_dim 64 and 128; 1 .. 8 q-heads per kv-head): kore_attn_decode_dev against the oracle
within 1e-4 of max|ref| and against kore_attn_decode_noalloc_dev (the same
kernels over the library's fixed array) bit for bit, the cache rows bit for
bit; many calls on one handle over a sliding ring; a captured 28-layer step
replayed three times against the eager decodes; two handles decoding on two
streams at once."""
import ctypes as C
import sys

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def _close(out, ref, what):
    ref = np.asarray(ref, np.float64)
    err = float(np.max(np.abs(np.asarray(out, np.float64) - ref)))
    assert err <= 1e-4 * float(np.max(np.abs(ref))), f"{what}: max|d| {err:.3e}"


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _fill(attn, rows, kvd, rng):
    from kore_amd import hip
    K = rng.standard_normal((rows, kvd)).astype(np.float32)
    V = rng.standard_normal((rows, kvd)).astype(np.float32)
    dk, dv = hip.DeviceBuffer.from_array(K), hip.DeviceBuffer.from_array(V)
    attn.append_dev(0, 0, rows, dk.ptr, dv.ptr)
    attn.sync()
    dk.free()
    dv.free()
    return K, V


@pytest.mark.parametrize("nh,nkv,hd,fill,steps", [
    (28, 4, 128, 4096, 3),     # Qwen2.5-7B: 64 splits of 64 rows
    (28, 4, 128, 40, 2),       # 2 splits
    (28, 4, 128, 560, 2),      # 35 splits
    (28, 4, 128, 8000, 2),     # 125 splits of 64 rows: two single-block workgroups per CU, then a
                               # last split of one row
    (28, 4, 128, 4421, 2),     # 127 splits of 35 rows (two blocks and three extra rows), two per CU
    (28, 4, 128, 9000, 2),     # 64 splits of 141 rows: the multi-block kernel
    (28, 4, 128, 12351, 2),    # multi-block, 193 rows per split: one extra row
    (16, 2, 128, 10623, 2),    # 8 q-heads per kv-head, multi-block, 83 rows per split: three extra rows
    (16, 2, 128, 12000, 2),    # 250 splits of 48 rows, two per CU: the combine's 32 splits per lane
    (14, 2, 64, 12000, 2),     # head_dim 64, two per CU (its registers would allow more: LDS-padded)
    (14, 2, 64, 20000, 2),     # head_dim 64, multi-block, one per CU (LDS-padded)
    (14, 2, 64, 511, 2),       # Qwen2.5-0.5B: 31 splits, head_dim 64
    (16, 2, 128, 1000, 2),     # 8 q-heads per kv-head
    (8, 8, 128, 2000, 2),      # 1 q-head per kv-head, 32 splits
    (12, 2, 128, 900, 2),      # 6 q-heads per kv-head, 56 splits
])
def test_decode_splits_vs_oracle_and_noalloc(nh, nkv, hd, fill, steps):
    from kore_amd import KoreAttn, hip
    E, kvd = nh * hd, nkv * hd
    _say(f"decode splits {nh}/{nkv}/{hd} fill {fill} steps {steps}")
    rng = np.random.default_rng(fill + nh)
    ctx = fill + steps + 1
    with KoreAttn(1, ctx, nh, nkv, hd, 1e6) as A, KoreAttn(1, ctx, nh, nkv, hd, 1e6) as B:
        seed_rng = np.random.default_rng(7)
        K, V = _fill(A, fill, kvd, seed_rng)
        _fill(B, fill, kvd, np.random.default_rng(7))
        kv = oracle.KV(1, ctx, nh, nkv, hd, 1e6)
        inv_f = oracle.inv_freq(hd, 1e6)
        kv.kcache()[0, :fill] = oracle.rope_rows(K, np.arange(fill), nkv, hd, inv_f)
        kv.vcache()[0, :fill] = V
        oa, ob = hip.DeviceBuffer(E), hip.DeviceBuffer(E)
        for pos in range(fill, fill + steps):
            q = rng.standard_normal(E).astype(np.float32) * 2
            k = rng.standard_normal(kvd).astype(np.float32)
            v = rng.standard_normal(kvd).astype(np.float32)
            dq, dk, dv = (hip.DeviceBuffer.from_array(x) for x in (q, k, v))
            A.decode_dev(0, pos, dq.ptr, dk.ptr, dv.ptr, oa.ptr)
            B.decode_noalloc_dev(0, pos, dq.ptr, dk.ptr, dv.ptr, ob.ptr)
            A.sync()
            B.sync()
            ra, rb = oa.download(), ob.download()
            assert np.array_equal(_bits(ra), _bits(rb)), f"position {pos}: decode_dev and decode_noalloc_dev differ"
            _close(ra, kv.decode(0, pos, q, k, v), f"position {pos} vs oracle")
            for b in (dq, dk, dv):
                b.free()
        ka, va = A.read_kv(0, 0, fill + steps)
        np.testing.assert_array_equal(ka, kv.kcache()[0, :fill + steps])
        np.testing.assert_array_equal(va, kv.vcache()[0, :fill + steps])
        oa.free()
        ob.free()
    kv.close()


def test_decode_many_calls_over_a_ring():
    """A 1.5B-shape ring of 1024 slots decoded 300 times past its end (the
    same split partials reused by every call) against the oracle's window
    decode."""
    from kore_amd import KoreAttn
    nh, nkv, hd, W = 12, 2, 128, 1024
    _say("decode: 300 ring decodes past the end")
    rng = np.random.default_rng(11)
    kv = oracle.KV(1, W, nh, nkv, hd, 1e6, window=W)
    with KoreAttn(1, W, nh, nkv, hd, 1e6, window=W) as A:
        for pos in range(W + 300):
            q = rng.standard_normal(nh * hd).astype(np.float32)
            k = rng.standard_normal(nkv * hd).astype(np.float32)
            v = rng.standard_normal(nkv * hd).astype(np.float32)
            out = A.decode(0, pos, q, k, v)
            ref = kv.decode(0, pos, q, k, v)
            if pos >= W - 200:
                _close(out, ref, f"ring position {pos}")
        kg, vg = A.read_kv(0, 0, W)
        np.testing.assert_array_equal(kg, kv.kcache()[0])
        np.testing.assert_array_equal(vg, kv.vcache()[0])
    kv.close()


def _graph_api():
    from kore_amd import hip
    h = hip.lib()
    vp = C.c_void_p
    h.hipStreamBeginCapture.argtypes = [vp, C.c_int]
    h.hipStreamEndCapture.argtypes = [vp, C.POINTER(vp)]
    h.hipGraphInstantiate.argtypes = [C.POINTER(vp), vp, vp, vp, C.c_size_t]
    h.hipGraphLaunch.argtypes = [vp, vp]
    h.hipGraphExecDestroy.argtypes = [vp]
    h.hipGraphDestroy.argtypes = [vp]
    return h


def test_captured_decodes_replay_the_eager_results():
    """A 28-layer 7B decode step captured on the handle's stream (no memset in
    the graph) and replayed three times, with eager decodes of the same step
    between the replays: every replay's outputs equal the eager ones bit for
    bit."""
    from kore_amd import KoreAttn, hip
    nl, nh, nkv, hd, fill = 28, 28, 4, 128, 2048
    E, kvd = nh * hd, nkv * hd
    _say("captured 28-layer decode step, 3 replays")
    h = _graph_api()
    rng = np.random.default_rng(5)
    with KoreAttn(nl, fill + 4, nh, nkv, hd, 1e6) as A:
        dk = hip.DeviceBuffer.from_array(rng.standard_normal((fill, kvd)).astype(np.float32))
        dv = hip.DeviceBuffer.from_array(rng.standard_normal((fill, kvd)).astype(np.float32))
        for l in range(nl):
            A.append_dev(l, 0, fill, dk.ptr, dv.ptr)
        A.sync()
        q = hip.DeviceBuffer.from_array(rng.standard_normal((nl, E)).astype(np.float32))
        k = hip.DeviceBuffer.from_array(rng.standard_normal((nl, kvd)).astype(np.float32))
        v = hip.DeviceBuffer.from_array(rng.standard_normal((nl, kvd)).astype(np.float32))
        eager, graphed = hip.DeviceBuffer(nl * E), hip.DeviceBuffer(nl * E)

        def step(out):
            for l in range(nl):
                A.decode_dev(l, fill, q.at(l * E), k.at(l * kvd), v.at(l * kvd), out.at(l * E))

        step(eager)
        A.sync()
        ref = eager.download()
        st = C.c_void_p(A.stream)
        graph, exe = C.c_void_p(), C.c_void_p()
        hip.check(h.hipStreamBeginCapture(st, 2), "hipStreamBeginCapture")   # relaxed mode
        step(graphed)
        hip.check(h.hipStreamEndCapture(st, C.byref(graph)), "hipStreamEndCapture")
        hip.check(h.hipGraphInstantiate(C.byref(exe), graph, None, None, 0), "hipGraphInstantiate")
        try:
            for rep in range(3):
                hip.check(h.hipGraphLaunch(exe, st), "hipGraphLaunch")
                A.sync()
                got = graphed.download()
                assert np.array_equal(_bits(got), _bits(ref)), f"replay {rep} differs from the eager decodes"
                step(eager)                # eager decodes between the replays
                A.sync()
                assert np.array_equal(_bits(eager.download()), _bits(ref)), f"eager step after replay {rep}"
        finally:
            h.hipGraphExecDestroy(exe)
            h.hipGraphDestroy(graph)
        for b in (dk, dv, q, k, v, eager, graphed):
            b.free()


def test_two_handles_on_two_streams_at_once():
    """Two handles (their own split partials) decoding 28 layers each on their
    own streams without a synchronisation between them: both equal their
    serial results bit for bit."""
    from kore_amd import KoreAttn, hip
    nl, nh, nkv, hd, fill = 28, 28, 4, 128, 3000
    E, kvd = nh * hd, nkv * hd
    _say("two handles decoding concurrently")
    rng = np.random.default_rng(9)
    hs = [KoreAttn(nl, fill + 2, nh, nkv, hd, 1e6) for _ in range(2)]
    try:
        bufs = []
        for A in hs:
            dk = hip.DeviceBuffer.from_array(rng.standard_normal((fill, kvd)).astype(np.float32))
            dv = hip.DeviceBuffer.from_array(rng.standard_normal((fill, kvd)).astype(np.float32))
            for l in range(nl):
                A.append_dev(l, 0, fill, dk.ptr, dv.ptr)
            A.sync()
            q = hip.DeviceBuffer.from_array(rng.standard_normal((nl, E)).astype(np.float32))
            k = hip.DeviceBuffer.from_array(rng.standard_normal((nl, kvd)).astype(np.float32))
            v = hip.DeviceBuffer.from_array(rng.standard_normal((nl, kvd)).astype(np.float32))
            bufs.append((dk, dv, q, k, v, hip.DeviceBuffer(nl * E)))

        def step(i):
            A, (_, _, q, k, v, out) = hs[i], bufs[i]
            for l in range(nl):
                A.decode_dev(l, fill, q.at(l * E), k.at(l * kvd), v.at(l * kvd), out.at(l * E))

        serial = []
        for i in range(2):
            step(i)
            hs[i].sync()
            serial.append(bufs[i][5].download())
        for _ in range(3):
            step(0)
            step(1)
            for i in range(2):
                hs[i].sync()
                assert np.array_equal(_bits(bufs[i][5].download()), _bits(serial[i])), f"handle {i} differs"
        for b in bufs:
            for x in b:
                x.free()
    finally:
        for A in hs:
            A.close()
