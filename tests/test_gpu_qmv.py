"""GPU parity of the quantised matvec (libkore_qmv.so) through its C ABI.

Bar: bit-identical to kore.  The Q8_K blocks must equal kore's
quantize_row_q8_K byte for byte and every row result must equal kore's
dot_q*_K_q8_K_avx2 (avx2=1) or dot_q*_K_q8_K_ref (avx2=0) bit for bit: on
kore's own golden outputs (tests/golden/qmv_*.npz), against the oracle (the
C restatement pinned to those outputs) on random shapes that exercise every
workgroup layout and tail, and on the full Qwen2.5-7B matrix shapes.  Every
test names its case before it touches the GPU.
"""
import ctypes as C
import json
import os
import sys

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = sorted(f[4:-5] for f in os.listdir(GOLD) if f.startswith("qmv_") and f.endswith(".json"))


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _assert_bits(out, ref, what):
    bad = np.flatnonzero(_bits(out) != _bits(ref))
    assert bad.size == 0, (f"{what}: {bad.size} rows differ, first row {bad[0]}: "
                           f"{out[bad[0]]!r} vs kore {ref[bad[0]]!r}")


def _weights(wtype, rows, nblk, rng):
    """Random blocks with finite f16 scales, some of them subnormal, zero or
    negative."""
    bb = oracle.BLOCK_BYTES[wtype]
    w = rng.integers(0, 256, size=(rows, nblk, bb), dtype=np.uint8)
    d = np.abs(rng.standard_normal((rows, nblk))) * 3e-3
    d[rng.random((rows, nblk)) < 0.05] *= -1.0
    d[rng.random((rows, nblk)) < 0.03] = 3e-6                  # f16 subnormal
    d[rng.random((rows, nblk)) < 0.02] = 0.0
    db = d.astype(np.float16).view(np.uint8).reshape(rows, nblk, 2)
    if wtype == oracle.TYPE_Q4K:
        w[:, :, 0:2] = db
        w[:, :, 2:4] = (np.abs(rng.standard_normal((rows, nblk))) * 1e-3).astype(np.float16).view(
            np.uint8).reshape(rows, nblk, 2)
    else:
        w[:, :, 208:210] = db
    return w.reshape(-1)


def _x(cols, rng):
    x = rng.standard_normal(cols).astype(np.float32)
    x[rng.random(cols) < 0.01] *= 20.0
    return x


# ---------------------------------------------------------------- golden

@pytest.mark.parametrize("name", FIXTURES)
def test_golden_replay(name):
    from kore_amd import qmv
    man = json.load(open(os.path.join(GOLD, f"qmv_{name}.json")))
    z = np.load(os.path.join(GOLD, f"qmv_{name}.npz"))
    _say(f"qmv golden {name}: type {man['type']}, {man['rows']} x {man['cols']}")
    xq = qmv.quantize(z["x"])
    assert xq.view(np.uint8).tobytes() == z["xq"].tobytes(), "Q8_K blocks differ from kore's"
    kore_xq = np.frombuffer(z["xq"].tobytes(), qmv.Q8K_DTYPE)
    with qmv.QMat(man["type"], man["rows"], man["cols"], z["weights"]) as w:
        _assert_bits(w.matvec(kore_xq, avx2=True), z["out_avx2"], f"{name} avx2")
        _assert_bits(w.matvec(kore_xq, avx2=False), z["out_ref"], f"{name} scalar")
        _assert_bits(w.mv(z["x"], avx2=True), z["out_avx2"], f"{name} mv avx2")
        _assert_bits(w.mv(z["x"], avx2=False), z["out_ref"], f"{name} mv scalar")


# ---------------------------------------------------------------- random shapes

SHAPES = [(1, 1), (37, 3), (129, 14), (64, 74), (21, 128), (300, 17), (16, 16)]


@pytest.mark.parametrize("wgs", ["0", "1"])
@pytest.mark.parametrize("rpw", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("wtype", [oracle.TYPE_Q4K, oracle.TYPE_Q6K])
def test_random_shapes_vs_oracle(wtype, rpw, wgs, monkeypatch):
    """Every wave layout (rows per wave), one tile per workgroup or long
    runs of tiles per workgroup (one workgroup per CU)."""
    from kore_amd import qmv
    monkeypatch.setenv("KORE_QMV_ROWS_PER_WAVE", str(rpw))
    monkeypatch.setenv("KORE_QMV_WGS_PER_CU", wgs)
    for si, (rows, nblk) in enumerate(SHAPES):
        _say(f"qmv random type {wtype} rows_per_wave {rpw} wgs/cu {wgs}: {rows} x {nblk * 256}")
        rng = np.random.default_rng(1000 * wtype + 10 * rpw + si)
        w = _weights(wtype, rows, nblk, rng)
        x = _x(nblk * 256, rng)
        xq = oracle.quantize_q8K(x)
        with qmv.QMat(wtype, rows, nblk * 256, w) as m:
            assert m.info().rows_per_wave == rpw
            for avx2 in (True, False):
                ref = oracle.qmatvec(wtype, w, rows, nblk * 256, xq, avx2=avx2)
                _assert_bits(m.matvec(xq, avx2=avx2), ref, f"{rows}x{nblk} avx2={avx2}")


# ---------------------------------------------------------------- quantiser

def test_quantize_edge_cases():
    from kore_amd import qmv
    _say("qmv quantize edge cases")
    rng = np.random.default_rng(77)
    blocks = []
    blocks.append(np.zeros(256))                                   # zero block
    blocks.append(np.full(256, 0.3))                               # constant
    b = rng.standard_normal(256); b[10], b[99] = -5.0, 5.0; blocks.append(b)    # tie: first wins
    b = rng.standard_normal(256); b[10], b[99] = 5.0, -5.0; blocks.append(b)
    blocks.append(rng.standard_normal(256) * 1e-39)                # subnormal inputs
    b = rng.standard_normal(256) * 1e-41; b[3] = 1e-39; blocks.append(b)  # -127/max overflows: x86 int path
    blocks.append(rng.standard_normal(256) * 3e38)                 # near FLT_MAX
    b = rng.standard_normal(256); b[7] = np.nan; blocks.append(b)  # NaN never wins
    b = rng.standard_normal(256); b[8] = np.inf; blocks.append(b)  # inf wins: iscale -0
    b = np.round(rng.standard_normal(256) * 16) / 16; b[0] = -127 / 16; blocks.append(b)  # halves
    b = rng.standard_normal(256); b[:128] = -0.0; blocks.append(b)
    # the largest magnitude twice inside one 16-value group, opposite signs: the first wins
    b = rng.standard_normal(256); b[3], b[7] = -6.0, 6.0; blocks.append(b)
    b = rng.standard_normal(256); b[3], b[7] = 6.0, -6.0; blocks.append(b)
    b = rng.standard_normal(256); b[255] = -7.0; blocks.append(b)              # the last value
    b = rng.standard_normal(256); b[40], b[200] = -np.inf, np.inf; blocks.append(b)   # -inf first: d = +inf
    b = rng.standard_normal(256); b[40], b[200] = np.inf, -np.inf; blocks.append(b)
    b = rng.standard_normal(256); b[16], b[17] = np.nan, 9.0; blocks.append(b)  # NaN beside the maximum
    blocks.append(np.full(256, np.nan))                                        # all NaN: a zero block
    b = np.zeros(256); b[::2] = -0.0; blocks.append(b)                         # signed zeros only
    x = np.concatenate(blocks).astype(np.float32)
    with np.errstate(all="ignore"):
        ref = oracle.quantize_q8K(x)
    got = qmv.quantize(x)
    for i in range(len(blocks)):
        assert got[i].tobytes() == ref[i].tobytes(), f"block {i} differs from kore's quantiser"


def test_quantize_many_random_blocks():
    from kore_amd import qmv
    _say("qmv quantize 4096 random blocks")
    rng = np.random.default_rng(78)
    x = (rng.standard_normal(4096 * 256) * np.repeat(10.0 ** rng.uniform(-6, 6, 4096), 256)).astype(np.float32)
    assert qmv.quantize(x).tobytes() == oracle.quantize_q8K(x).tobytes()


# ---------------------------------------------------------------- device API

def test_device_api_matches_host_api():
    from kore_amd import hip, qmv
    _say("qmv device-pointer API, Q6_K 200 x 4608")
    rng = np.random.default_rng(79)
    rows, cols = 200, 4608
    w = _weights(oracle.TYPE_Q6K, rows, cols // 256, rng)
    x = _x(cols, rng)
    dx = hip.DeviceBuffer.from_array(x)
    dq = hip.DeviceBuffer((cols // 256 * 292 + 3) // 4)
    do = hip.DeviceBuffer(rows)
    # the tensor from a device copy of the raw blocks
    draw = hip.DeviceBuffer((w.size + 3) // 4)
    hip.check(hip.lib().hipMemcpy(draw.ptr, w.ctypes.data, w.size, hip.H2D), "upload")
    with qmv.QMat(oracle.TYPE_Q6K, rows, cols, device_ptr=draw.ptr) as m:
        qmv.quantize_dev(dx.ptr, cols, dq.ptr)
        for avx2 in (True, False):
            m.matvec_dev(dq.ptr, do.ptr, avx2=avx2)
            hip.synchronize()
            _assert_bits(do.download(), m.mv(x, avx2=avx2), f"dev vs host avx2={avx2}")
        # misaligned activations are refused before any launch
        with pytest.raises(qmv.QmvError) as e:
            m.matvec_dev(dq.ptr + 4, do.ptr)
        assert e.value.code == qmv.KORE_QMV_E_INVALID
    for b in (dx, dq, do, draw):
        b.free()


@pytest.mark.parametrize("fuse", ["0", "1"])
def test_grouped_and_fused_launches(fuse, monkeypatch):
    """kore's q/k/v (and gate/up) matvecs share one quant(): one grouped launch,
    with the quantisation inside it (fuse 1) or apart (fuse 0), gives kore's
    bits for every matrix of the group."""
    from kore_amd import hip, qmv
    monkeypatch.setenv("KORE_QMV_FUSE", fuse)
    groups = [
        [(oracle.TYPE_Q4K, 300), (oracle.TYPE_Q4K, 64), (oracle.TYPE_Q6K, 64)],      # q, k, v
        [(oracle.TYPE_Q4K, 1000), (oracle.TYPE_Q4K, 1000)],                         # gate, up
        [(oracle.TYPE_Q6K, 77), (oracle.TYPE_Q4K, 5), (oracle.TYPE_Q6K, 130), (oracle.TYPE_Q4K, 16)],
    ]
    for gi, (group, nblk) in enumerate(zip(groups, (14, 14, 74))):
        for extra in ((), (128,)) if gi == 2 else ((),):
            nb = extra[0] if extra else nblk
            cols = nb * 256
            _say(f"qmv group {gi} fuse {fuse}: {[(t, r) for t, r in group]} x {cols}")
            rng = np.random.default_rng(300 + gi + nb)
            ws = [_weights(t, r, nb, rng) for t, r in group]
            x = _x(cols, rng)
            xq = oracle.quantize_q8K(x)
            mats = [qmv.QMat(t, r, cols, w) for (t, r), w in zip(group, ws)]
            dx = hip.DeviceBuffer.from_array(x)
            douts = [hip.DeviceBuffer(r) for _, r in group]
            for avx2 in (True, False):
                qmv.mv_group_dev(mats, dx.ptr, [d.ptr for d in douts], avx2=avx2)
                hip.synchronize()
                for (t, r), w, d in zip(group, ws, douts):
                    _assert_bits(d.download(), oracle.qmatvec(t, w, r, cols, xq, avx2=avx2),
                                 f"group {gi} type {t} rows {r} avx2={avx2}")
                mats[0].mv_dev(dx.ptr, douts[0].ptr, avx2=avx2)
                hip.synchronize()
                t, r = group[0]
                _assert_bits(douts[0].download(), oracle.qmatvec(t, ws[0], r, cols, xq, avx2=avx2), "mv_dev")
            for m in mats:
                m.close()
            for d in douts + [dx]:
                d.free()


def _splitmix64(z):
    z = (z + np.uint64(0x9E3779B97F4A7C15)).astype(np.uint64)
    z = ((z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)).astype(np.uint64)
    z = ((z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)).astype(np.uint64)
    return z ^ (z >> np.uint64(31))


def test_synth_matches_its_definition():
    from kore_amd import hip, qmv
    for wtype, rows, cols, seed in ((oracle.TYPE_Q4K, 3, 512, 5), (oracle.TYPE_Q6K, 5, 768, 6)):
        _say(f"qmv synth type {wtype} {rows} x {cols}")
        nbytes = rows * cols // 256 * oracle.BLOCK_BYTES[wtype]
        buf = hip.DeviceBuffer((nbytes + 3) // 4)
        qmv.synth_dev(wtype, rows, cols, seed, buf.ptr)
        hip.synchronize()
        got = np.zeros(nbytes, np.uint8)
        hip.check(hip.lib().hipMemcpy(got.ctypes.data, buf.ptr, nbytes, hip.D2H), "download")
        buf.free()
        with np.errstate(over="ignore"):
            key = _splitmix64(np.array([seed], np.uint64))[0]
            h = _splitmix64(key ^ np.arange(nbytes // 2, dtype=np.uint64)).astype(np.uint64)
        words = (h & np.uint64(0xFFFF)).astype(np.uint16)
        wpb = oracle.BLOCK_BYTES[wtype] // 2
        wi = np.arange(nbytes // 2) % wpb
        low = (h & np.uint64(0x3FF)).astype(np.uint16)
        if wtype == oracle.TYPE_Q4K:
            words = np.where(wi == 0, 0x1C00 | low, np.where(wi == 1, 0x1800 | low, words))
        else:
            words = np.where(wi == 104, 0x1C00 | low, words)
        assert np.array_equal(got.view(np.uint16), words.astype(np.uint16))


# ---------------------------------------------------------------- 7B shapes

# Qwen2.5-7B: n_embd 3584, n_ff 18944, 4 kv-heads x 128, vocab 152064
SHAPES_7B = [
    ("attn_q", oracle.TYPE_Q4K, 3584, 3584),
    ("attn_k", oracle.TYPE_Q4K, 512, 3584),
    ("attn_v", oracle.TYPE_Q6K, 512, 3584),
    ("attn_output", oracle.TYPE_Q4K, 3584, 3584),
    ("ffn_gate", oracle.TYPE_Q4K, 18944, 3584),
    ("ffn_down", oracle.TYPE_Q6K, 3584, 18944),
    ("ffn_down_q4k", oracle.TYPE_Q4K, 3584, 18944),
    ("output", oracle.TYPE_Q6K, 152064, 3584),
]


@pytest.mark.parametrize("name,wtype,rows,cols", SHAPES_7B)
def test_7b_matrix_every_row_bitwise(name, wtype, rows, cols):
    from kore_amd import hip, qmv
    _say(f"qmv 7B {name}: type {wtype}, {rows} x {cols}")
    nbytes = rows * cols // 256 * oracle.BLOCK_BYTES[wtype]
    raw = hip.DeviceBuffer((nbytes + 3) // 4)
    qmv.synth_dev(wtype, rows, cols, 4242 + rows, raw.ptr)
    hip.synchronize()
    w = np.zeros(nbytes, np.uint8)
    hip.check(hip.lib().hipMemcpy(w.ctypes.data, raw.ptr, nbytes, hip.D2H), "download")
    x = _x(cols, np.random.default_rng(rows + cols))
    with qmv.QMat(wtype, rows, cols, device_ptr=raw.ptr) as m:
        raw.free()
        xq = qmv.quantize(x)
        ref_xq = oracle.quantize_q8K(x)
        assert xq.tobytes() == ref_xq.tobytes()
        for avx2 in (True, False):
            _assert_bits(m.matvec(xq, avx2=avx2), oracle.qmatvec(wtype, w, rows, cols, ref_xq, avx2=avx2),
                         f"{name} avx2={avx2}")


def test_repeated_calls_are_identical():
    from kore_amd import qmv
    _say("qmv repeated calls, Q4_K 1000 x 3584")
    rng = np.random.default_rng(80)
    w = _weights(oracle.TYPE_Q4K, 1000, 14, rng)
    x = _x(3584, rng)
    with qmv.QMat(oracle.TYPE_Q4K, 1000, 3584, w) as m:
        first = m.mv(x)
        for _ in range(5):
            assert np.array_equal(_bits(m.mv(x)), _bits(first))


# ---------------------------------------------------------------- batched matmul

QMM = sorted(f[4:-5] for f in os.listdir(GOLD) if f.startswith("qmm_") and f.endswith(".json"))


def _close_kore(out, ref, what):
    """kore's own comparison (kore_kernels.cpp:742): max|d| <= 1e-4 * max|ref| + 1e-6."""
    out = np.asarray(out, np.float64).reshape(-1)
    ref = np.asarray(ref, np.float64).reshape(-1)
    err = float(np.max(np.abs(out - ref)))
    bound = 1e-4 * float(np.max(np.abs(ref))) + 1e-6
    assert err <= bound, f"{what}: max|d| {err:.3e} > {bound:.3e}"


@pytest.mark.parametrize("name", QMM)
def test_matmul_batch_golden(name):
    from kore_amd import qmv
    man = json.load(open(os.path.join(GOLD, f"qmm_{name}.json")))
    z = np.load(os.path.join(GOLD, f"qmm_{name}.npz"))
    _say(f"qmm golden {name}: type {man['type']}, {man['rows']} x {man['cols']}, B {man['B']}")
    with qmv.QMat(man["type"], man["rows"], man["cols"], z["weights"]) as m:
        out = m.matmul_batch(z["x"])
    _close_kore(out, z["out_avx2"], f"{name} vs kore avx2")
    _close_kore(out, z["out_ref"], f"{name} vs kore scalar")


GEMM_SHAPES = [  # type, rows, nblk, B
    (oracle.TYPE_Q4K, 1, 1, 1), (oracle.TYPE_Q6K, 100, 3, 17), (oracle.TYPE_Q4K, 257, 2, 16),
    (oracle.TYPE_Q4K, 3584, 14, 64), (oracle.TYPE_Q6K, 200, 74, 33), (oracle.TYPE_Q6K, 65, 14, 48),
    (oracle.TYPE_Q4K, 130, 128, 5),
    (oracle.TYPE_Q6K, 64, 74, 64),     # one tile whose 74 blocks are split among 37 workgroups
    (oracle.TYPE_Q4K, 5000, 3, 20),    # 79 tiles of 3 blocks
    (oracle.TYPE_Q4K, 64, 1, 64),      # a single iteration
]


@pytest.mark.parametrize("wtype,rows,nblk,B", GEMM_SHAPES)
def test_matmul_batch_vs_oracle(wtype, rows, nblk, B):
    from kore_amd import qmv
    _say(f"qmm random type {wtype}: {rows} x {nblk * 256}, B {B}")
    rng = np.random.default_rng(rows * 7 + nblk * 3 + B)
    w = _weights(wtype, rows, nblk, rng)
    x = np.stack([_x(nblk * 256, rng) for _ in range(B)])
    with qmv.QMat(wtype, rows, nblk * 256, w) as m:
        out = m.matmul_batch(x)
        again = m.matmul_batch(x)
    assert np.array_equal(_bits(out), _bits(again)), "repeated calls differ"
    _close_kore(out, oracle.matmul_batch(wtype, w, rows, nblk * 256, x, avx2=True), "vs oracle")


@pytest.mark.parametrize("wtype,B", [(oracle.TYPE_Q4K, 40), (oracle.TYPE_Q6K, 20)])
def test_matmul_batch_activation_ranges(wtype, B):
    """Activations of very different magnitudes per row (10^-20 .. 10^20, an
    all-zero row, a row whose values span 16 orders of magnitude): the
    batched matmul scales each activation by its own power of two, so every
    row is held to kore's tolerance against its own maximum."""
    from kore_amd import qmv
    rows, nblk = 300, 14
    _say(f"qmm activation ranges type {wtype}, B {B}")
    rng = np.random.default_rng(97 + B)
    w = _weights(wtype, rows, nblk, rng)
    x = np.stack([_x(nblk * 256, rng) for _ in range(B)])
    x *= (10.0 ** rng.integers(-20, 21, size=B)).astype(np.float32)[:, None]
    x[1] = 0.0
    x[2, ::2] *= 1e-16
    x = x.astype(np.float32)
    with qmv.QMat(wtype, rows, nblk * 256, w) as m:
        out = m.matmul_batch(x)
    ref = oracle.matmul_batch(wtype, w, rows, nblk * 256, x, avx2=True)
    assert np.all(out[1] == 0.0)
    for b in range(B):
        if b != 1:
            _close_kore(out[b] / np.float64(np.max(np.abs(ref[b]))), ref[b] / np.float64(np.max(np.abs(ref[b]))),
                        f"activation {b} (scale {np.max(np.abs(x[b])):.1e})")


@pytest.mark.parametrize("wtype", [oracle.TYPE_Q4K, oracle.TYPE_Q6K])
def test_matmul_batch_tiny_and_nonfinite_rows(wtype):
    """Activations whose maximum is a subnormal or barely normal float (2^-118,
    2^-130, 2^-145), and rows holding +inf, -inf or NaN, next to an ordinary
    row.  Tiny rows: kore's fp32 chain itself runs on the subnormal grid
    there (quantum 2^-149 per rounding), so each output is held to the exact
    float64 product within 1e-4 of the row's maximum plus 64 quanta, and to
    kore's own tolerance against kore.  Non-finite rows: every output is
    non-finite, as every one of kore's is; the ordinary row is unaffected."""
    from kore_amd import qmv
    rows, nblk, B = 200, 14, 7
    cols = nblk * 256
    _say(f"qmm tiny and non-finite rows type {wtype}")
    rng = np.random.default_rng(4242 + wtype)
    w = _weights(wtype, rows, nblk, rng)
    x = np.stack([_x(cols, rng) for _ in range(B)]).astype(np.float64)
    for b, e in ((1, -118), (2, -130), (3, -145)):
        x[b] = x[b] / np.max(np.abs(x[b])) * 2.0 ** e
    x = x.astype(np.float32)
    x[4, 17] = np.inf
    x[5, 1000] = -np.inf
    x[6, 3] = np.nan
    assert np.max(np.abs(x[3])) > 0 and np.max(np.abs(x[3])) < 2.0 ** -126   # a subnormal maximum
    with qmv.QMat(wtype, rows, cols, w) as m:
        out = m.matmul_batch(x)
    ref = oracle.matmul_batch(wtype, w, rows, cols, x, avx2=True)
    deq = np.stack([oracle.dequant_row(wtype, w[r * nblk * oracle.BLOCK_BYTES[wtype]:
                                                 (r + 1) * nblk * oracle.BLOCK_BYTES[wtype]], cols)
                    for r in range(rows)]).astype(np.float64)
    _close_kore(out[0], ref[0], "ordinary row vs kore")
    quantum = 2.0 ** -149
    for b in (1, 2, 3):
        exact = deq @ x[b].astype(np.float64)
        err = float(np.max(np.abs(out[b] - exact)))
        bound = 1e-4 * float(np.max(np.abs(exact))) + 64 * quantum
        assert np.max(np.abs(out[b])) > 0, f"tiny row {b}: all-zero outputs"
        assert err <= bound, f"tiny row {b} (max |x| {np.max(np.abs(x[b])):.2e}): |d| {err:.3e} > {bound:.3e}"
        _close_kore(out[b], ref[b], f"tiny row {b} vs kore")
    for b in (4, 5, 6):
        assert not np.any(np.isfinite(ref[b])), f"kore's row {b} has finite outputs"
        assert not np.any(np.isfinite(out[b])), f"row {b}: finite outputs where kore's are not"


def test_split_matmul_refuses_cols_without_a_split():
    """A caller's split holds kore_qmv_split_bytes(cols) bytes: a tensor whose
    cols have none (ffn_down's 18944) is refused before anything launches."""
    from kore_amd import hip, qmv
    _say("qmm split refusal for 18944 cols")
    rng = np.random.default_rng(5)
    cols = 18944
    m = qmv.QMat(oracle.TYPE_Q4K, 8, cols, _weights(oracle.TYPE_Q4K, 8, cols // 256, rng))
    try:
        assert qmv.split_bytes(cols) == 0
        x16, do = hip.DeviceBuffer(qmv.split_bytes(3584) // 4), hip.DeviceBuffer(64 * 8)
        with pytest.raises(qmv.QmvError) as e:
            qmv.matmul_batch_group_split_dev([m], x16.ptr, 4, [do.ptr])
        assert e.value.code == qmv.KORE_QMV_E_UNSUPPORTED
        hip.synchronize()
        x16.free()
        do.free()
    finally:
        m.close()


def _fp32_path_cases():
    """Run in a child process started with KORE_GEMM=fp32 (the fp32 matmul
    kernel; the variable is read once per process)."""
    from kore_amd import qmv
    assert qmv.split_bytes(3584) == 0, "KORE_GEMM=fp32 did not select the fp32 path"
    for wtype, rows, nblk, B in [(oracle.TYPE_Q4K, 257, 2, 16), (oracle.TYPE_Q6K, 200, 74, 33),
                                 (oracle.TYPE_Q4K, 3584, 14, 64), (oracle.TYPE_Q6K, 64, 74, 64)]:
        print(f"[gpu-case] fp32 path type {wtype}: {rows} x {nblk * 256}, B {B}", flush=True)
        rng = np.random.default_rng(rows + nblk + B)
        w = _weights(wtype, rows, nblk, rng)
        x = np.stack([_x(nblk * 256, rng) for _ in range(B)])
        with qmv.QMat(wtype, rows, nblk * 256, w) as m:
            out = m.matmul_batch(x)
            again = m.matmul_batch(x)
        assert np.array_equal(_bits(out), _bits(again)), "repeated calls differ"
        _close_kore(out, oracle.matmul_batch(wtype, w, rows, nblk * 256, x, avx2=True), "fp32 path vs oracle")
    print("FP32_PATH_OK", flush=True)


def test_matmul_batch_fp32_path_in_a_fresh_process():
    import subprocess
    _say("qmm fp32 path (KORE_GEMM=fp32) in a child process")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, KORE_GEMM="fp32")
    r = subprocess.run([sys.executable, "-c", "import tests.test_gpu_qmv as t; t._fp32_path_cases()"], cwd=root,
                       env=env, capture_output=True, text=True, timeout=110)
    assert r.returncode == 0 and "FP32_PATH_OK" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]


def test_matmul_batch_device_api_and_rejections():
    from kore_amd import hip, qmv
    _say("qmm device API, Q4_K 600 x 2048, B 40")
    rng = np.random.default_rng(91)
    rows, cols, B = 600, 2048, 40
    w = _weights(oracle.TYPE_Q4K, rows, cols // 256, rng)
    x = np.stack([_x(cols, rng) for _ in range(B)])
    with qmv.QMat(oracle.TYPE_Q4K, rows, cols, w) as m:
        dx = hip.DeviceBuffer.from_array(x)
        do = hip.DeviceBuffer(B * rows)
        m.matmul_batch_dev(dx.ptr, B, do.ptr)
        hip.synchronize()
        assert np.array_equal(_bits(do.download()), _bits(m.matmul_batch(x).reshape(-1)))
        for nb in (0, 65):
            with pytest.raises(qmv.QmvError) as e:
                m.matmul_batch_dev(dx.ptr, nb, do.ptr)
            assert e.value.code == qmv.KORE_QMV_E_INVALID
        dx.free()
        do.free()


@pytest.mark.parametrize("name,wtype,rows,cols", [("attn_q", oracle.TYPE_Q4K, 3584, 3584),
                                                  ("ffn_gate", oracle.TYPE_Q4K, 18944, 3584),
                                                  ("ffn_down", oracle.TYPE_Q6K, 3584, 18944)])
def test_matmul_batch_7b_shapes(name, wtype, rows, cols):
    """Full Qwen2.5-7B matrices, 64 activations; 192 sampled rows against the
    oracle (its cost on the CPU is the bound here)."""
    from kore_amd import hip, qmv
    _say(f"qmm 7B {name}: type {wtype}, {rows} x {cols}, B 64")
    nbytes = rows * cols // 256 * oracle.BLOCK_BYTES[wtype]
    raw = hip.DeviceBuffer((nbytes + 3) // 4)
    qmv.synth_dev(wtype, rows, cols, 777 + rows, raw.ptr)
    hip.synchronize()
    w = np.zeros(nbytes, np.uint8)
    hip.check(hip.lib().hipMemcpy(w.ctypes.data, raw.ptr, nbytes, hip.D2H), "download")
    rng = np.random.default_rng(cols)
    x = np.stack([_x(cols, rng) for _ in range(64)])
    with qmv.QMat(wtype, rows, cols, device_ptr=raw.ptr) as m:
        raw.free()
        out = m.matmul_batch(x)
    rb = cols // 256 * oracle.BLOCK_BYTES[wtype]
    pick = np.sort(rng.choice(rows, 192, replace=False))
    wsub = np.concatenate([w[r * rb:(r + 1) * rb] for r in pick])
    ref = oracle.matmul_batch(wtype, wsub, len(pick), cols, x, avx2=True)
    _close_kore(out[:, pick], ref, name)


@pytest.mark.parametrize("shapes,B", [
    ([(oracle.TYPE_Q4K, 300), (oracle.TYPE_Q4K, 64), (oracle.TYPE_Q6K, 65)], 37),   # q, k, v with v in Q6_K
    ([(oracle.TYPE_Q4K, 700), (oracle.TYPE_Q4K, 700)], 64),                          # gate, up
    ([(oracle.TYPE_Q6K, 17), (oracle.TYPE_Q4K, 1), (oracle.TYPE_Q6K, 129), (oracle.TYPE_Q4K, 64)], 16),
])
def test_matmul_batch_group(shapes, B):
    """One grouped launch: every output within kore's tolerance of the oracle
    and of the matrix's own single launch."""
    from kore_amd import hip, qmv
    cols = 2048
    _say(f"qmm group {shapes}, cols {cols}, B {B}")
    rng = np.random.default_rng(len(shapes) * 100 + B)
    ws = [_weights(t, r, cols // 256, rng) for t, r in shapes]
    x = np.stack([_x(cols, rng) for _ in range(B)])
    mats = [qmv.QMat(t, r, cols, w) for (t, r), w in zip(shapes, ws)]
    try:
        dx = hip.DeviceBuffer.from_array(x)
        outs = [hip.DeviceBuffer(B * r) for _, r in shapes]
        for rep in range(2):
            qmv.matmul_batch_group_dev(mats, dx.ptr, B, [o.ptr for o in outs])
            hip.synchronize()
            got = [o.download().reshape(B, r) for o, (_, r) in zip(outs, shapes)]
            if rep == 0:
                first = [g.copy() for g in got]
            else:
                for g0, g1 in zip(first, got):
                    assert np.array_equal(_bits(g0), _bits(g1)), "repeated grouped calls differ"
        for k, ((t, r), w) in enumerate(zip(shapes, ws)):
            _close_kore(got[k], oracle.matmul_batch(t, w, r, cols, x, avx2=True), f"group member {k} vs oracle")
            _close_kore(got[k], mats[k].matmul_batch(x), f"group member {k} vs its single launch")
        dx.free()
        for o in outs:
            o.free()
    finally:
        for m in mats:
            m.close()


def test_matmul_batch_group_rejections():
    from kore_amd import hip, qmv
    rng = np.random.default_rng(3)
    a = qmv.QMat(oracle.TYPE_Q4K, 64, 512, _weights(oracle.TYPE_Q4K, 64, 2, rng))
    b = qmv.QMat(oracle.TYPE_Q4K, 64, 768, _weights(oracle.TYPE_Q4K, 64, 3, rng))
    try:
        dx, do = hip.DeviceBuffer(64 * 768), hip.DeviceBuffer(64 * 64)
        with pytest.raises(qmv.QmvError):               # unequal cols
            qmv.matmul_batch_group_dev([a, b], dx.ptr, 4, [do.ptr, do.ptr])
        with pytest.raises(qmv.QmvError):               # five matrices
            qmv.matmul_batch_group_dev([a] * 5, dx.ptr, 4, [do.ptr] * 5)
        dx.free()
        do.free()
    finally:
        a.close()
        b.close()
