#!/usr/bin/env python3
"""Benchmark of the MI355X attention path of kore (libkore_attn.so).

Headline workload: Qwen2.5-7B-shape single-token decode attention, batch 1,
28 layers (28 q-heads / 4 kv-heads, head_dim 128), fp32 KV cache sized for
ctx 8192 and filled to 4096 positions, one new token per step at positions
4096, 4097, ...; q/k/v are seeded counter-based N(0,1) values with 1 % of
channels scaled x20.  One step = one token through all 28 layers, each layer
one kore_attn_decode_dev call (kore's per-layer attention block,
kore.cpp:1405-1455), driven from C++ (libkore_attn_bench.so) so no Python
runs between launches.

Also reported (under "matvec"): the Q4_K/Q6_K x Q8_K matrix-vector products
of one Qwen2.5-7B-shape token (libkore_qmv.so): 28 layers x (q, k, v, o, gate,
up, down) plus the output head, 197 matrices / 4.37 GB of weights, each
quant() + mv() pair of kore's forward() (kore.cpp:1418-1477), bit-identical
to kore's AVX2 results; with kore's own multithreaded matvec timed on the host.

Reported next to it: Qwen2.5-7B-shape causal prefill attention of a
2048-token prompt at position 0 over 28 layers (kore.cpp:1503-1563), and the
CPU restatement of kore's attention (bit-identical to kore's own code) timed
on this host on a bounded sample of the same inputs, single-threaded as
kore's attention is (its loops at kore.cpp:1432 and 1542 sit outside
parallel_rows).  The CPU leg doubles as a parity check: its outputs for the
same (layer, position) are compared with the GPU's.

    python bench.py [--steps 128] [--warmup 8] [--prefill-steps 3] [--no-cpu]

Prints one JSON line.  One GPU only: --gpus N with N > 1 exits with a message.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "7B decode attn µs/layer + HBM GB/s @ctx4096; prefill attn TFLOP/s"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, published
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix, published

# Qwen2.5-7B attention geometry
NL, NH, NKV, HD = 28, 28, 4, 128
E, KVD = NH * HD, NKV * HD
ROPE_BASE = 1e6
DEC_CTX, DEC_POS0 = 8192, 4096
DEC_SEED, DEC_PER_MILLE, DEC_OUTLIER = 7, 10, 20.0
DEC_STEPS = 128                # the configured decode steps (positions 4096..4223)
PF_N, PF_SEED = 2048, 3
WARM_SECONDS = 0.5             # least decode work ahead of the timed region (steady clocks)

# HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE on these
# kernels and workloads, each counter scaled by what it reads for a 256 MiB device copy
# (fetch x 2.0, write x 1.0): decode layer = split + combine kernel, prefill layer =
# append + prefill + prefill combine kernel.  Re-measure when a kernel changes.
TRAFFIC_DECODE_BYTES = 19_082_000
TRAFFIC_PREFILL_BYTES = 141_000_000
# the same for the matvec leg's dominant launch, ffn_gate + ffn_up of one layer (76.55 MB
# of weights, activations and outputs algorithmic)
TRAFFIC_MATVEC_BYTES = {"ffn_gate_q4k+ffn_up_q4k": 80_449_000}
# the same for the batched matmul leg's dominant launch, ffn_gate + ffn_up of one layer on 64
# activations (87.17 MB algorithmic), fp16 path: split pre-pass 1.93 MB, main kernel 124.3 MB
# (the partials of split tiles included), fix-up 35.1 MB
TRAFFIC_GEMM_BYTES = {"ffn_gate_q4k+ffn_up_q4k": 161_290_000}
FP16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 matrix, published
# MFMA passes per product of the fp16 batched matmul: Q4_K hi and lo parts of the
# activations (the minimums' MFMA adds 1/32), Q6_K also the weights' integer remainder
GEMM16_PASSES = {12: 2 + 1 / 32, 14: 3}

# Qwen2.5-7B matrix shapes of the matvec leg
QMV_FF, QMV_VOCAB = 18944, 152064
QMV_Q4K, QMV_Q6K = 12, 14
QMV_SEED = 17


def _more_bits(i: int, n: int) -> bool:
    # layers whose attn_v and ffn_down a Q4_K_M file keeps in Q6_K (llama.cpp's
    # use_more_bits rule); the others are Q4_K, like attn_q/k/o and ffn_gate/up
    return i < n // 8 or i >= 7 * n // 8 or (i - n // 8) % 3 == 2


def qmv_token_matrices():
    """(name, type, rows, cols) of every weight matrix one 7B token multiplies."""
    mats = []
    for l in range(NL):
        hi = QMV_Q6K if _more_bits(l, NL) else QMV_Q4K
        mats += [(f"blk.{l}.attn_q", QMV_Q4K, E, E), (f"blk.{l}.attn_k", QMV_Q4K, KVD, E),
                 (f"blk.{l}.attn_v", hi, KVD, E), (f"blk.{l}.attn_output", QMV_Q4K, E, E),
                 (f"blk.{l}.ffn_gate", QMV_Q4K, QMV_FF, E), (f"blk.{l}.ffn_up", QMV_Q4K, QMV_FF, E),
                 (f"blk.{l}.ffn_down", hi, E, QMV_FF)]
    mats.append(("output", QMV_Q6K, QMV_VOCAB, E))
    return mats


def qmv_weight_bytes(wtype: int, rows: int, cols: int) -> int:
    return rows * (cols // 256) * (144 if wtype == QMV_Q4K else 210)


def q_stream(layer): return (1 << 32) | layer
def k_stream(layer): return (2 << 32) | layer
def v_stream(layer): return (3 << 32) | layer


def decode_bytes(L: int) -> int:
    """Algorithmic HBM bytes of one decode layer attending L positions: K and
    V rows read once per kv-head, q in and out, the new k/v row in and its
    append."""
    return 2 * L * KVD * 4 + 2 * E * 4 + 4 * KVD * 4


def prefill_flops(pos0: int, n: int) -> int:
    """QK^T and PV flops over the causal (unmasked) pairs of one layer."""
    pairs = n * pos0 + n * (n + 1) // 2
    return NH * 4 * HD * pairs


def _stats(ms):
    a = np.asarray(ms, np.float64)
    return dict(mean=float(a.mean()), median=float(np.median(a)), p90=float(np.percentile(a, 90)),
                min=float(a.min()), max=float(a.max()))


def _bench_lib():
    from kore_amd import _lib
    _lib.lib()
    # the timing build's driver when the package was pointed at the timing library (--decode-timeline)
    timing = os.path.basename(_lib.LIB_PATH) == "libkore_attn_tl.so"
    path = os.path.join(ROOT, "kore_amd", "libkore_attn_bench_tl.so" if timing else "libkore_attn_bench.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built; run `make -C kore_amd/csrc`")
    L = C.CDLL(path)
    vp, i = C.c_void_p, C.c_int
    L.kab_decode_run.argtypes = [vp, i, i, i, i, vp, vp, vp, i, vp, i, vp, C.POINTER(C.c_float),
                                 C.POINTER(C.c_double)]
    L.kab_prefill_run.argtypes = [vp, i, i, i, i, vp, vp, vp, vp, vp, C.POINTER(C.c_float), C.POINTER(C.c_double)]
    L.kab_decode_host_run.argtypes = [vp, i, i, i, vp, vp, vp, i, vp, C.POINTER(C.c_double)]
    L.kab_prefill_host_run.argtypes = [vp, i, i, i, vp, vp, vp, vp, C.POINTER(C.c_double)]
    return L


def _check(rc, what):
    if rc != 0:
        from kore_amd import _lib
        raise RuntimeError(f"{what} failed ({rc}): {_lib.lib().kore_attn_last_error(None).decode()}")


# ------------------------------------------------------------------ GPU legs

def gpu_decode(steps: int, warmup: int, extras: bool = True):
    from kore_amd import KoreAttn, hip, synth_dev
    B = _bench_lib()
    attn = KoreAttn(NL, DEC_CTX, NH, NKV, HD, ROPE_BASE)
    st = attn.stream
    # cache positions 0..4095 of every layer through the append path
    qb, kb, vb = hip.DeviceBuffer(DEC_POS0 * E), hip.DeviceBuffer(DEC_POS0 * KVD), hip.DeviceBuffer(DEC_POS0 * KVD)
    ob = hip.DeviceBuffer(DEC_POS0 * E)
    for l in range(NL):
        synth_dev(qb.ptr, DEC_POS0, E, DEC_SEED, q_stream(l), 0, 1, DEC_PER_MILLE, DEC_OUTLIER, st)
        synth_dev(kb.ptr, DEC_POS0, KVD, DEC_SEED, k_stream(l), 0, 2, DEC_PER_MILLE, DEC_OUTLIER, st)
        synth_dev(vb.ptr, DEC_POS0, KVD, DEC_SEED, v_stream(l), 0, 3, DEC_PER_MILLE, DEC_OUTLIER, st)
        attn.prefill_dev(l, 0, DEC_POS0, qb.ptr, kb.ptr, vb.ptr, ob.ptr)
    attn.sync()
    for b in (qb, kb, vb, ob):
        b.free()
    n_in = max(steps, warmup, DEC_STEPS)
    dq, dk, dv = hip.DeviceBuffer(NL * n_in * E), hip.DeviceBuffer(NL * n_in * KVD), hip.DeviceBuffer(NL * n_in * KVD)
    for l in range(NL):
        synth_dev(dq.at(l * n_in * E), n_in, E, DEC_SEED, q_stream(l), DEC_POS0, 1, DEC_PER_MILLE, DEC_OUTLIER, st)
        synth_dev(dk.at(l * n_in * KVD), n_in, KVD, DEC_SEED, k_stream(l), DEC_POS0, 2, DEC_PER_MILLE, DEC_OUTLIER, st)
        synth_dev(dv.at(l * n_in * KVD), n_in, KVD, DEC_SEED, v_stream(l), DEC_POS0, 3, DEC_PER_MILLE, DEC_OUTLIER, st)
    attn.sync()
    out = hip.DeviceBuffer(steps * NL * E)
    wall, wall2, region = C.c_double(0), C.c_double(0), C.c_float(0)
    # warm-up: the requested steps, then more of them until WARM_SECONDS of decode work have run, so
    # the timed region starts at the device's steady clocks whatever --warmup is
    t_warm, warm_steps = time.perf_counter(), 0
    while warm_steps < warmup or time.perf_counter() - t_warm < WARM_SECONDS:
        n_w = max(1, min(warmup, steps)) if warmup else min(8, steps)
        _check(B.kab_decode_run(attn.handle, NL, DEC_POS0, 1, n_w, dq.ptr, dk.ptr, dv.ptr, n_in, out.ptr,
                                steps, None, None, C.byref(wall)), "decode warmup")
        warm_steps += n_w
    warm_s = time.perf_counter() - t_warm
    print(f"[bench] decode: {steps} timed steps x {NL} layers at positions {DEC_POS0}.. (after {warm_steps} "
          f"warm-up steps, {warm_s:.2f} s)", file=sys.stderr, flush=True)
    # the timed steps: host clock and one HIP event pair around the region
    _check(B.kab_decode_run(attn.handle, NL, DEC_POS0, 1, steps, dq.ptr, dk.ptr, dv.ptr, n_in, out.ptr, steps,
                            None, C.byref(region), C.byref(wall)), "decode timed")
    # the same steps again with an event pair around every launch (per-launch
    # spread; re-running a step rewrites the same cache row with the same data)
    launch_ms = np.zeros(steps * NL, np.float32)
    _check(B.kab_decode_run(attn.handle, NL, DEC_POS0, 1, steps, dq.ptr, dk.ptr, dv.ptr, n_in, out.ptr, steps,
                            launch_ms.ctypes.data, None, C.byref(wall2)), "decode per-launch events")
    if not extras:
        out.free()
        return dict(attn=attn, launch_ms=launch_ms, wall_ms=wall.value, region_ms=region.value,
                    buffers=(dq, dk, dv), warm_steps=warm_steps, warm_s=warm_s)
    # all 128 configured steps once more, untimed, for the parity check
    out.free()
    par = hip.DeviceBuffer(DEC_STEPS * NL * E)
    _check(B.kab_decode_run(attn.handle, NL, DEC_POS0, 1, DEC_STEPS, dq.ptr, dk.ptr, dv.ptr, n_in, par.ptr,
                            DEC_STEPS, None, None, C.byref(wall2)), "decode parity pass")
    outs = par.download().reshape(DEC_STEPS, NL, E)
    par.free()
    # the host-pointer entry point kore's forward() would call (kore_attn_decode:
    # H2D of q/k/v, the kernels, D2H of the output, per layer), on the timed steps
    hq = dq.download(NL * n_in * E).reshape(NL, n_in, E)
    hk = dk.download(NL * n_in * KVD).reshape(NL, n_in, KVD)
    hv = dv.download(NL * n_in * KVD).reshape(NL, n_in, KVD)
    hout = np.zeros((NL, E), np.float32)
    host_steps = min(steps, 32)
    wall_h = C.c_double(0)
    _check(B.kab_decode_host_run(attn.handle, NL, DEC_POS0, host_steps, hq.ctypes.data, hk.ctypes.data,
                                 hv.ctypes.data, n_in, hout.ctypes.data, C.byref(wall_h)), "decode host pass")
    info = attn.info()
    return dict(attn=attn, outs=outs, launch_ms=launch_ms, wall_ms=wall.value, region_ms=region.value,
                num_cu=info.num_cu, buffers=(dq, dk, dv), host_us_per_layer=wall_h.value * 1e3 / (host_steps * NL),
                host_steps=host_steps, warm_steps=warm_steps, warm_s=warm_s)


TL_SPLIT_STAMPS = ("start", "K requested", "q staged", "single rows scored", "V requested", "block done",
                   "wave state in LDS", "past the barrier", "partial stored", "end", "q requested")
TL_COMB_STAMPS = ("start", "partials loaded", "end")


def decode_timeline(steps: int, raw_path: str = "", samples: int = 16, config: str = "7b"):
    """The decode workload on the timing build of the attention library: libkore_attn_tl.so, whose
    decode_split_kernel and decode_combine_kernel keep s_memrealtime stamps (100 MHz, one counter for
    the whole device) per wave / per workgroup in registers and write them when each ends.  config
    "7b": the headline workload (28 layers, cache filled to 4096, `steps` steps after the timed
    warm-up); "3b": the 3B decode at position 32767 (36 layers, the same position repeated).  The
    stamps of the last launch of each kernel (the last layer of the last step) are read: per stamp
    the median, 10th percentile and maximum over the split kernel's waves and the combine's
    workgroups, in us from the first split wave's start.  Then `samples` more single steps, each read
    the same way, give per XCD (workgroup index mod 8, the order in which the dispatcher deals
    workgroups to the XCDs) the median over samples of the XCD's earliest workgroup start and latest
    workgroup end.  The stamps perturb the kernels a little; use them for where the time goes, the
    plain bench for how long it takes."""
    from kore_amd import KoreAttn, _lib, hip, synth_dev
    L = _lib.lib()   # main() pointed the package at the timing build before anything loaded it
    read = L.kore_attn_tl_read
    read.restype = C.c_int
    read.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t]
    B = _bench_lib()
    wall, region = C.c_double(0), C.c_float(0)
    if config == "7b":
        dec = gpu_decode(steps, 0, extras=False)
        attn, (dq, dk, dv) = dec["attn"], dec["buffers"]
        nl, nh, nkv, hd, pos, pos_step, n_in = NL, NH, NKV, HD, DEC_POS0, 1, max(steps, DEC_STEPS)
        per = dec["region_ms"] / 1e3 / (steps * NL)
    else:
        nl, nh, nkv, hd, pos, pos_step, n_in = 36, 16, 2, 128, 32767, 0, 1
        attn = KoreAttn(nl, 32768, nh, nkv, hd, ROPE_BASE)
        _fill_cache(attn, nl, pos, nkv * hd, 9, attn.stream)
        dq, dk, dv = hip.DeviceBuffer(nl * nh * hd), hip.DeviceBuffer(nl * nkv * hd), hip.DeviceBuffer(nl * nkv * hd)
        for l in range(nl):
            synth_dev(dq.at(l * nh * hd), 1, nh * hd, 9, q_stream(l), pos, 1, 0, 1.0, attn.stream)
            synth_dev(dk.at(l * nkv * hd), 1, nkv * hd, 9, k_stream(l), pos, 2, 0, 1.0, attn.stream)
            synth_dev(dv.at(l * nkv * hd), 1, nkv * hd, 9, v_stream(l), pos, 3, 0, 1.0, attn.stream)
        attn.sync()
        o = hip.DeviceBuffer(nl * nh * hd)
        t_warm = time.perf_counter()
        while time.perf_counter() - t_warm < WARM_SECONDS:
            _check(B.kab_decode_run(attn.handle, nl, pos, 0, 4, dq.ptr, dk.ptr, dv.ptr, 1, o.ptr, 1, None, None,
                                    C.byref(wall)), "decode warmup")
        _check(B.kab_decode_run(attn.handle, nl, pos, 0, steps, dq.ptr, dk.ptr, dv.ptr, 1, o.ptr, 1, None,
                                C.byref(region), C.byref(wall)), "decode timed")
        o.free()
        per = region.value / 1e3 / (steps * nl)
    info = attn.info()
    n_split = max(1, min(info.num_cu // nkv, 128))
    n_wg = n_split * nkv
    waves = n_wg * 4
    comb_wg = nh * (hd // 32)
    ts = np.zeros((waves, len(TL_SPLIT_STAMPS)), np.uint64)
    tc = np.zeros((comb_wg, len(TL_COMB_STAMPS)), np.uint64)

    def grab():
        if read(ts.ctypes.data, ts.size, tc.ctypes.data, tc.size) != 0:
            raise RuntimeError("kore_attn_tl_read failed")
        t0 = int(ts[:, 0].min())
        return (ts.astype(np.int64) - t0) / 100.0, (tc.astype(np.int64) - t0) / 100.0

    us_s, us_c = grab()
    out = hip.DeviceBuffer(nl * nh * hd)
    xs, xe, spans, gaps = [], [], [], []
    for i in range(samples):
        _check(B.kab_decode_run(attn.handle, nl, pos, pos_step, 1, dq.ptr, dk.ptr, dv.ptr, n_in, out.ptr, 1,
                                None, None, C.byref(wall)), "decode timeline sample")
        s_i, c_i = grab()
        wg_start = s_i[:, 0].reshape(n_wg, 4).min(1)
        wg_end = s_i[:, TL_SPLIT_STAMPS.index("end")].reshape(n_wg, 4).max(1)
        xs.append([wg_start[x::8].min() for x in range(8)])
        xe.append([wg_end[x::8].max() for x in range(8)])
        spans.append(wg_end.max())
        gaps.append(c_i[:, 0].min() - wg_end.max())
    out.free()
    for b in (dq, dk, dv):
        b.free()
    attn.close()

    def row(x):
        return {"median": round(float(np.median(x)), 2), "p10": round(float(np.percentile(x, 10)), 2),
                "max": round(float(np.max(x)), 2)}

    if raw_path:
        np.savez(raw_path, split=us_s, combine=us_c, xcd_start=np.asarray(xs), xcd_end=np.asarray(xe))
    return {"config": config, "us_per_layer_gpu": round(per * 1e6, 3), "steps": steps,
            "splits_per_kv_head": n_split, "split_waves": waves, "combine_workgroups": comb_wg,
            "unit": "us from the first split wave's start",
            "split": {name: row(us_s[:, i]) for i, name in enumerate(TL_SPLIT_STAMPS)},
            "split_median_by_wave": {name: [round(float(np.median(us_s[w::4, i])), 2) for w in range(4)]
                                     for i, name in enumerate(TL_SPLIT_STAMPS)},
            "combine": {name: row(us_c[:, i]) for i, name in enumerate(TL_COMB_STAMPS)},
            "samples": samples, "split_span": row(spans), "gap_to_combine": row(gaps),
            "xcd_first_start_median": [round(float(v), 2) for v in np.median(np.asarray(xs), 0)],
            "xcd_last_end_median": [round(float(v), 2) for v in np.median(np.asarray(xe), 0)]}


SWEEP_7B = (256, 1024, 2048, 3072, 4096, 4352, 4420, 5000, 6144, 8192, 8704, 9000, 12288, 16384, 24576, 32767)
SWEEP_3B = (2048, 4096, 8192, 16384, 17408, 20000, 32767)


def decode_sweep():
    """The decode across the context: Qwen2.5-7B shape (28 layers, cache of 32768 slots) and 3B
    shape (36 layers, 32768 slots), each filled once through the append path; per position the
    step's us per layer over 40 repeated steps at that position (HIP events, time-based warm-up)
    and its fraction of 8 TB/s, with the kernel the split rule picks (one or two workgroups per
    CU, single- or multi-block)."""
    from kore_amd import KoreAttn
    out = {}
    for name, (nl, nh, nkv, hd), poss in (("7b", (28, 28, 4, 128), SWEEP_7B), ("3b", (36, 16, 2, 128), SWEEP_3B)):
        rows = []
        with KoreAttn(nl, 32768, nh, nkv, hd, ROPE_BASE) as a:
            _fill_cache(a, nl, 32767, nkv * hd, 7, a.stream)
            for pos in poss:
                r, _ = _decode_leg(a, nl, pos, 0, 40, 2, nh, nkv, hd, 7, lambda s, p=pos: p + 1)
                rows.append({"position": pos, "us_per_layer_gpu": r["us_per_layer_gpu"],
                             "frac": r["roofline"]["frac"]})
                print(f"[bench] sweep {name} {pos}: {r['us_per_layer_gpu']} us", file=sys.stderr, flush=True)
        out[name] = rows
    return out


def gpu_prefill(steps: int, warmup: int):
    from kore_amd import KoreAttn, hip, synth_dev
    B = _bench_lib()
    attn = KoreAttn(NL, PF_N, NH, NKV, HD, ROPE_BASE)
    st = attn.stream
    dq, dk, dv = hip.DeviceBuffer(NL * PF_N * E), hip.DeviceBuffer(NL * PF_N * KVD), hip.DeviceBuffer(NL * PF_N * KVD)
    for l in range(NL):
        synth_dev(dq.at(l * PF_N * E), PF_N, E, PF_SEED, q_stream(l), 0, 1, 0, 1.0, st)
        synth_dev(dk.at(l * PF_N * KVD), PF_N, KVD, PF_SEED, k_stream(l), 0, 2, 0, 1.0, st)
        synth_dev(dv.at(l * PF_N * KVD), PF_N, KVD, PF_SEED, v_stream(l), 0, 3, 0, 1.0, st)
    attn.sync()
    out = hip.DeviceBuffer(NL * PF_N * E)
    wall, region = C.c_double(0), C.c_float(0)
    if warmup:
        _check(B.kab_prefill_run(attn.handle, NL, 0, PF_N, warmup, dq.ptr, dk.ptr, dv.ptr, out.ptr, None, None,
                                 C.byref(wall)), "prefill warmup")
    launch_ms = np.zeros(steps * NL, np.float32)
    print(f"[bench] prefill: {steps} timed passes x {NL} layers of {PF_N} rows", file=sys.stderr, flush=True)
    # per-launch events cost ~1 us against ~450 us launches: one pass gives both
    _check(B.kab_prefill_run(attn.handle, NL, 0, PF_N, steps, dq.ptr, dk.ptr, dv.ptr, out.ptr,
                             launch_ms.ctypes.data, C.byref(region), C.byref(wall)), "prefill timed")
    HL = 4   # layers of the host-pointer round trip
    outs = out.download(HL * PF_N * E).reshape(HL, PF_N, E)   # the first layers for the parity checks
    # the host-pointer entry point kore's forward_batch() would call
    # (kore_attn_prefill: H2D of q/k/v, append + attention, D2H of the rows)
    hq = dq.download(HL * PF_N * E)
    hk = dk.download(HL * PF_N * KVD)
    hv = dv.download(HL * PF_N * KVD)
    hout = np.zeros(HL * PF_N * E, np.float32)
    wall_h = C.c_double(0)
    _check(B.kab_prefill_host_run(attn.handle, HL, 0, PF_N, hq.ctypes.data, hk.ctypes.data, hv.ctypes.data,
                                  hout.ctypes.data, C.byref(wall_h)), "prefill host pass")
    host_equal = bool(np.array_equal(hout.view(np.uint32), outs.reshape(-1).view(np.uint32)))
    attn.close()
    for b in (dq, dk, dv, out):
        b.free()
    return dict(outs=outs, launch_ms=launch_ms, wall_ms=wall.value, region_ms=region.value,
                host_us_per_layer=wall_h.value * 1e3 / HL, host_layers=HL, host_equals_device=host_equal)


def _decode_bytes_geom(L: int, nh: int, nkv: int, hd: int) -> int:
    return 2 * L * nkv * hd * 4 + 2 * nh * hd * 4 + 4 * nkv * hd * 4


def _prefill_flops_geom(pos0: int, n: int, nh: int, hd: int) -> int:
    return nh * 4 * hd * (n * pos0 + n * (n + 1) // 2)


def _fill_cache(attn, n_layer, rows, kvd, seed, stream):
    """Cache rows 0..rows-1 of every layer through the append path."""
    from kore_amd import hip, synth_dev
    kb, vb = hip.DeviceBuffer(rows * kvd), hip.DeviceBuffer(rows * kvd)
    for l in range(n_layer):
        synth_dev(kb.ptr, rows, kvd, seed, k_stream(l), 0, 2, 0, 1.0, stream)
        synth_dev(vb.ptr, rows, kvd, seed, v_stream(l), 0, 3, 0, 1.0, stream)
        attn.append_dev(l, 0, rows, kb.ptr, vb.ptr)
    attn.sync()
    kb.free()
    vb.free()


def _decode_leg(attn, n_layer, pos_first, pos_step, steps, warmup, nh, nkv, hd, seed, attended, keep_outs=False):
    """Timed decode steps (one kore_attn_decode_dev per layer and step);
    `attended(s)` is the number of positions step s attends.  keep_outs: the
    outputs of the steps in order from the cache as it is on entry ([steps][layer][E];
    one untimed pass ahead of the warm-up when the steps move, the timed
    region's last outputs when they repeat one position)."""
    from kore_amd import hip, synth_dev
    B = _bench_lib()
    st = attn.stream
    E_, kvd = nh * hd, nkv * hd
    n_in = max(steps, warmup) if pos_step else 1
    dq, dk, dv = hip.DeviceBuffer(n_layer * n_in * E_), hip.DeviceBuffer(n_layer * n_in * kvd), \
        hip.DeviceBuffer(n_layer * n_in * kvd)
    for l in range(n_layer):
        synth_dev(dq.at(l * n_in * E_), n_in, E_, seed, q_stream(l), pos_first, 1, 0, 1.0, st)
        synth_dev(dk.at(l * n_in * kvd), n_in, kvd, seed, k_stream(l), pos_first, 2, 0, 1.0, st)
        synth_dev(dv.at(l * n_in * kvd), n_in, kvd, seed, v_stream(l), pos_first, 3, 0, 1.0, st)
    attn.sync()
    out = hip.DeviceBuffer(n_layer * E_)
    wall, wall2, region = C.c_double(0), C.c_double(0), C.c_float(0)
    outs = None
    if keep_outs and pos_step:
        par = hip.DeviceBuffer(steps * n_layer * E_)
        _check(B.kab_decode_run(attn.handle, n_layer, pos_first, pos_step, steps, dq.ptr, dk.ptr, dv.ptr, n_in,
                                par.ptr, steps, None, None, C.byref(wall)), "decode parity pass")
        outs = par.download().reshape(steps, n_layer, E_)
        par.free()
    t_warm = time.perf_counter()
    while True:
        _check(B.kab_decode_run(attn.handle, n_layer, pos_first, pos_step, max(warmup, 1), dq.ptr, dk.ptr, dv.ptr,
                                n_in, out.ptr, 1, None, None, C.byref(wall)), "decode warmup")
        if time.perf_counter() - t_warm >= WARM_SECONDS / 2:
            break
    _check(B.kab_decode_run(attn.handle, n_layer, pos_first, pos_step, steps, dq.ptr, dk.ptr, dv.ptr, n_in,
                            out.ptr, 1, None, C.byref(region), C.byref(wall)), "decode timed")
    if keep_outs and not pos_step:
        outs = out.download().reshape(1, n_layer, E_)
    lm = np.zeros(steps * n_layer, np.float32)
    _check(B.kab_decode_run(attn.handle, n_layer, pos_first, pos_step, steps, dq.ptr, dk.ptr, dv.ptr, n_in,
                            out.ptr, 1, lm.ctypes.data, None, C.byref(wall2)), "decode per-launch events")
    for b in (dq, dk, dv, out):
        b.free()
    nbytes = sum(_decode_bytes_geom(attended(s), nh, nkv, hd) for s in range(steps)) * n_layer
    mean_s = region.value / 1e3 / (steps * n_layer)
    ach = nbytes / (steps * n_layer) / mean_s / 1e9
    res = {"us_per_layer_gpu": round(mean_s * 1e6, 3), "launch_us_median": round(float(np.median(lm)) * 1e3, 3),
           "gbs_wall": round(nbytes / (wall.value / 1e3) / 1e9, 2),
           "roofline": {"bound": "hbm", "achieved": round(ach, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(ach / HBM_PEAK_GBS, 4)}}
    return res, outs


def _parity_decode_layers(n_layer, rows, nh, nkv, hd, seed, pos_first, outs, threads, window=0, kv_rows=None):
    """The oracle's decode (kore.cpp:1405-1455; with `window`, the last
    `window` positions of a ring) for every layer of a workload whose cache
    rows 0..rows-1 were filled through the append path from synth(seed) and
    whose steps s decode position pos_first + s with synth(seed) inputs:
    max|d|/max|ref| over outs [steps][layer][E].  kv_rows(l) (optional) returns
    the GPU's K and V rows 0..rows (the decoded row included) of layer l, held
    bit for bit to the oracle's."""
    import oracle
    n_steps = outs.shape[0]
    E_, kvd = nh * hd, nkv * hd
    inv_f = oracle.inv_freq(hd, ROPE_BASE)
    ctx = window if window else rows + n_steps

    def layer(l):
        kv = oracle.KV(1, ctx, nh, nkv, hd, ROPE_BASE, window=window)
        k0 = oracle.synth(rows, kvd, seed, k_stream(l), 0, 2)
        kv.kcache()[0, :rows] = oracle.rope_rows(k0, np.arange(rows), nkv, hd, inv_f)
        kv.vcache()[0, :rows] = oracle.synth(rows, kvd, seed, v_stream(l), 0, 3)
        q = oracle.synth(n_steps, E_, seed, q_stream(l), pos_first, 1)
        k = oracle.synth(n_steps, kvd, seed, k_stream(l), pos_first, 2)
        v = oracle.synth(n_steps, kvd, seed, v_stream(l), pos_first, 3)
        errs = [_rel_err(outs[s, l], kv.decode(0, pos_first + s, q[s], k[s], v[s])) for s in range(n_steps)]
        digest = _kv_digest(kv.kcache()[0], kv.vcache()[0]) if kv_rows is not None else None
        kv.close()
        return errs, digest

    res = _pool(layer, range(n_layer), threads)
    e = np.array([r[0] for r in res])
    out = {"max_rel_err": float(e.max()), "layers": n_layer, "steps": n_steps}
    if kv_rows is not None:   # one caller per handle: the GPU rows are read on this thread
        out["kv_bitwise"] = all(_kv_digest(*kv_rows(l)) == r[1] for l, r in enumerate(res))
    return out


def _kv_digest(k, v):
    import hashlib
    return hashlib.sha256(np.ascontiguousarray(k).tobytes()).hexdigest() + \
        hashlib.sha256(np.ascontiguousarray(v).tobytes()).hexdigest()


def gpu_other_workloads(quick: bool, parity_threads: int = 0):
    """The other attention workloads of the path, each on its own handle:
    0.5B single-layer decode at 511, 3B decode at 32767 over 36 layers, 1.5B
    1024-row chunk at 7168 then sliding-window decode at ctx 8192.  With
    parity_threads > 0 each is also compared with the oracle on that many host
    threads (every layer, every step; the 1.5B chunk's every row on four
    layers), returned as the second value."""
    import oracle
    from kore_amd import KoreAttn, hip, synth_dev
    B = _bench_lib()
    res, par = {}, {}
    reps = 20 if quick else 50
    # 0.5B: 14/2/64, one layer, cache 0..510, decode at 511
    with KoreAttn(1, 512, 14, 2, 64, ROPE_BASE) as a:
        _fill_cache(a, 1, 511, 128, 11, a.stream)
        r, outs = _decode_leg(a, 1, 511, 0, reps * 10, 10, 14, 2, 64, 11, lambda s: 512, keep_outs=True)
        r["workload"] = "Qwen2.5-0.5B-shape decode, 1 layer, 14/2/64, position 511 (cache 0..510)"
        res["decode_0p5b_pos511"] = r
        if parity_threads:
            par["c1_decode_0p5b"] = _parity_decode_layers(1, 511, 14, 2, 64, 11, 511, outs, 1,
                                                          kv_rows=lambda l: a.read_kv(l, 0, 512))
    print("[bench] 0.5B decode done", file=sys.stderr, flush=True)
    # 3B: 16/2/128, 36 layers, ctx 32768, decode at 32767
    with KoreAttn(36, 32768, 16, 2, 128, ROPE_BASE) as a:
        _fill_cache(a, 36, 32767, 256, 9, a.stream)
        r, outs = _decode_leg(a, 36, 32767, 0, reps, 2, 16, 2, 128, 9, lambda s: 32768, keep_outs=True)
        r["workload"] = "Qwen2.5-3B-shape decode, 36 layers, 16/2/128, position 32767 (cache 0..32766)"
        res["decode_3b_pos32767"] = r
        if parity_threads:
            par["c4_decode_3b"] = _parity_decode_layers(36, 32767, 16, 2, 128, 9, 32767, outs,
                                                        min(parity_threads, 8),
                                                        kv_rows=lambda l: a.read_kv(l, 0, 32768))
    print("[bench] 3B decode done", file=sys.stderr, flush=True)
    # 1.5B: 12/2/128, 28 layers, ring of 8192 slots
    nl, nh, nkv, hd, W, c0, cn = 28, 12, 2, 128, 8192, 7168, 1024
    with KoreAttn(nl, W, nh, nkv, hd, ROPE_BASE, window=W) as a:
        st = a.stream
        _fill_cache(a, nl, c0, nkv * hd, 5, st)
        E_, kvd = nh * hd, nkv * hd
        dq, dk, dv = hip.DeviceBuffer(nl * cn * E_), hip.DeviceBuffer(nl * cn * kvd), hip.DeviceBuffer(nl * cn * kvd)
        for l in range(nl):
            synth_dev(dq.at(l * cn * E_), cn, E_, 5, q_stream(l), c0, 1, 0, 1.0, st)
            synth_dev(dk.at(l * cn * kvd), cn, kvd, 5, k_stream(l), c0, 2, 0, 1.0, st)
            synth_dev(dv.at(l * cn * kvd), cn, kvd, 5, v_stream(l), c0, 3, 0, 1.0, st)
        a.sync()
        out = hip.DeviceBuffer(nl * cn * E_)
        wall, region = C.c_double(0), C.c_float(0)
        _check(B.kab_prefill_run(a.handle, nl, c0, cn, 1, dq.ptr, dk.ptr, dv.ptr, out.ptr, None, None,
                                 C.byref(wall)), "chunk warmup")
        P = 2
        lm = np.zeros(P * nl, np.float32)
        _check(B.kab_prefill_run(a.handle, nl, c0, cn, P, dq.ptr, dk.ptr, dv.ptr, out.ptr, lm.ctypes.data,
                                 C.byref(region), C.byref(wall)), "chunk timed")
        chunk_layers = (0, 9, 18, 27)
        chunk_outs = {l: out.download(cn * E_, offset=l * cn * E_).reshape(cn, E_) for l in chunk_layers} \
            if parity_threads else None
        for b in (dq, dk, dv, out):
            b.free()
        F = _prefill_flops_geom(c0, cn, nh, hd)
        per_s = region.value / 1e3 / (P * nl)
        ach = F / per_s / 1e12
        chunk = {"us_per_layer_gpu": round(per_s * 1e6, 2), "flop_per_layer": F,
                 "roofline": {"bound": "mfma", "achieved": round(ach, 3), "peak": FP32_MFMA_PEAK_TFLOPS,
                              "unit": "TFLOP/s", "frac": round(ach / FP32_MFMA_PEAK_TFLOPS, 4)}}
        dec, outs = _decode_leg(a, nl, W, 1, 256, 8, nh, nkv, hd, 5, lambda s: W, keep_outs=bool(parity_threads))
        res["chunk_1p5b_1024_at_7168"] = dict(chunk, workload="Qwen2.5-1.5B-shape causal prefill chunk, 28 layers, "
                                                              "12/2/128, 1024 rows at 7168 onto 7168 cached rows")
        res["decode_1p5b_sliding_8192"] = dict(dec, workload="Qwen2.5-1.5B-shape decode, 28 layers, ring of 8192 "
                                                             "slots, 256 steps at positions 8192..8447")
    if parity_threads:
        # the chunk: every row of four layers against the oracle's batched attention
        # (kore's AVX2 hd_dot / hd_fma arithmetic), 64-row pieces on the host threads
        inv_f = oracle.inv_freq(hd, ROPE_BASE)

        def chunk_piece(item):
            l, z0 = item
            k = np.concatenate([oracle.synth(c0, kvd, 5, k_stream(l), 0, 2),
                                oracle.synth(cn, kvd, 5, k_stream(l), c0, 2)])
            v = np.concatenate([oracle.synth(c0, kvd, 5, v_stream(l), 0, 3),
                                oracle.synth(cn, kvd, 5, v_stream(l), c0, 3)])
            K = oracle.rope_rows(k[:c0 + z0 + 64], np.arange(c0 + z0 + 64), nkv, hd, inv_f)
            q = oracle.synth(64, E_, 5, q_stream(l), c0 + z0, 1)
            qr = oracle.rope_rows(q, np.arange(c0 + z0, c0 + z0 + 64), nh, hd, inv_f)
            ref = oracle.attn_batch(qr, c0 + z0, K, v[:c0 + z0 + 64], nh, nkv, hd, avx2=True)
            return _rel_err(chunk_outs[l][z0:z0 + 64], ref)

        errs = _pool(chunk_piece, [(l, z0) for l in chunk_layers for z0 in range(0, cn, 64)], parity_threads)
        par["c5_chunk_1p5b"] = {"max_rel_err": float(max(errs)), "layers": list(chunk_layers), "rows": cn}
        par["c5_sliding_decode_1p5b"] = _parity_decode_layers(nl, c0 + cn, nh, nkv, hd, 5, W, outs,
                                                              parity_threads, window=W)
    print("[bench] 1.5B chunk + sliding decode done", file=sys.stderr, flush=True)
    return res, par


class _KqbOp(C.Structure):
    _fields_ = [("kind", C.c_int), ("n_t", C.c_int), ("t", C.c_int * 4), ("x", C.c_void_p), ("n", C.c_longlong),
                ("xq", C.c_void_p), ("out", C.c_void_p * 4)]


def _op(kind, tensors=(), x=None, n=0, xq=None, outs=()):
    o = _KqbOp()
    o.kind, o.n_t, o.x, o.n, o.xq = kind, len(tensors), x, n, xq
    for k, t in enumerate(tensors):
        o.t[k] = t
    for k, p in enumerate(outs):
        o.out[k] = p
    return o


def _qmv_bench_lib():
    from kore_amd import qmv
    path = os.path.join(ROOT, "kore_amd", "libkore_qmv_bench.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built; run `make -C kore_amd/csrc`")
    qmv.lib()
    B = C.CDLL(path)
    B.kqb_run.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                          C.POINTER(C.c_float), C.POINTER(C.c_double)]
    return B


def qmv_tensors():
    """The 197 weight matrices of one 7B token (qmv_token_matrices), synthetic,
    resident on the device; the bytes of the first are kept for the parity
    checks against kore's arithmetic."""
    from kore_amd import hip, qmv
    mats = qmv_token_matrices()
    biggest = max(qmv_weight_bytes(t, r, c) for _, t, r, c in mats)
    raw = hip.DeviceBuffer((biggest + 3) // 4)
    tensors, first_raw = [], None
    print(f"[bench] creating {len(mats)} synthetic weight matrices", file=sys.stderr, flush=True)
    for idx, (name, t, r, c) in enumerate(mats):
        qmv.synth_dev(t, r, c, QMV_SEED * 1000 + idx, raw.ptr)
        if idx == 0:
            hip.synchronize()
            first_raw = np.zeros(qmv_weight_bytes(t, r, c), np.uint8)
            hip.check(hip.lib().hipMemcpy(first_raw.ctypes.data, raw.ptr, first_raw.size, hip.D2H), "download")
        tensors.append(qmv.QMat(t, r, c, device_ptr=raw.ptr))
    raw.free()
    return mats, tensors, first_raw


def _act(rng, n):
    x = rng.standard_normal(n).astype(np.float32)
    x[rng.random(n) < 0.01] *= 20.0
    return x


def _kqb_runner(B, ops, tensors):
    from kore_amd import qmv
    arr = (_KqbOp * len(ops))(*ops)
    handles = (C.c_void_p * len(tensors))(*[m.handle.value for m in tensors])
    wall = C.c_double(0)

    def run(n, op_ms=None, reg=None):
        rc = B.kqb_run(arr, len(ops), handles, 1, n, None, op_ms, reg, C.byref(wall))
        if rc != 0:
            raise RuntimeError(f"kqb_run failed ({rc}): {qmv.lib().kore_qmv_last_error(None).decode()}")
        return wall.value
    return run


def _mv_key(mats, ts):
    """Name of a grouped matvec launch: its matrices' roles and types."""
    return "+".join(mats[ti][0].split(".")[-1] + ("" if mats[ti][0] == "output" else
                                                   ("_q6k" if mats[ti][1] == QMV_Q6K else "_q4k")) for ti in ts)


def _gemm_key(mats, ts):
    return "+".join(mats[ti][0].split(".")[-1] + ("_q6k" if mats[ti][1] == QMV_Q6K else "_q4k") for ti in ts)


def _class_passes(B, ops, keys, tensors, reps: int):
    """GPU time per launch of each kind of launch (key): the launches of one
    kind, in layer order, back to back between one HIP event pair on the
    stream they run on, the kinds in turn, `reps` times.  Between two passes of
    one kind the others stream far more than the 256 MB MALL, so each pass
    reads its weights from HBM as the token does; the time per launch then
    holds the kernel and the dependent-launch gap, as in the token, and no
    per-launch event (which adds ~2.4 us to each launch it brackets)."""
    kinds = list(dict.fromkeys(keys))
    runners = {k: _kqb_runner(B, [o for o, kk in zip(ops, keys) if kk == k], tensors) for k in kinds}
    count = {k: keys.count(k) for k in kinds}
    out = {k: [] for k in kinds}
    reg = C.c_float(0)
    for _ in range(reps):
        for k in kinds:
            runners[k](1, reg=C.byref(reg))
            out[k].append(reg.value / count[k])
    return out


def gpu_matvec(qt, tokens: int, warmup: int):
    """One 7B token's quant() + mv() sequence (kore.cpp:1418-1477) over 28
    distinct layers plus the output head, replayed `tokens` times from C++."""
    from kore_amd import hip
    B = _qmv_bench_lib()
    mats, tensors, first_raw = qt
    rng = np.random.default_rng(QMV_SEED)
    xs = [_act(rng, E) for _ in range(4)] + [_act(rng, QMV_FF)]
    dx = [hip.DeviceBuffer.from_array(x) for x in xs]
    outs = [hip.DeviceBuffer(r) for _, _, r, _ in mats]
    # kore's forward(): quant(xb) -> q, k, v; quant(att) -> o; quant(xb) -> gate, up;
    # quant(gate) -> down; quant(xb) -> output (kore.cpp:1418-1477).  Matrices that
    # share an input go in one launch (kore_qmv_mv_group_dev), the quantisation
    # fused into it where that is cheaper.
    ops, op_mats = [], []
    for l in range(NL):
        b = 7 * l
        for ts, x in (((b, b + 1, b + 2), dx[0]), ((b + 3,), dx[1]), ((b + 4, b + 5), dx[2]), ((b + 6,), dx[4])):
            ops.append(_op(2, ts, x.ptr, outs=[outs[i].ptr for i in ts]))
            op_mats.append(ts)
    ops.append(_op(2, (7 * NL,), dx[3].ptr, outs=[outs[7 * NL].ptr]))
    op_mats.append((7 * NL,))
    run = _kqb_runner(B, ops, tensors)
    region = C.c_float(0)
    if warmup:
        run(warmup)
    print(f"[bench] matvec: {tokens} timed tokens x {len(ops)} launches", file=sys.stderr, flush=True)
    wall_ms = run(tokens, reg=C.byref(region))
    region_ms = region.value
    # time per launch of each kind (one event pair around each kind's launches)
    class_ms = _class_passes(B, ops, [_mv_key(mats, ts) for ts in op_mats], tensors, min(tokens, 4))
    got = outs[0].download()      # for the bitwise check of the first matrix against kore's arithmetic
    for b in dx + outs:
        b.free()
    return dict(mats=mats, op_mats=op_mats, wall_ms=wall_ms, region_ms=region_ms,
                class_ms=class_ms, first_raw=first_raw, first_x=xs[0], first_out=got)


GEMM_B = 64      # kore's prefill chunk, KORE_BMAX (kore.cpp:690)


def gpu_gemm(qt, chunks: int, warmup: int):
    """forward_batch()'s seven matmul_batch_float calls per layer
    (kore.cpp:1524-1526, 1566, 1575-1576, 1585) for one 64-token chunk over
    the 28 distinct 7B layers, replayed `chunks` times from C++."""
    from kore_amd import hip
    B = _qmv_bench_lib()
    mats, tensors, first_raw = qt
    rng = np.random.default_rng(QMV_SEED + 1)
    xb = np.stack([_act(rng, E) for _ in range(GEMM_B)])
    att = np.stack([_act(rng, E) for _ in range(GEMM_B)])
    gate = np.stack([_act(rng, QMV_FF) for _ in range(GEMM_B)])
    dxb, datt, dgate = (hip.DeviceBuffer.from_array(a) for a in (xb, att, gate))
    # kore's per-role output buffers, reused by every layer (bq, bk, bv, bo, bgate, bup, bo)
    douts = [hip.DeviceBuffer(GEMM_B * r) for r in (E, KVD, KVD, E, QMV_FF, QMV_FF, E)]
    # q+k+v and gate+up share their input: one grouped launch each
    # (kore_qmv_matmul_batch_group_dev); attn_output and ffn_down alone
    ops, op_mats = [], []
    for l in range(NL):
        b = 7 * l
        for js, x in (((0, 1, 2), dxb), ((3,), datt), ((4, 5), dxb), ((6,), dgate)):
            ts = tuple(b + j for j in js)
            ops.append(_op(4, ts, x.ptr, n=GEMM_B, outs=[douts[j].ptr for j in js]))
            op_mats.append(ts)
    run = _kqb_runner(B, ops, tensors)
    region = C.c_float(0)
    if warmup:
        run(warmup)
    print(f"[bench] gemm: {chunks} timed {GEMM_B}-token chunks x {len(ops)} launches", file=sys.stderr, flush=True)
    wall_ms = run(chunks, reg=C.byref(region))
    region_ms = region.value
    class_ms = _class_passes(B, ops, [_gemm_key(mats, ts) for ts in op_mats], tensors, min(chunks, 3))
    # the last layer's attn_q output is overwritten by later layers: run layer 0's alone for the check
    one = _kqb_runner(B, ops[:1], tensors)
    one(1)
    got = douts[0].download().reshape(GEMM_B, E)
    for b in [dxb, datt, dgate] + douts:
        b.free()
    return dict(mats=mats, op_mats=op_mats, wall_ms=wall_ms, region_ms=region_ms,
                class_ms=class_ms, first_raw=first_raw, first_x=xb, first_out=got)


def _klb():
    """libkore_layer_bench.so with its two drivers typed."""
    from kore_amd.layer import _Weights
    from kore_amd.layer import lib as layer_lib
    layer_lib()
    path = os.path.join(ROOT, "kore_amd", "libkore_layer_bench.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built; run `make -C kore_amd/csrc`")
    B = C.CDLL(path)
    vp = C.c_void_p
    B.klb_tokens.argtypes = [vp, C.POINTER(_Weights), C.c_int, vp, vp, vp, C.c_float, vp, C.c_int, C.c_int, C.c_int,
                             vp, vp, C.c_int, C.c_int, C.POINTER(C.c_float), C.POINTER(C.c_double)]
    B.klb_prefill.argtypes = [vp, C.POINTER(_Weights), C.c_int, vp, vp, vp, C.c_float, vp, C.c_int, C.c_int, C.c_int,
                              vp, vp, C.c_int, C.POINTER(C.c_float), C.POINTER(C.c_double)]
    return B


def _engine_weights(qt, rng):
    """The 28 layers' device weights (the synthetic Q4_K_M matrices of qt plus
    norms and biases) as kore_layer_weights, and the output norm."""
    from kore_amd import hip
    from kore_amd.layer import LayerWeights, _Weights
    _, tensors, _ = qt
    lws, bufs = [], []
    for l in range(NL):
        lw = LayerWeights()
        lw.mats = tensors[7 * l:7 * l + 7]
        for name, n, scale in (("attn_norm", E, 0.1), ("ffn_norm", E, 0.1), ("bq", E, 0.5), ("bk", KVD, 0.5),
                               ("bv", KVD, 0.5)):
            a = (rng.standard_normal(n) * scale + (1.0 if "norm" in name else 0.0)).astype(np.float32)
            lw.bufs[name] = hip.DeviceBuffer.from_array(a)
            bufs.append(lw.bufs[name])
        lws.append(lw)
    warr = (_Weights * NL)(*[lw.struct() for lw in lws])
    out_norm = hip.DeviceBuffer.from_array((1 + 0.1 * rng.standard_normal(E)).astype(np.float32))
    return warr, out_norm, bufs + [out_norm]


def gpu_token(qt, tokens: int, warmup: int):
    """Whole 7B decode tokens as kore's forward() runs them (kore.cpp:1397-1484):
    28 layers through kore_layer_decode_dev (rmsnorm+quant+q/k/v+bias, RoPE +
    append + attention, Wo + residual, rmsnorm+quant+gate/up, SwiGLU+quant+down
    + residual) and the logits (rmsnorm+quant+output head), at positions
    4096.. over a cache filled to 4096, driven from C++."""
    from kore_amd import KoreAttn, hip
    from kore_amd.layer import Layer
    from kore_amd.layer import lib as layer_lib
    B = _klb()
    _, tensors, _ = qt
    rng = np.random.default_rng(QMV_SEED + 2)
    attn = KoreAttn(NL, DEC_CTX, NH, NKV, HD, ROPE_BASE)
    print("[bench] token: filling the 28-layer cache to 4096", file=sys.stderr, flush=True)
    _fill_cache(attn, NL, DEC_POS0, KVD, 11, None)
    warr, out_norm, bufs = _engine_weights(qt, rng)
    emb = hip.DeviceBuffer.from_array(np.stack([_act(rng, E) for _ in range(tokens)]))
    x, logits = hip.DeviceBuffer(E), hip.DeviceBuffer(QMV_VOCAB)
    L = Layer(E, QMV_FF, NH, NKV, 1e-6)
    region, wall = C.c_float(0), C.c_double(0)

    def run(reps, reg=None):
        rc = B.klb_tokens(L._h, warr, NL, attn.handle, tensors[7 * NL].handle, out_norm.ptr, 1e-6, emb.ptr, E,
                          tokens, DEC_POS0, x.ptr, logits.ptr, 1, reps, reg, C.byref(wall))
        if rc != 0:
            raise RuntimeError(f"klb_tokens failed ({rc}): {layer_lib().kore_layer_last_error(L._h).decode()}")

    if warmup:
        run(warmup)
    print(f"[bench] token: {tokens} timed 7B tokens at positions {DEC_POS0}..", file=sys.stderr, flush=True)
    run(1, C.byref(region))
    res = dict(region_ms=region.value, wall_ms=wall.value, tokens=tokens)
    L.close()
    for b in bufs + [emb, x, logits]:
        b.free()
    attn.close()
    return res


PROMPT_NB = 64   # kore's KORE_BMAX rows per forward_batch() call (kore.cpp:690)


def gpu_prompt(qt, chunks: int, warmup: int):
    """A 7B prompt prefill as kore's forward_batch() runs it (kore.cpp:1486-1598)
    in 64-token chunks at positions 0, 64, ..: per chunk 28 layers through
    kore_layer_prefill_dev (rmsnorm rows, q/k/v matmul + bias, RoPE + append +
    causal attention, Wo + residual, rmsnorm rows, gate/up matmul, SwiGLU, down
    + residual), and after the prompt's last chunk its last row's logits (kore's
    prompt loop asks for logits on the last chunk only, kore.cpp:1727-1733),
    driven from C++."""
    from kore_amd import KoreAttn, hip
    from kore_amd.layer import Layer
    from kore_amd.layer import lib as layer_lib
    B = _klb()
    _, tensors, _ = qt
    rng = np.random.default_rng(QMV_SEED + 3)
    n_tok = chunks * PROMPT_NB
    attn = KoreAttn(NL, n_tok, NH, NKV, HD, ROPE_BASE)
    warr, out_norm, bufs = _engine_weights(qt, rng)
    emb = hip.DeviceBuffer.from_array(np.stack([_act(rng, E) for _ in range(n_tok)]))
    x, logits = hip.DeviceBuffer(PROMPT_NB * E), hip.DeviceBuffer(QMV_VOCAB)
    L = Layer(E, QMV_FF, NH, NKV, 1e-6)
    region, wall = C.c_float(0), C.c_double(0)

    def run(reps, reg=None):
        rc = B.klb_prefill(L._h, warr, NL, attn.handle, tensors[7 * NL].handle, out_norm.ptr, 1e-6, emb.ptr, E,
                           PROMPT_NB, chunks, x.ptr, logits.ptr, reps, reg, C.byref(wall))
        if rc != 0:
            raise RuntimeError(f"klb_prefill failed ({rc}): {layer_lib().kore_layer_last_error(L._h).decode()}")

    if warmup:
        run(warmup)
    print(f"[bench] prompt: {n_tok} timed 7B prompt tokens in {chunks} chunks", file=sys.stderr, flush=True)
    run(1, C.byref(region))
    res = dict(region_ms=region.value, wall_ms=wall.value, chunks=chunks, tokens=n_tok)
    L.close()
    for b in bufs + [emb, x, logits]:
        b.free()
    attn.close()
    return res


def prompt_report(p, mats):
    """Matmul flops per chunk: 2 * 64 * rows * cols over the 28 layers' seven
    matrices (attention and the logits matvec not counted)."""
    layer_mats = [m for m in mats if not m[0].startswith("output")]
    flops = sum(2 * PROMPT_NB * r * c for _, _, r, c in layer_mats)
    s_chunk = p["region_ms"] / 1e3 / p["chunks"]
    return {
        "workload": f"Qwen2.5-7B-shape prompt prefill as kore's forward_batch() runs it: {p['tokens']} tokens in "
                    f"{p['chunks']} chunks of 64 at positions 0, 64, .. (28 layers: rmsnorm rows, q/k/v batched "
                    "matmul + bias, RoPE + append + causal attention, Wo + residual, rmsnorm rows, gate/up matmul, "
                    "SwiGLU, down + residual; after the prompt's last chunk its last row's logits, as kore's "
                    "prompt loop asks for them), synthetic Q4_K/Q6_K weights",
        "ms_per_chunk_gpu": round(s_chunk * 1e3, 3),
        "ms_per_chunk_wall": round(p["wall_ms"] / p["chunks"], 3),
        "tokens_per_s": round(PROMPT_NB / s_chunk, 1),
        "matmul_flop_per_chunk": flops,
        "matmul_tflops_effective": round(flops / s_chunk / 1e12, 2),
    }


def cpu_prompt(seconds: float, threads: int):
    """kore's own forward_batch() (oracle/_ref/kore_layer_ref --time-batch, built
    from kore.cpp) on the synthetic 7B engine, 64-token chunks."""
    import subprocess

    import oracle
    if not os.path.exists(oracle.REF_LAYER_BIN):
        return None
    r = subprocess.run([oracle.REF_LAYER_BIN, "--time-batch", str(threads), str(seconds / CPU_RUNS), str(CPU_RUNS)],
                       capture_output=True, text=True, check=True, timeout=seconds + 300)
    j = json.loads(r.stdout)
    st = _runs([64 * c / t for c, t in zip(j["run_chunks"], j["run_seconds"])], "tokens/s")
    return {"value": round(st["median"], 3), "unit": "tokens/s", "cores": j["threads"], "kind": "reference",
            "best": round(st["best"], 3), "runs": st["runs"], "threads": j["threads"], "host": _host(),
            "sample": f"kore's own forward_batch() (kore.cpp:1486-1598, matmul_batch_float with AVX2: "
                      f"{bool(j['avx2'])}) built from kore.cpp with kore's flags, {j['threads']} threads, on a "
                      f"synthetic Qwen2.5-7B-shape engine: {j['chunks']} chunks of 64 tokens at positions 0..511 "
                      f"in turn (logits after the 8-chunk prompt's last chunk, as kore's prompt loop asks for them) "
                      f"in {j['seconds']:.1f} s over {CPU_RUNS} timed runs (after one warm-up chunk; value = median run, "
                      f"best = fastest run); host {_cpu_model()}"}


def token_report(t, mats):
    wbytes = sum(qmv_weight_bytes(tp, r, c) for _, tp, r, c in mats)
    kv = sum(2 * (DEC_POS0 + i + 1) * KVD * 4 * NL for i in range(t["tokens"])) / t["tokens"]
    s_tok = t["region_ms"] / 1e3 / t["tokens"]
    return {
        "workload": "Qwen2.5-7B-shape decode tokens as kore's forward() with logits runs them: embedding row in, "
                    "28 layers (rmsnorm + Q8_K + q/k/v + bias in one launch, RoPE + append + attention, Wo + "
                    "residual, rmsnorm + Q8_K + gate/up, SwiGLU + Q8_K + down + residual) and the output head "
                    "(rmsnorm + Q8_K + 152064-row Q6_K matvec); 4.37 GB of synthetic Q4_K/Q6_K weights, fp32 KV "
                    f"cache filled to {DEC_POS0}, {t['tokens']} tokens at positions {DEC_POS0}.., kore's AVX2 "
                    "matvec order",
        "ms_per_token_gpu": round(s_tok * 1e3, 4),
        "ms_per_token_wall": round(t["wall_ms"] / t["tokens"], 4),
        "tokens_per_s": round(1.0 / s_tok, 1),
        "weight_bytes_per_token": wbytes,
        "kv_bytes_per_token": int(kv),
        "gbs": round((wbytes + kv) / s_tok / 1e9, 1),
        "frac_of_hbm_peak": round((wbytes + kv) / s_tok / 1e9 / HBM_PEAK_GBS, 4),
    }


def cpu_token(seconds: float, threads: int):
    """kore's own forward() with logits (oracle/_ref/kore_layer_ref --time, built
    from kore.cpp) on a synthetic 7B engine at position 4096."""
    import subprocess

    import oracle
    if not os.path.exists(oracle.REF_LAYER_BIN):
        return None
    r = subprocess.run([oracle.REF_LAYER_BIN, "--time", str(threads), str(seconds / CPU_RUNS), str(DEC_POS0),
                        str(CPU_RUNS)], capture_output=True, text=True, check=True, timeout=seconds + 300)
    j = json.loads(r.stdout)
    st = _runs([n / t for n, t in zip(j["run_tokens"], j["run_seconds"])], "tokens/s")
    return {"value": round(st["median"], 3), "unit": "tokens/s", "cores": j["threads"], "kind": "reference",
            "best": round(st["best"], 3), "runs": st["runs"], "threads": j["threads"], "host": _host(),
            "sample": f"kore's own forward() with logits (kore.cpp:1397-1484, AVX2 matvecs: {bool(j['avx2'])}, "
                      f"attention on one thread as in kore) built from kore.cpp with kore's flags, {j['threads']} "
                      f"threads, on a synthetic Qwen2.5-7B-shape engine at positions {j['pos']}..: {j['tokens']} "
                      f"tokens in {j['seconds']:.1f} s over {CPU_RUNS} timed runs (value = median run, best = fastest run); "
                      f"host {_cpu_model()}"}


def kore_token_dropin(seconds: float, threads: int):
    """kore's own forward() with logits with the attention drop-in linked in
    (oracle/_ref/kore_layer_gpu --time: kore.cpp with INTEGRATION.md's binding
    applied, kore_attn_decode per layer through the host-pointer entry point,
    kore's matvecs on the host threads) on the same synthetic 7B engine."""
    import subprocess

    import oracle
    if not os.path.exists(oracle.REF_LAYER_GPU_BIN):
        return None
    r = subprocess.run([oracle.REF_LAYER_GPU_BIN, "--time", str(threads), str(seconds / CPU_RUNS), str(DEC_POS0),
                        str(CPU_RUNS)], capture_output=True, text=True, check=True, timeout=seconds + 300)
    j = json.loads(r.stdout)
    st = _runs([n / t for n, t in zip(j["run_tokens"], j["run_seconds"])], "tokens/s")
    return {"value": round(st["median"], 3), "unit": "tokens/s", "threads": j["threads"], "best": round(st["best"], 3),
            "runs": st["runs"],
            "sample": f"kore's own forward() with logits, built from kore.cpp with the attention binding of "
                      f"INTEGRATION.md applied (RoPE, KV cache and attention through kore_attn_decode, host "
                      f"buffers in and out per layer) and linked to libkore_attn.so; matvecs on {j['threads']} host "
                      f"threads (AVX2: {bool(j['avx2'])}); same synthetic Qwen2.5-7B-shape engine at positions "
                      f"{j['pos']}..: {j['tokens']} tokens in {j['seconds']:.1f} s over {CPU_RUNS} timed runs "
                      f"(value = median run)"}


def gemm_report(g, chunks: int):
    mats, op_mats = g["mats"], g["op_mats"]
    flops = sum(2 * GEMM_B * mats[ti][2] * mats[ti][3] for ts in op_mats for ti in ts)
    chunk_s = g["region_ms"] / 1e3 / chunks
    per = {}
    for ts in op_mats:
        key = _gemm_key(mats, ts)
        d = per.setdefault(key, {"launches_per_chunk": 0, "ms": g["class_ms"][key],
                                 "flop": sum(2 * GEMM_B * mats[ti][2] * mats[ti][3] for ti in ts),
                                 "weight_bytes": sum(qmv_weight_bytes(*mats[ti][1:]) for ti in ts)})
        d["launches_per_chunk"] += 1
    # the fp16 path (default) is bound by the fp16 MFMA rate on its MFMA work (the algorithmic
    # flops times the passes); the fp32 path (KORE_GEMM=fp32) by the fp32 MFMA rate
    fp16 = os.environ.get("KORE_GEMM", "") != "fp32"
    table = {}
    for ts in op_mats:
        key = _gemm_key(mats, ts)
        per[key]["mfma_flop"] = sum(2 * GEMM_B * mats[ti][2] * mats[ti][3] * (GEMM16_PASSES[mats[ti][1]] if fp16 else 1)
                                    for ti in ts)
    peak = FP16_MFMA_PEAK_TFLOPS if fp16 else FP32_MFMA_PEAK_TFLOPS
    for key, d in per.items():
        us = float(np.mean(d["ms"])) * 1e3
        tf = d["flop"] / (us / 1e6) / 1e12
        mtf = d["mfma_flop"] / (us / 1e6) / 1e12
        table[key] = {"launches_per_chunk": d["launches_per_chunk"], "us_mean": round(us, 2), "flop": d["flop"],
                      "tflops": round(tf, 2), "mfma_tflops": round(mtf, 2), "frac": round(mtf / peak, 4),
                      "weight_gbs": round(d["weight_bytes"] / (us / 1e6) / 1e9, 1),
                      "us_per_chunk": round(us * d["launches_per_chunk"], 1)}
    dom = max(table, key=lambda k: table[k]["us_per_chunk"])
    return {
        "workload": "Qwen2.5-7B-shape prefill chunk, matmul half: 28 layers x forward_batch's seven "
                    "matmul_batch_float calls (attn_q, attn_k, attn_v, attn_output, ffn_gate, ffn_up, ffn_down) "
                    f"on {GEMM_B} activations at once, q+k+v and gate+up as one grouped launch each (112 launches), "
                    "the same synthetic Q4_K / Q6_K matrices as the matvec leg, activations N(0,1) with 1% x20, "
                    "fp32 out",
        "flop_per_chunk": flops,
        "tokens_per_chunk": GEMM_B,
        "launches_per_chunk": len(op_mats),
        "ms_per_chunk_gpu": round(chunk_s * 1e3, 4),
        "ms_per_chunk_wall": round(g["wall_ms"] / chunks, 4),
        "tflops": round(flops / chunk_s / 1e12, 2),
        "prefill_tokens_per_s_matmuls": round(GEMM_B / chunk_s, 1),
        "chunks": chunks,
        "per_matrix": table,
        "path": "fp16 MFMA (exact integer weights, split activations)" if fp16 else "fp32 MFMA",
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": table[dom]["mfma_tflops"],
                     "peak": peak, "unit": "TFLOP/s", "frac": table[dom]["frac"],
                     "traffic": TRAFFIC_GEMM_BYTES.get(dom) if fp16 else None},
    }


def matvec_report(g, tokens: int):
    mats, op_mats = g["mats"], g["op_mats"]
    wbytes = sum(qmv_weight_bytes(t, r, c) for _, t, r, c in mats)
    tok_s = g["region_ms"] / 1e3 / tokens
    per = {}
    for ts in op_mats:
        alg = sum(qmv_weight_bytes(*mats[ti][1:]) + mats[ti][2] * 4 for ti in ts)
        alg += mats[ts[0]][3] * 4          # the fp32 input, read once
        key = _mv_key(mats, ts)
        d = per.setdefault(key, {"launches_per_token": 0, "ms": g["class_ms"][key], "bytes": alg})
        d["launches_per_token"] += 1
    table = {}
    for key, d in per.items():
        us = float(np.mean(d["ms"])) * 1e3
        gbs = d["bytes"] / (us / 1e6) / 1e9
        table[key] = {"launches_per_token": d["launches_per_token"], "us_mean": round(us, 2),
                      "algorithmic_bytes": d["bytes"], "gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                      "us_per_token": round(us * d["launches_per_token"], 1)}
    dom = max(table, key=lambda k: table[k]["us_per_token"])
    return {
        "workload": "Qwen2.5-7B-shape token, matvec half: 28 layers x (attn_q, attn_k, attn_v, attn_output, "
                    "ffn_gate, ffn_up, ffn_down) + output head = 197 matrices, Q4_K with attn_v/ffn_down in Q6_K on "
                    "14 layers (Q4_K_M's use_more_bits rule) and a Q6_K output head; each preceded by kore's Q8_K "
                    "quantisation of its input; synthetic weights (hashed bytes, finite f16 scales), activations "
                    "N(0,1) with 1% x20; kore's AVX2 summation order; per layer 4 calls: q+k+v and gate+up "
                    "as one grouped launch each",
        "weight_bytes_per_token": wbytes,
        "launches_per_token": len(op_mats),
        "ms_per_token_gpu": round(tok_s * 1e3, 4),
        "ms_per_token_wall": round(g["wall_ms"] / tokens, 4),
        "weight_gbs": round(wbytes / tok_s / 1e9, 1),
        "weight_frac_of_hbm_peak": round(wbytes / tok_s / 1e9 / HBM_PEAK_GBS, 4),
        "tokens": tokens,
        "per_matrix": table,
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": table[dom]["gbs"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": table[dom]["frac"], "traffic": TRAFFIC_MATVEC_BYTES.get(dom)},
    }


def cpu_matvec(seconds: float, threads: int):
    """kore's own quant() + mv() (oracle/_ref/kore_qmv_ref, built from
    kore.cpp) on the 7B ffn_gate shape, cycling over 16 copies so the weights
    come from DRAM; falls back to the oracle's restatement (one thread) where
    that build is absent."""
    import struct
    import subprocess
    import tempfile

    import oracle
    rows, cols = QMV_FF, E
    rng = np.random.default_rng(5)
    w = rng.integers(0, 256, size=(rows, cols // 256, 144), dtype=np.uint8)
    w[:, :, 0:2] = np.frombuffer(np.float16(3e-3).tobytes(), np.uint8)
    w[:, :, 2:4] = np.frombuffer(np.float16(1e-3).tobytes(), np.uint8)
    x = rng.standard_normal(cols).astype(np.float32)
    if os.path.exists(oracle.REF_QMV_BIN):
        with tempfile.TemporaryDirectory() as td:
            job = os.path.join(td, "job.bin")
            with open(job, "wb") as f:
                f.write(struct.pack("<3i", QMV_Q4K, rows, cols))
                f.write(w.tobytes())
                f.write(x.tobytes())
            r = subprocess.run([oracle.REF_QMV_BIN, "--time", str(threads), str(seconds / CPU_RUNS), "16", job,
                                str(CPU_RUNS)], capture_output=True, text=True, check=True, timeout=seconds + 300)
        j = json.loads(r.stdout)
        st = _runs([j["weight_bytes"] * n / t / 1e9 for n, t in zip(j["run_reps"], j["run_seconds"])], "GB/s")
        return {"value": round(st["median"], 2), "unit": "GB/s", "cores": j["threads"], "kind": "reference",
                "best": round(st["best"], 2), "runs": st["runs"], "threads": j["threads"], "host": _host(),
                "sample": f"kore's own quantize_row_q8_K + matvec_mt (kore.cpp:422-446, 677-682, AVX2 dot "
                          f"products: {bool(j['avx2'])}) built from kore.cpp with kore's flags, {j['threads']} "
                          f"threads, on the 7B ffn_gate shape ({rows} x {cols} Q4_K, 38.2 MB) cycling over 16 "
                          f"copies: {j['reps']} matvecs in {j['seconds']:.1f} s over {CPU_RUNS} timed runs (value = median "
                          f"run, best = fastest run); host {_cpu_model()}"}
    xq = oracle.quantize_q8K(x)
    t0, n = time.perf_counter(), 0
    while time.perf_counter() - t0 < seconds:
        oracle.qmatvec(QMV_Q4K, w, rows, cols, xq, avx2=True)
        n += 1
    el = time.perf_counter() - t0
    return {"value": round(w.size * n / el / 1e9, 2), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"the oracle's restatement of kore's AVX2 Q4_K dot product, one thread, 7B ffn_gate "
                      f"shape, {n} matvecs in {el:.1f} s; host {_cpu_model()}"}


def cpu_gemm(seconds: float, threads: int):
    """kore's own matmul_batch_float (oracle/_ref/kore_qmv_ref --time-batch,
    built from kore.cpp) on the 7B ffn_gate shape with 64 activations; falls
    back to the oracle's restatement (one thread) where that build is absent."""
    import struct
    import subprocess
    import tempfile

    import oracle
    rows, cols = QMV_FF, E
    rng = np.random.default_rng(6)
    w = rng.integers(0, 256, size=(rows, cols // 256, 144), dtype=np.uint8)
    w[:, :, 0:2] = np.frombuffer(np.float16(3e-3).tobytes(), np.uint8)
    w[:, :, 2:4] = np.frombuffer(np.float16(1e-3).tobytes(), np.uint8)
    x = rng.standard_normal((GEMM_B, cols)).astype(np.float32)
    flop = 2 * GEMM_B * rows * cols
    if os.path.exists(oracle.REF_QMV_BIN):
        with tempfile.TemporaryDirectory() as td:
            job = os.path.join(td, "job.bin")
            with open(job, "wb") as f:
                f.write(struct.pack("<4i", QMV_Q4K, rows, cols, GEMM_B))
                f.write(w.tobytes())
                f.write(x.tobytes())
            r = subprocess.run([oracle.REF_QMV_BIN, "--time-batch", str(threads), str(seconds / CPU_RUNS), job,
                                str(CPU_RUNS)], capture_output=True, text=True, check=True, timeout=seconds + 300)
        j = json.loads(r.stdout)
        st = _runs([flop * n / t / 1e12 for n, t in zip(j["run_reps"], j["run_seconds"])], "TFLOP/s")
        return {"value": round(st["median"], 5), "unit": "TFLOP/s", "cores": j["threads"], "kind": "reference",
                "best": round(st["best"], 5), "runs": st["runs"], "threads": j["threads"], "host": _host(),
                "sample": f"kore's own matmul_batch_float (kore.cpp:783-845, AVX2 path: {bool(j['avx2'])}) built "
                          f"from kore.cpp with kore's flags, {j['threads']} threads, on the 7B ffn_gate shape "
                          f"({rows} x {cols} Q4_K) with {GEMM_B} activations: {j['reps']} calls in "
                          f"{j['seconds']:.1f} s over {CPU_RUNS} timed runs (value = median run, best = fastest run); host "
                          f"{_cpu_model()}"}
    t0, n = time.perf_counter(), 0
    while time.perf_counter() - t0 < seconds:
        oracle.matmul_batch(QMV_Q4K, w.reshape(-1), rows, cols, x[:8], avx2=True)
        n += 1
    el = time.perf_counter() - t0
    return {"value": round(2 * 8 * rows * cols * n / el / 1e12, 5), "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"the oracle's restatement of kore's AVX2 matmul_batch_float, one thread, 7B ffn_gate "
                      f"shape, 8 activations, {n} calls in {el:.1f} s; host {_cpu_model()}"}


def read_calibration():
    """What one launch of a plain streaming read (kore_hbm_probe.hip) moves per
    size on this device, and the time of an empty dependent launch."""
    from kore_amd import hip, qmv
    qmv.lib()
    B = C.CDLL(os.path.join(ROOT, "kore_amd", "libkore_qmv_bench.so"))
    B.kqb_read_probe.argtypes = [C.c_void_p, C.c_int64, C.c_int, C.c_int, C.c_int, C.c_void_p,
                                 C.POINTER(C.c_float)]
    total = 4 << 30
    buf = hip.DeviceBuffer(total // 4)
    hip.check(hip.lib().hipMemset(buf.ptr, 1, total), "hipMemset")
    sink = hip.DeviceBuffer(8192 * 256)
    out = {"kernel": "grid-stride read of 16-byte chunks, 4 loads in flight per thread, 256 threads per "
                     "workgroup; launches back to back on one stream, buffer copies rotated",
           "sizes": []}
    us = C.c_float(0)
    for mb in (8, 17, 38, 76, 150, 447, 1024, 4096):
        nbytes = mb << 20
        # enough copies that one rotation covers 1 GiB, four times the 256 MB MALL:
        # no launch finds its bytes in the memory-side cache
        rot = max(1, min(total // nbytes, max(8, -(-(1 << 30) // nbytes))))
        row = {"mbytes": mb}
        for grid in (1024, 2048, 4096):
            reps = 10 if mb >= 1024 else 100
            rc = B.kqb_read_probe(buf.ptr, nbytes, rot, grid, reps, sink.ptr, C.byref(us))
            if rc != 0:
                raise RuntimeError(f"kqb_read_probe failed ({rc})")
            row[f"grid{grid}"] = {"us": round(us.value, 2), "gbs": round(nbytes / (us.value * 1e-6) / 1e9, 1)}
        out["sizes"].append(row)
        print(f"[bench] read calibration {mb} MB done", file=sys.stderr, flush=True)
    rc = B.kqb_read_probe(buf.ptr, 16, 1, 0, 1000, sink.ptr, C.byref(us))
    if rc != 0:
        raise RuntimeError(f"kqb_read_probe failed ({rc})")
    out["empty_launch_us"] = round(us.value, 3)
    buf.free()
    sink.free()
    return out


def decode_floor(nbytes: int, rounds: int):
    """What the device allows for the decode layer's launch pattern, measured
    in the same run: each round one launch that reads the layer's algorithmic
    bytes once (every load issued up front; 1, 2, 4 or 8 16-byte loads per
    thread, the fastest kept) and one dependent empty launch, back to back,
    over NL rotated buffers as the decode rotates its layers (NL x 17 MB, more
    than the 256 MB MALL).  Also the read launches alone."""
    from kore_amd import hip, qmv
    qmv.lib()
    B = C.CDLL(os.path.join(ROOT, "kore_amd", "libkore_qmv_bench.so"))
    B.kqb_floor_probe.argtypes = [C.c_void_p, C.c_int64, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p,
                                  C.POINTER(C.c_float)]
    nb = (int(nbytes) + 15) // 16 * 16
    buf = hip.DeviceBuffer(nb * NL // 4)
    hip.check(hip.lib().hipMemset(buf.ptr, 1, nb * NL), "hipMemset")
    sink = hip.DeviceBuffer(nb // 16 + 256)
    us = C.c_float(0)
    out = {}
    for with_launch, key in ((1, "read_plus_dependent_launch_us"), (0, "read_only_us")):
        per_us = {}
        for per in (1, 2, 4, 8):
            rc = B.kqb_floor_probe(buf.ptr, nb, NL, per, with_launch, rounds, sink.ptr, C.byref(us))
            if rc != 0:
                raise RuntimeError(f"kqb_floor_probe failed ({rc})")
            per_us[per] = round(us.value, 3)
        best = min(per_us, key=per_us.get)
        out[key] = per_us[best]
        out[key.replace("_us", "_loads_per_thread")] = best
    buf.free()
    sink.free()
    out["bytes"] = nb
    out["rounds"] = rounds
    return out


# ------------------------------------------------------------------ CPU legs

def _rel_err(out, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(out, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


CPU_RUNS = 3   # timed runs of every CPU baseline: median and best are reported (kore_kernels.cpp:706-714)


def _runs(rates, unit):
    """Median and best of the per-run rates (higher is better)."""
    r = [float(x) for x in rates]
    return {"median": float(np.median(r)), "best": max(r), "runs": [round(x, 6) for x in r], "unit": unit}


def _host():
    try:
        aff = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        aff = os.cpu_count()
    flags = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    flags = line
                    break
    except OSError:
        pass
    return {"cpu_model": _cpu_model(), "nproc": os.cpu_count(), "cpus_allowed": aff,
            "avx2": " avx2" in flags, "fma": " fma" in flags}


def _pool(fn, items, threads):
    from concurrent.futures import ThreadPoolExecutor
    with ThreadPoolExecutor(max_workers=max(1, threads)) as ex:
        return list(ex.map(fn, items))


def decode_parity(gpu_outs, gpu_attn, threads: int, n_layers: int = NL, n_steps: int = DEC_STEPS):
    """All 128 configured steps x 28 layers of the 7B decode (positions
    4096..4223, cache rows 0..4095 filled through the append path) against
    the oracle - kore's scalar decode, bit-identical to kore (kore.cpp:1405-1455)
    - and against a float64 evaluation of the same attention over the same
    fp32 roped rows (oracle ko_attn_ref64), which splits the GPU-to-kore
    difference into the GPU's own error and kore's.  The layers are
    independent, so they run on `threads` host threads (the oracle's C calls
    release the GIL).  The GPU's cache rows of every layer are compared bit
    for bit with the oracle's."""
    import oracle
    inv_f = oracle.inv_freq(HD, ROPE_BASE)
    n_pos = DEC_POS0 + n_steps
    kv_gpu = [gpu_attn.read_kv(l, 0, n_pos) for l in range(n_layers)]   # one caller per handle

    def layer(l):
        k_all = oracle.synth(n_pos, KVD, DEC_SEED, k_stream(l), 0, 2, DEC_PER_MILLE, DEC_OUTLIER)
        v_all = oracle.synth(n_pos, KVD, DEC_SEED, v_stream(l), 0, 3, DEC_PER_MILLE, DEC_OUTLIER)
        q_all = oracle.synth(n_steps, E, DEC_SEED, q_stream(l), DEC_POS0, 1, DEC_PER_MILLE, DEC_OUTLIER)
        kc = oracle.rope_rows(k_all, np.arange(n_pos), NKV, HD, inv_f)
        kv_ok = bool(np.array_equal(kc, kv_gpu[l][0]) and np.array_equal(v_all, kv_gpu[l][1]))
        qr = oracle.rope_rows(q_all, np.arange(DEC_POS0, n_pos), NH, HD, inv_f)
        e_gk, e_ge, e_ke = [], [], []
        for st in range(n_steps):
            pos = DEC_POS0 + st
            ref = oracle.attn_decode(qr[st], kc[:pos + 1], v_all[:pos + 1], pos, NH, NKV, HD)
            ex = oracle.attn_ref64(qr[st], kc, v_all, np.arange(pos + 1), NH, NKV, HD)
            g = gpu_outs[st, l]
            e_gk.append(_rel_err(g, ref))
            e_ge.append(_rel_err(g, ex))
            e_ke.append(_rel_err(ref, ex))
        return kv_ok, e_gk, e_ge, e_ke

    t0 = time.perf_counter()
    res = _pool(layer, range(n_layers), threads)
    gk = np.array([r[1] for r in res])   # [layer][step]
    ge = np.array([r[2] for r in res])
    ke = np.array([r[3] for r in res])
    worst = np.unravel_index(int(np.argmax(gk)), gk.shape)
    return {
        "decode_steps_compared": n_steps, "decode_layers_compared": n_layers,
        "decode_max_rel_err": float(gk.max()),
        "decode_max_rel_err_at": {"step": int(worst[1]), "position": DEC_POS0 + int(worst[1]), "layer": int(worst[0])},
        "decode_step_max_rel_err": [float(f"{x:.3g}") for x in gk.max(axis=0)],
        "decode_kv_bitwise": all(r[0] for r in res),
        "decode_error_budget": {
            "gpu_vs_float64_max": float(ge.max()), "kore_vs_float64_max": float(ke.max()),
            "gpu_vs_float64_mean": float(ge.mean()), "kore_vs_float64_mean": float(ke.mean()),
            "note": "max|d|/max|ref| per (step, layer) against a float64 evaluation over the same fp32 roped "
                    "q and cache rows (oracle ko_attn_ref64)"},
        "decode_parity_seconds": round(time.perf_counter() - t0, 2), "decode_parity_threads": threads,
    }


def cpu_decode(seconds: float):
    """The oracle's decode (kore.cpp:1405-1455, scalar, one thread as kore's
    attention runs) timed on this host: CPU_RUNS runs of at least
    seconds / CPU_RUNS each, every run decoding position 4096 (4097 rows
    attended) of the same workload layer after layer (re-decoding a position
    rewrites the same cache row with the same data, so every call does the
    same work)."""
    import oracle
    kv = oracle.KV(NL, DEC_POS0 + 1, NH, NKV, HD, ROPE_BASE)
    inv_f = oracle.inv_freq(HD, ROPE_BASE)
    kc, vc = kv.kcache(), kv.vcache()
    ins = []
    for l in range(NL):
        k0 = oracle.synth(DEC_POS0, KVD, DEC_SEED, k_stream(l), 0, 2, DEC_PER_MILLE, DEC_OUTLIER)
        kc[l, :DEC_POS0] = oracle.rope_rows(k0, np.arange(DEC_POS0), NKV, HD, inv_f)
        vc[l, :DEC_POS0] = oracle.synth(DEC_POS0, KVD, DEC_SEED, v_stream(l), 0, 3, DEC_PER_MILLE, DEC_OUTLIER)
        ins.append(tuple(oracle.synth(1, d, DEC_SEED, st(l), DEC_POS0, t, DEC_PER_MILLE, DEC_OUTLIER)[0]
                         for d, st, t in ((E, q_stream, 1), (KVD, k_stream, 2), (KVD, v_stream, 3))))
    per_call = []
    for _ in range(CPU_RUNS):
        n, t0 = 0, time.perf_counter()
        while True:
            l = n % NL
            kv.decode(l, DEC_POS0, *ins[l])
            n += 1
            el = time.perf_counter() - t0
            if n >= NL and el >= seconds / CPU_RUNS:
                break
        per_call.append(el / n)
    kv.close()
    b = decode_bytes(DEC_POS0 + 1)
    gbs = _runs([b / t / 1e9 for t in per_call], "GB/s")
    return dict(gbs=gbs, us_per_layer=[t * 1e6 for t in per_call])


def cpu_prefill(gpu_outs=None):
    """The oracle's batched causal attention (kore.cpp:1503-1563 with the AVX2
    hd_dot/hd_fma arithmetic, one thread) on whole 2048-row layers of the same
    workload: CPU_RUNS runs of one layer each (layers 0, 1, ..), each compared
    with the GPU's rows of that layer."""
    import oracle
    kv = oracle.KV(CPU_RUNS, PF_N, NH, NKV, HD, ROPE_BASE)
    t, err = [], 0.0
    for l in range(CPU_RUNS):
        q = oracle.synth(PF_N, E, PF_SEED, q_stream(l), 0, 1)
        k = oracle.synth(PF_N, KVD, PF_SEED, k_stream(l), 0, 2)
        v = oracle.synth(PF_N, KVD, PF_SEED, v_stream(l), 0, 3)
        t0 = time.perf_counter()
        ref = kv.prefill(l, 0, q, k, v, avx2=True)
        t.append(time.perf_counter() - t0)
        if gpu_outs is not None and l < gpu_outs.shape[0]:
            err = max(err, _rel_err(gpu_outs[l], ref))
    kv.close()
    F = prefill_flops(0, PF_N)
    return dict(tflops=_runs([F / x / 1e12 for x in t], "TFLOP/s"), seconds=float(sum(t)), max_rel_err=err)


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ---------------------------------------------------------------------- main

def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128, help="timed decode steps (tokens), 28 layers each")
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prefill-steps", type=int, default=3, help="timed 28-layer prefill passes")
    ap.add_argument("--prefill-warmup", type=int, default=1)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--prefill-only", action="store_true",
                    help="run only the 7B 2048-row prefill leg (for profiling its kernels on their own)")
    ap.add_argument("--decode-only", action="store_true",
                    help="run only the 7B decode leg, without the parity pass or any CPU work (for profiling)")
    ap.add_argument("--no-other", action="store_true", help="skip the 0.5B / 3B / 1.5B workloads")
    ap.add_argument("--cpu-seconds", type=float, default=9.0,
                    help="time of each CPU baseline, split over its timed runs")
    ap.add_argument("--no-matvec", action="store_true", help="skip the 7B-token matvec leg")
    ap.add_argument("--matvec-only", action="store_true", help="run only the matvec leg (for profiling)")
    ap.add_argument("--matvec-tokens", type=int, default=10, help="timed 7B tokens of the matvec leg")
    ap.add_argument("--matvec-warmup", type=int, default=2)
    ap.add_argument("--no-gemm", action="store_true", help="skip the 7B prefill-chunk batched matmul leg")
    ap.add_argument("--gemm-only", action="store_true", help="run only the batched matmul leg (for profiling)")
    ap.add_argument("--gemm-chunks", type=int, default=5, help="timed 64-token chunks of the batched matmul leg")
    ap.add_argument("--gemm-warmup", type=int, default=1)
    ap.add_argument("--no-token", action="store_true", help="skip the whole-token decode leg")
    ap.add_argument("--token-only", action="store_true", help="run only the whole-token decode leg")
    ap.add_argument("--token-count", type=int, default=32, help="timed 7B decode tokens of the whole-token leg")
    ap.add_argument("--no-prompt", action="store_true", help="skip the whole-prompt prefill leg")
    ap.add_argument("--prompt-only", action="store_true", help="run only the whole-prompt prefill leg")
    ap.add_argument("--prompt-chunks", type=int, default=8, help="64-token chunks of the whole-prompt leg")
    ap.add_argument("--cpu-threads", type=int, default=16,
                    help="threads of kore's own matvec in the CPU baseline (the GPU box's CPU share)")
    ap.add_argument("--decode-timeline", action="store_true",
                    help="only run the decode workload on the timing build (libkore_attn_tl.so) and report "
                         "per-wave s_memrealtime stamps of the last layer's kernels")
    ap.add_argument("--timeline-config", default="7b", choices=("7b", "3b"),
                    help="with --decode-timeline: the 7B decode at 4096.. (default) or the 3B decode at 32767")
    ap.add_argument("--timeline-raw", default="", help="with --decode-timeline: also save every stamp (us) "
                                                            "to this .npz file")
    ap.add_argument("--decode-sweep", action="store_true",
                    help="only time the 7B and 3B decode at positions across the context (32768 slots)")
    ap.add_argument("--read-calibration", action="store_true",
                    help="only time a plain streaming read kernel per launch size (the yardstick of the "
                         "HBM-bound kernels) and an empty launch")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 8 device-to-device copies of 256 MiB (the runtime's copy kernel), "
                         "the known-size reference for HBM byte counters")
    args = ap.parse_args(argv)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}): the "
              "attention path runs on a single MI355X and has no multi-GPU leg.", file=sys.stderr)
        return 2
    if args.steps < 1 or args.steps + DEC_POS0 > DEC_CTX or args.warmup > args.steps:
        print("--steps must be in 1..4096 and --warmup <= --steps", file=sys.stderr)
        return 2

    if args.decode_timeline:
        from kore_amd import _lib
        _lib.LIB_PATH = os.path.join(ROOT, "kore_amd", "libkore_attn_tl.so")
    from kore_amd import hip
    if args.copy_calibration:
        n = 64 << 20   # floats: 256 MiB
        src, dst = hip.DeviceBuffer(n), hip.DeviceBuffer(n)
        for _ in range(8):
            hip.check(hip.lib().hipMemcpy(dst.ptr, src.ptr, n * 4, hip.D2D), "hipMemcpy D2D")
        hip.synchronize()
        print(json.dumps({"copy_calibration_bytes": n * 4, "copies": 8}), flush=True)
        return 0
    if args.read_calibration:
        print(json.dumps(read_calibration()), flush=True)
        return 0
    dev_name = hip.device_name(0)
    clk = C.c_int(0)
    hip.lib().hipDeviceGetAttribute(C.byref(clk), 5, 0)   # hipDeviceAttributeClockRate (kHz)

    if args.matvec_only or args.gemm_only or args.token_only or args.prompt_only:
        qt = qmv_tensors()
        if args.prompt_only:
            out = {"prompt": prompt_report(gpu_prompt(qt, args.prompt_chunks, 1), qt[0])}
        elif args.token_only:
            out = {"token": token_report(gpu_token(qt, args.token_count, 1), qt[0])}
        elif args.matvec_only:
            out = {"matvec": matvec_report(gpu_matvec(qt, args.matvec_tokens, args.matvec_warmup),
                                           args.matvec_tokens)}
        else:
            out = {"gemm": gemm_report(gpu_gemm(qt, args.gemm_chunks, args.gemm_warmup), args.gemm_chunks)}
        for m in qt[1]:
            m.close()
        print(json.dumps(out), flush=True)
        return 0
    if args.prefill_only:
        pf = gpu_prefill(args.prefill_steps, args.prefill_warmup)
        F = prefill_flops(0, PF_N)
        per = pf["region_ms"] / 1e3 / (args.prefill_steps * NL)
        print(json.dumps({"prefill": {"us_per_layer_gpu": round(per * 1e6, 2), "flop_per_layer": F,
                                      "tflops": round(F / per / 1e12, 3),
                                      "frac": round(F / per / 1e12 / FP32_MFMA_PEAK_TFLOPS, 4)}}), flush=True)
        return 0
    if args.decode_sweep:
        print(json.dumps({"decode_sweep": decode_sweep()}), flush=True)
        return 0
    if args.decode_timeline:
        print(json.dumps({"decode_timeline": decode_timeline(args.steps, args.timeline_raw,
                                                             config=args.timeline_config)}), flush=True)
        return 0
    if args.decode_only:
        dec = gpu_decode(args.steps, args.warmup, extras=False)
        per = dec["region_ms"] / 1e3 / (args.steps * NL)
        nbytes = sum(decode_bytes(DEC_POS0 + s + 1) for s in range(args.steps)) / args.steps
        dec["attn"].close()
        floor = decode_floor(nbytes, max(args.steps * NL, 64 * NL))
        print(json.dumps({"decode": {"us_per_layer_gpu": round(per * 1e6, 3), "bytes_per_layer": int(nbytes),
                                     "gbs": round(nbytes / per / 1e9, 1), "floor_us": floor["read_plus_dependent_launch_us"],
                                     "layer_over_floor": round(per * 1e6 / floor["read_plus_dependent_launch_us"],
                                                               3)}}), flush=True)
        return 0
    pf = None
    if not args.no_prefill:
        pf = gpu_prefill(args.prefill_steps, args.prefill_warmup)
    dec = gpu_decode(args.steps, args.warmup)
    mean_bytes = sum(decode_bytes(DEC_POS0 + s + 1) for s in range(args.steps)) / args.steps
    print("[bench] decode floor: read of the layer's bytes + one dependent launch", file=sys.stderr, flush=True)
    floor = decode_floor(mean_bytes, max(args.steps * NL, 64 * NL))
    other, other_par = (None, {}) if args.no_other else gpu_other_workloads(
        quick=args.steps < 64, parity_threads=0 if args.no_cpu else args.cpu_threads)
    qt = None if (args.no_matvec and args.no_gemm) else qmv_tensors()
    mv = None if args.no_matvec else gpu_matvec(qt, args.matvec_tokens, args.matvec_warmup)
    gm = None if args.no_gemm else gpu_gemm(qt, args.gemm_chunks, args.gemm_warmup)
    tk = None if (args.no_token or qt is None) else gpu_token(qt, args.token_count, 1)
    pr = None if (args.no_prompt or qt is None) else gpu_prompt(qt, args.prompt_chunks, 1)
    if qt is not None:
        for m in qt[1]:
            m.close()

    K, W = args.steps, args.warmup
    total_bytes = sum(decode_bytes(DEC_POS0 + s + 1) for s in range(K)) * NL
    wall_s = dec["wall_ms"] / 1e3
    value = total_bytes / wall_s / 1e9
    lm = dec["launch_ms"].astype(np.float64)
    # GPU time per launch: the HIP event pair around the timed region over the
    # K * NL launches (split + combine kernel of every layer, gaps included)
    mean_launch_s = dec["region_ms"] / 1e3 / (K * NL)
    bytes_per_launch = total_bytes / (K * NL)
    achieved = bytes_per_launch / mean_launch_s / 1e9
    res = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(dec["wall_ms"] / K, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "Qwen2.5-7B-shape decode attention, batch 1, 28 layers, fp32 KV cache ctx 8192 "
                        f"filled to {DEC_POS0}, {K} steps at positions {DEC_POS0}..{DEC_POS0 + K - 1}, "
                        "inputs N(0,1) with 1% of channels x20",
            "n_layer": NL, "n_head": NH, "n_head_kv": NKV, "head_dim": HD, "ctx": DEC_CTX,
            "pos_first": DEC_POS0, "rope_base": ROPE_BASE,
        },
        "decode": {
            "us_per_layer_gpu": round(mean_launch_s * 1e6, 3),
            "us_per_layer_wall": round(dec["wall_ms"] / (K * NL) * 1e3, 3),
            "warmup_steps_run": dec["warm_steps"], "warmup_seconds": round(dec["warm_s"], 3),
            "floor": dict(floor, layer_over_floor=round(mean_launch_s * 1e6 / floor["read_plus_dependent_launch_us"], 3),
                          note="same run: one launch reading the layer's mean algorithmic bytes once plus one "
                               "dependent empty launch per round, 28 rotated buffers; the decode layer's time over it"),
            "launch_us_events": {k: round(v * 1e3, 3) for k, v in _stats(lm).items()},
            "bytes_per_launch_mean": int(bytes_per_launch),
            "host_pointer_us_per_layer": round(dec["host_us_per_layer"], 3),
            "host_pointer_note": f"kore_attn_decode (the synchronous host-pointer call kore's forward() would make: "
                                 f"H2D of q/k/v, the kernels, D2H of the output) per layer over {dec['host_steps']} "
                                 "steps x 28 layers, steady_clock; PCIe-inclusive, not the value",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": TRAFFIC_DECODE_BYTES,
        },
        "device": {"name": dev_name, "num_cu": dec["num_cu"], "clock_mhz": clk.value // 1000},
    }
    if pf is not None:
        P = args.prefill_steps
        plm = pf["launch_ms"].astype(np.float64)
        F = prefill_flops(0, PF_N)
        p_per_s = pf["region_ms"] / 1e3 / (P * NL)
        p_ach = F / p_per_s / 1e12
        res["prefill"] = {
            "workload": f"Qwen2.5-7B-shape causal prefill attention, {PF_N} rows at position 0, 28 layers, "
                        "inputs N(0,1)",
            "tflops": round(F * NL * P / (pf["wall_ms"] / 1e3) / 1e12, 3),
            "us_per_layer_gpu": round(p_per_s * 1e6, 2),
            "launch_us_events": {k: round(v * 1e3, 2) for k, v in _stats(plm).items()},
            "flop_per_layer": F,
            "steps": P,
            "host_pointer_us_per_layer": round(pf["host_us_per_layer"], 2),
            "host_pointer_equals_device": pf["host_equals_device"],
            "host_pointer_note": f"kore_attn_prefill (the synchronous host-pointer call kore's forward_batch() would "
                                 f"make: H2D of q/k/v, append + attention, D2H of the rows) per layer over "
                                 f"{pf['host_layers']} layers, steady_clock; PCIe-inclusive",
            "roofline": {"bound": "mfma", "achieved": round(p_ach, 3), "peak": FP32_MFMA_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(p_ach / FP32_MFMA_PEAK_TFLOPS, 4),
                         "traffic": TRAFFIC_PREFILL_BYTES},
        }
    if other is not None:
        res["other_workloads"] = other
    if mv is not None:
        res["matvec"] = matvec_report(mv, args.matvec_tokens)
    if gm is not None:
        res["gemm"] = gemm_report(gm, args.gemm_chunks)
    if tk is not None:
        res["token"] = token_report(tk, qt[0])
    if pr is not None:
        res["prompt"] = prompt_report(pr, qt[0])
    if not args.no_cpu:
        print(f"[bench] parity: {DEC_STEPS} decode steps x {NL} layers against the oracle and float64, "
              f"{args.cpu_threads} host threads", file=sys.stderr, flush=True)
        res["parity"] = dict(decode_parity(dec["outs"], dec["attn"], args.cpu_threads), tolerance=1e-4)
        res["parity"].update(other_par)
        print(f"[bench] cpu baseline: decode ({CPU_RUNS} runs, {args.cpu_seconds:.0f} s)", file=sys.stderr, flush=True)
        cd = cpu_decode(args.cpu_seconds)
        host = _host()
        res["cpu_baseline"] = {
            "value": round(cd["gbs"]["median"], 4),
            "unit": "GB/s",
            "cores": 1,
            "kind": "port",
            "best": round(cd["gbs"]["best"], 4),
            "runs": cd["gbs"]["runs"],
            "threads": 1,
            "host": host,
            "sample": f"{CPU_RUNS} timed runs of at least {args.cpu_seconds / CPU_RUNS:.1f} s, each decoding position "
                      f"{DEC_POS0} ({DEC_POS0 + 1} rows attended) of the same workload over its {NL} layers in turn, "
                      f"{float(np.median(cd['us_per_layer'])):.0f} us per layer (median run); value = median run, "
                      "best = fastest run; C restatement of kore.cpp:1405-1455 (bit-identical to kore's own "
                      "forward()), gcc -O3, one thread: kore's attention runs on the calling thread whatever "
                      "--threads is (kore.cpp:1432 sits outside parallel_rows); "
                      f"host {host['cpu_model']}, nproc {host['nproc']}, {host['cpus_allowed']} cpus allowed",
        }
        if mv is not None:
            import oracle
            print(f"[bench] cpu baseline: kore's matvec, {args.cpu_threads} threads", file=sys.stderr, flush=True)
            res["matvec"]["cpu_baseline"] = cpu_matvec(args.cpu_seconds, args.cpu_threads)
            t, r, c = mv["mats"][0][1:]
            ref = oracle.qmatvec(t, mv["first_raw"], r, c, oracle.quantize_q8K(mv["first_x"]), avx2=True)
            res["parity"]["matvec_first_matrix_bitwise"] = bool(
                np.array_equal(ref.view(np.uint32), mv["first_out"].view(np.uint32)))
        if gm is not None:
            import oracle
            print(f"[bench] cpu baseline: kore's batched matmul, {args.cpu_threads} threads", file=sys.stderr,
                  flush=True)
            res["gemm"]["cpu_baseline"] = cpu_gemm(args.cpu_seconds, args.cpu_threads)
            t, r, c = gm["mats"][0][1:]
            ref = oracle.matmul_batch(t, gm["first_raw"], r, c, gm["first_x"], avx2=True)
            err = float(np.max(np.abs(ref.astype(np.float64) - gm["first_out"])))
            bound = 1e-4 * float(np.max(np.abs(ref))) + 1e-6
            res["parity"]["gemm_first_matrix_max_abs_err"] = err
            res["parity"]["gemm_first_matrix_within_kore_tolerance"] = bool(err <= bound)
        if tk is not None:
            print(f"[bench] cpu baseline: kore's forward(), {args.cpu_threads} threads", file=sys.stderr, flush=True)
            res["token"]["cpu_baseline"] = cpu_token(args.cpu_seconds, args.cpu_threads)
            print(f"[bench] kore's forward() with the attention drop-in, {args.cpu_threads} threads", file=sys.stderr,
                  flush=True)
            res["token"]["kore_with_attention_dropin"] = kore_token_dropin(args.cpu_seconds, args.cpu_threads)
        if pr is not None:
            print(f"[bench] cpu baseline: kore's forward_batch(), {args.cpu_threads} threads", file=sys.stderr,
                  flush=True)
            res["prompt"]["cpu_baseline"] = cpu_prompt(args.cpu_seconds, args.cpu_threads)
        if pf is not None:
            print(f"[bench] cpu baseline: prefill ({CPU_RUNS} runs of one 2048-row layer)", file=sys.stderr,
                  flush=True)
            cp = cpu_prefill(pf["outs"])
            res["prefill"]["cpu_baseline"] = {
                "value": round(cp["tflops"]["median"], 5), "unit": "TFLOP/s", "cores": 1, "kind": "port",
                "best": round(cp["tflops"]["best"], 5), "runs": cp["tflops"]["runs"], "threads": 1,
                "sample": f"{CPU_RUNS} timed runs, each one whole {PF_N}-row causal prefill layer of the same "
                          f"workload (layers 0..{CPU_RUNS - 1}), {cp['seconds']:.1f} s in all; value = median run, "
                          "best = fastest run; C restatement of kore.cpp:1503-1563 with kore's AVX2 hd_dot/hd_fma "
                          "arithmetic (bit-identical to kore's own forward_batch()), one thread as kore's attention",
            }
            res["parity"]["prefill_max_rel_err"] = cp["max_rel_err"]
            res["parity"]["prefill_layers_compared"] = CPU_RUNS
    dec["attn"].close()
    res["summary"] = _summary(res)
    print(json.dumps(res), flush=True)
    return 0


def _summary(res):
    """The figures of every leg in a few hundred bytes, last on the line (a
    truncated tail of the output still shows them)."""
    def g(*path):
        d = res
        for k in path:
            if not isinstance(d, dict) or k not in d:
                return None
            d = d[k]
        return d
    par = res.get("parity", {})
    out = {
        "c2_decode_7b_us_per_layer": g("decode", "us_per_layer_gpu"),
        "c2_floor_us": g("decode", "floor", "read_plus_dependent_launch_us"),
        "c2_over_floor": g("decode", "floor", "layer_over_floor"),
        "c2_frac": g("roofline", "frac"),
        "c3_prefill_7b_us_per_layer": g("prefill", "us_per_layer_gpu"),
        "c3_frac": g("prefill", "roofline", "frac"),
        "c1_decode_0p5b_us": g("other_workloads", "decode_0p5b_pos511", "us_per_layer_gpu"),
        "c4_decode_3b_us_per_layer": g("other_workloads", "decode_3b_pos32767", "us_per_layer_gpu"),
        "c4_frac": g("other_workloads", "decode_3b_pos32767", "roofline", "frac"),
        "c5_chunk_1p5b_us_per_layer": g("other_workloads", "chunk_1p5b_1024_at_7168", "us_per_layer_gpu"),
        "c5_chunk_frac": g("other_workloads", "chunk_1p5b_1024_at_7168", "roofline", "frac"),
        "c5_sliding_decode_us_per_layer": g("other_workloads", "decode_1p5b_sliding_8192", "us_per_layer_gpu"),
        "token_ms": g("token", "ms_per_token_gpu"),
        "prompt_ms_per_chunk": g("prompt", "ms_per_chunk_gpu"),
        "matvec_ms_per_token": g("matvec", "ms_per_token_gpu"),
        "gemm_ms_per_chunk": g("gemm", "ms_per_chunk_gpu"),
        "parity_max_rel_err": {k: (par[k].get("max_rel_err") if isinstance(par.get(k), dict) else None)
                               for k in ("c1_decode_0p5b", "c4_decode_3b", "c5_chunk_1p5b", "c5_sliding_decode_1p5b")},
    }
    out["parity_max_rel_err"]["c2_decode_7b"] = par.get("decode_max_rel_err")
    out["parity_max_rel_err"]["c3_prefill_7b"] = par.get("prefill_max_rel_err")
    return out


if __name__ == "__main__":
    sys.exit(main())
