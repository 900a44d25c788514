#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-matmul path (one GPU).

Headline (BASELINE.json metric, config 1): q4_0 GEMV, M=1, K=4096 -> N=14336,
reported as algorithmic GB/s (packed weight bytes + 4K + 4N per step, the
reference's bytes_moved, benchmarks/cases/qgemv.cpp:119-124).  A "step" is
one GEMV over one synthetic batch; the K timed steps are captured in one HIP
graph and replayed once, between two device synchronisations.  Each step
reads a different copy of the weights (ceil(256 MB / footprint) + 1 copies)
so that every step streams from HBM, not from the 256 MB Infinity Cache.

`legs` holds every part of BASELINE.json's metric, each with its roofline and
CPU baseline: q4_0 and q8_0 GEMV at K4096xN14336 (GB/s, HBM), the W8A8 int8
GEMM at M=2048, K=4096, N=4096 and 14336 (TOPS, int8 MFMA), and config 3's
per-token activation quantizer.  Secondary lines (same discipline) cover the
other BASELINE configs: q8_0 GEMV (config 0), q4_0 K=14336 -> N=4096, the
q8_0 small-batch GEMM (config 2), the other W8A8 producers, and the
per-layer sums of the 32-layer decoder sweep (config 4).

cpu_baseline: the reference's own x86 routes (compiled from the reference
sources into oracle/_ref by oracle/Makefile) on this host's cores -- q4_0
gguf_gemv_avx2 (q4_rows), q8_0_gemv_ref, the dispatched int8_gemm (AVX-512
VNNI where present) on 64 of the 2048 rows, and quantize_int8 -- at the
physical cores of NUMA node 0 available to this process and at 1 thread.
The same legs gate each GPU result (contract tolerance for the GEMVs, bit
for bit for the int8 GEMM) before its number is reported.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "quixicore-cpu_amd"))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, published
INT8_PEAK_TOPS = 5000.0      # MI355X dense int8 MFMA, published (POP/s)
FP32_PEAK_TFLOPS = 157.3     # MI355X fp32, published
MALL_BYTES = 256 << 20       # Infinity Cache


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=1000)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--only", choices=["headline", "all", "copy", "stream", "w8a8", "qgemm", "prefill",
                                      "legs", "cint8", "decode", "layer"],
                   default="all",
                   help="copy: a plain 64 MiB device copy, the calibration kernel for "
                        "FETCH_SIZE / WRITE_SIZE counter runs; w8a8 / qgemm / prefill / legs / "
                        "cint8 / decode (qgemv_w8a8, fused up_gate and QKV) / layer (the "
                        "config-4 sweep): only those cases (for profiling), no JSON line")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--rows-per-wave", type=int, default=0)
    p.add_argument("--eager", action="store_true",
                   help="time eager launches instead of one graph replay (for counter runs)")
    return p.parse_args()


EAGER = False


# When set, every case keeps one copy of its inputs (cache-resident figures:
# the 256 MB Infinity Cache holds the weights between steps).
RESIDENT = False


def rotation(footprint):
    if RESIDENT:
        return 1
    return int(math.ceil(MALL_BYTES / footprint)) + 1


def time_steps(launch, steps, warmup):
    """W eager warmup steps, then exactly K steps captured in one graph and
    replayed between synchronisations (after one untimed replay of the new
    graph).  Returns (wall ms/step, GPU ms/step from HIP events recorded on the
    launch stream around the replay)."""
    import torch
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for i in range(warmup):
            launch(i)
    torch.cuda.synchronize()
    if EAGER:
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            t0 = time.perf_counter()
            start.record(stream)
            for i in range(steps):
                launch(warmup + i)
            end.record(stream)
            torch.cuda.synchronize()
            t1 = time.perf_counter()
        LAST_SAMPLES.clear()
        return (t1 - t0) * 1e3 / steps, start.elapsed_time(end) / steps
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(steps):
            launch(warmup + i)
    torch.cuda.synchronize()
    # One untimed replay of the new graph first.  A replay that starts on an
    # idle GPU (the synchronisation before the timed region) runs slower than
    # replays queued back to back: q4_0 headline, 200 steps per replay, 8.52
    # us per step timed against a 7.83 us median over 20 replays queued after
    # it; the default of 1000 steps per replay shrinks that start-up share.
    with torch.cuda.stream(stream):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        start.record(stream)
        graph.replay()
        end.record(stream)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
    wall_ms = (t1 - t0) * 1e3 / steps
    gpu_ms = start.elapsed_time(end) / steps
    # the reference harness's statistic (median of >= 20 samples after warmup,
    # benchmarks/harness/timing.cpp:19-85): 20 more replays of the same graph,
    # each bracketed by events; per-step GPU time of each replay
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(SAMPLES)]
    with torch.cuda.stream(stream):
        for a, b in evs:
            a.record(stream)
            graph.replay()
            b.record(stream)
    torch.cuda.synchronize()
    per = sorted(a.elapsed_time(b) / steps for a, b in evs)
    LAST_SAMPLES.clear()
    LAST_SAMPLES.update({"gpu_ms_median": per[len(per) // 2], "gpu_ms_p20": per[len(per) // 5],
                         "gpu_ms_p80": per[(4 * len(per)) // 5], "samples": len(per)})
    del graph
    return wall_ms, gpu_ms


SAMPLES = 20
LAST_SAMPLES = {}


def samples():
    """Median / p20 / p80 per-step GPU time of the replays after the last
    time_steps call (empty for eager timing)."""
    return dict(LAST_SAMPLES)


def contract_gate(qc, fmt, packed, X, Y, n, k, rows):
    """Correctness gate of one GPU result before it is timed: the given
    activation rows of Y against the f64 contract |y - y64| <= 1e-4 *
    ||x||_2 * ||w_hat_row||_2 (tests/correctness/test_qgemv.cpp:278-303).
    The weights are dequantized by the library's unpack kernel (bit-exact with
    the reference's unpackers, tested) and multiplied in float64 on the GPU."""
    import torch
    w = qc.unpack(fmt, packed, n, k).double()
    wn = w.norm(dim=1)
    xr = X.reshape(-1, k)[rows].double()
    y64 = xr @ w.T.contiguous()
    del w
    err = (Y.reshape(-1, n)[rows].double() - y64).abs()
    bound = 1e-4 * xr.norm(dim=1, keepdim=True) * wn[None, :]
    worst = float((err / bound.clamp_min(1e-300)).max()) * 1e-4
    torch.cuda.synchronize()
    return {"pass": bool((err <= bound).all()), "rows_checked": len(rows),
            "max_norm_err_vs_f64": worst}


def w8a8_gate(w, x, ws, as_, y, rows):
    """Bit-exact gate of int8_gemm outputs on the given rows: the int32 dots
    from a float64 product (exact: every partial sum is an integer below
    2^53) and the reference's epilogue (float(dot) * ws[n]) * as[m]
    (kernels/quantization/int8_gemm_ref.cpp:9-32) as two separately rounded
    f32 multiplies."""
    import torch
    acc = x[rows].double() @ w.double().T.contiguous()
    want = (acc.float() * ws[None, :]) * as_[rows, None]
    ok = torch.equal(y[rows].view(torch.int32), want.view(torch.int32))
    return {"pass": bool(ok), "rows_checked": len(rows), "bit_exact": True}


STREAM_SIZES = (("17.9MB_q8_0_k4096_n4096", 17858560), ("33.1MB_q4_0_k4096_n14336", 33103872),
                ("62.5MB_q8_0_k4096_n14336", 62464000), ("256MB", 256 << 20))


def stream_ceiling(qc, steps, warmup, sizes=STREAM_SIZES, wpcs=(1, 2, 4, 8, 16)):
    """The streaming-read ceiling at the GEMV footprints: qc_hip_stream_read
    (16-byte non-temporal loads, sixteen in flight per thread) over rotated buffers of
    each size, one launch per step, timed like the GEMV; best over 1-16
    workgroups per CU."""
    import torch
    dev = torch.device("cuda:0")
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    out = torch.empty(cus * 16 * 256, dtype=torch.int32, device=dev)
    cases = {}
    for name, nbytes in sizes:
        nb = (nbytes + 15) // 16 * 16
        copies = rotation(nb)
        bufs = [torch.empty(nb, dtype=torch.uint8, device=dev).random_(0, 255) for _ in range(copies)]
        best = None
        for wpc in wpcs:
            grid = cus * wpc

            def launch(i, grid=grid):
                st = qc.lib.qc_hip_stream_read(qc._ptr(bufs[i % copies]), nb, qc._ptr(out), grid,
                                               qc._stream(None))
                if st:
                    raise RuntimeError(f"stream_read status {st}")

            wall, gpu = time_steps(launch, steps, warmup)
            r = {"bytes": nb, "copies": copies, "grid": grid, "wall_ms": wall, "gpu_ms": gpu, **samples(),
                 "gbs": nb / (wall * 1e-3) / 1e9, "kernel_gbs": nb / (gpu * 1e-3) / 1e9}
            if best is None or r["gpu_ms"] < best["gpu_ms"]:
                best = r
        cases[f"stream_read_{name}"] = best
        del bufs
    return cases


def gemv_case(qc, fmt, n, k, steps, warmup, seed, gate=False):
    """Rotated copies of packed weights; returns timing and one output.  With
    `gate`, every output of one launch is checked against the f64 contract
    before timing."""
    import torch
    dev = torch.device("cuda:0")
    bb = qc.BLOCK_BYTES[fmt]
    wbytes = n * (k // 32) * bb
    copies = rotation(wbytes)
    g = torch.Generator(device=dev).manual_seed(seed)
    packs = []
    for c in range(copies):
        w = torch.randn((n, k), generator=g, device=dev) * 0.02
        packs.append(qc.pack(fmt, w))
        del w
    x = torch.randn(k, generator=g, device=dev)
    y = torch.empty(n, dtype=torch.float32, device=dev)

    def launch(i):
        st = qc.qgemv_raw(fmt, packs[i % copies], x, y, n, k)
        if st:
            raise RuntimeError(f"qgemv status {st}")

    check = None
    if gate:
        launch(0)
        check = contract_gate(qc, fmt, packs[0], x, y, n, k, [0])
    wall, gpu = time_steps(launch, steps, warmup)
    alg = wbytes + 4 * k + 4 * n
    r = {"bytes": alg, "weight_bytes": wbytes, "copies": copies, "wall_ms": wall,
         "gpu_ms": gpu, **samples(), "gbs": alg / (wall * 1e-3) / 1e9,
         "kernel_gbs": alg / (gpu * 1e-3) / 1e9}
    if gate:
        r["check"] = check
    return r, packs[0], x, y


def gemv_w8a8_case(qc, fmt, n, k, steps, warmup, seed):
    """qgemv_w8a8 (per-block int8 activations) on rotated weight copies; the
    asynchronous form (device status word), as a decode loop would call it."""
    import torch
    dev = torch.device("cuda:0")
    wbytes = n * (k // 32) * qc.BLOCK_BYTES[fmt]
    copies = rotation(wbytes)
    g = torch.Generator(device=dev).manual_seed(seed)
    packs = []
    for c in range(copies):
        w = torch.randn((n, k), generator=g, device=dev) * 0.02
        packs.append(qc.pack(fmt, w))
        del w
    x = torch.randn(k, generator=g, device=dev)
    y = torch.empty(n, dtype=torch.float32, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev)

    def launch(i):
        st = qc.qgemv_w8a8_raw(fmt, packs[i % copies], x, y, n, k, status)
        if st:
            raise RuntimeError(f"qgemv_w8a8 status {st}")

    wall, gpu = time_steps(launch, steps, warmup)
    alg = wbytes + 4 * k + 4 * n
    return {"bytes": alg, "weight_bytes": wbytes, "copies": copies, "wall_ms": wall,
            "gpu_ms": gpu, **samples(), "gbs": alg / (wall * 1e-3) / 1e9,
            "kernel_gbs": alg / (gpu * 1e-3) / 1e9}


def fused_case(qc, kind, fmt, rows, k, steps, warmup, seed, gate=False):
    """One fused decode launch over one x: kind "up_gate" (rows = (n, n)) or
    "qkv" (rows = (q, kv, kv)), rotated weight copies.  With `gate`, every
    projection of one launch is checked against the f64 contract first."""
    import torch
    dev = torch.device("cuda:0")
    bb = qc.BLOCK_BYTES[fmt]
    wbytes = sum(r * (k // 32) * bb for r in rows)
    copies = rotation(wbytes)
    g = torch.Generator(device=dev).manual_seed(seed)
    sets = []
    for c in range(copies):
        mats = []
        for r in rows:
            w = torch.randn((r, k), generator=g, device=dev) * 0.02
            mats.append(qc.pack(fmt, w))
            del w
        sets.append(mats)
    x = torch.randn(k, generator=g, device=dev)
    ys = [torch.empty(r, dtype=torch.float32, device=dev) for r in rows]

    def launch(i):
        m = sets[i % copies]
        if kind == "up_gate":
            st = qc.qgemv_up_gate_raw(fmt, m[0], m[1], x, ys[0], ys[1], rows[0], k)
        else:
            st = qc.qgemv_qkv_raw(fmt, m[0], m[1], m[2], x, ys[0], ys[1], ys[2], rows[0], rows[1], k)
        if st:
            raise RuntimeError(f"{kind} status {st}")

    check = None
    if gate:
        launch(0)
        parts = [contract_gate(qc, fmt, p, x, y, r, k, [0]) for p, y, r in zip(sets[0], ys, rows)]
        check = {"pass": all(p["pass"] for p in parts), "rows_checked": 1,
                 "max_norm_err_vs_f64": max(p["max_norm_err_vs_f64"] for p in parts)}
    wall, gpu = time_steps(launch, steps, warmup)
    alg = wbytes + 4 * k + 4 * sum(rows)
    r = {"bytes": alg, "copies": copies, "wall_ms": wall, "gpu_ms": gpu, **samples(),
         "gbs": alg / (wall * 1e-3) / 1e9, "kernel_gbs": alg / (gpu * 1e-3) / 1e9}
    if gate:
        r["check"] = check
    return r


def qgemm_case(qc, n, k, m, steps, warmup, seed, fmt=0, gate=False):
    """Small-batch / prefill qgemm on rotated weight copies.  With `gate`, the
    first and last activation rows of one launch (and a middle one) are
    checked against the f64 contract before timing."""
    import torch
    dev = torch.device("cuda:0")
    wbytes = n * (k // 32) * qc.BLOCK_BYTES[fmt]
    copies = rotation(wbytes + 4 * m * k)
    g = torch.Generator(device=dev).manual_seed(seed)
    packs = [qc.pack(fmt, torch.randn((n, k), generator=g, device=dev) * 0.02) for _ in range(copies)]
    x = torch.randn((m, k), generator=g, device=dev)
    y = torch.empty((m, n), dtype=torch.float32, device=dev)

    def launch(i):
        st = qc.qgemm_raw(fmt, packs[i % copies], x, y, m, n, k)
        if st:
            raise RuntimeError(f"qgemm status {st}")

    check = None
    if gate:
        launch(0)
        check = contract_gate(qc, fmt, packs[0], x, y, n, k, sorted({0, m // 2, m - 1}))
    wall, gpu = time_steps(launch, steps, warmup)
    alg = wbytes + 4 * m * k + 4 * m * n
    flops = 2.0 * m * n * k
    r = {"m": m, "n": n, "k": k, "bytes": alg, "wall_ms": wall, "gpu_ms": gpu, **samples(),
         "gbs": alg / (wall * 1e-3) / 1e9, "kernel_gbs": alg / (gpu * 1e-3) / 1e9,
         "kernel_tflops": flops / (gpu * 1e-3) / 1e12}
    if gate:
        r["check"] = check
    return r


def cint8_case(qc, n, k, m, steps, warmup, groups=1, mode=0):
    """Prepared storage projection over canonical int8 weights (C ABI
    qc_hip_cint8_project): f32 x [m][k], f32 y; mode 1 = SwiGLU over two
    [n][k] matrices.  Rotated weight copies; bytes = codes + scales + x + y."""
    import torch
    dev = torch.device("cuda:0")
    nw = 2 if mode == 1 else 1
    wbytes = nw * (n * k + 4 * n * groups)
    copies = rotation(wbytes)
    g = torch.Generator(device=dev).manual_seed(31)
    mats = []
    for _ in range(copies):
        ws = []
        for _ in range(nw):
            codes = torch.randint(-127, 128, (n, k), generator=g, device=dev, dtype=torch.int8)
            scales = torch.rand(n * groups, generator=g, device=dev) * 1e-3 + 1e-5
            ws.append((codes, scales))
        mats.append(ws)
    structs = [[qc.cint8_weights(c, s_, None, n, k, groups) for c, s_ in ws] for ws in mats]
    x = torch.randn((m, k), generator=g, device=dev)
    y = torch.empty((m, n), dtype=torch.float32, device=dev)

    def launch(i):
        st = qc.cint8_project_raw(mode, structs[i % copies], x, 0, m, [y], [0])
        if st:
            raise RuntimeError(f"cint8 status {st}")

    wall, gpu = time_steps(launch, steps, warmup)
    alg = wbytes + 4 * m * k + 4 * m * n
    return {"m": m, "n": n, "k": k, "groups": groups, "bytes": alg, "copies": copies,
            "wall_ms": wall, "gpu_ms": gpu, **samples(), "gbs": alg / (wall * 1e-3) / 1e9,
            "kernel_gbs": alg / (gpu * 1e-3) / 1e9}


def quant_case(qc, m, k, steps, warmup):
    import torch
    dev = torch.device("cuda:0")
    fp = 4 * m * k + m * k + 4 * m
    copies = rotation(fp)
    xs = [torch.randn((m, k), device=dev) for _ in range(copies)]
    codes = torch.empty((m, k), dtype=torch.int8, device=dev)
    scales = torch.empty((m, 1), dtype=torch.float32, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev)

    def launch(i):
        st = qc.quantize_int8_raw(xs[i % copies], codes, scales, m, k, 0, status)
        if st:
            raise RuntimeError(f"quantize status {st}")

    wall, gpu = time_steps(launch, steps, warmup)
    return {"m": m, "k": k, "bytes": fp, "wall_ms": wall, "gpu_ms": gpu, **samples(),
            "gbs": fp / (wall * 1e-3) / 1e9, "kernel_gbs": fp / (gpu * 1e-3) / 1e9}


def norm_quant_case(qc, m, k, steps, warmup):
    """rms_norm_add_quant_int8 (the W8A8 producer): reads x, residual and the
    weight, writes residual_out, codes and per-row scales."""
    import torch
    dev = torch.device("cuda:0")
    fp = 4 * m * k * 3 + m * k + 4 * m + 4 * k
    copies = rotation(fp)
    xs = [torch.randn((m, k), device=dev) for _ in range(copies)]
    rs = [torch.randn((m, k), device=dev) for _ in range(copies)]
    w = torch.randn(k, device=dev)
    out = torch.empty((m, k), dtype=torch.float32, device=dev)
    codes = torch.empty((m, k), dtype=torch.int8, device=dev)
    scales = torch.empty((m, 1), dtype=torch.float32, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev)

    def launch(i):
        st = qc.rms_norm_add_quant_int8_raw(xs[i % copies], rs[i % copies], w, codes, out, scales,
                                            m, k, 1e-5, 0, status)
        if st:
            raise RuntimeError(f"rms_norm_add_quant status {st}")

    wall, gpu = time_steps(launch, steps, warmup)
    return {"m": m, "k": k, "bytes": fp, "wall_ms": wall, "gpu_ms": gpu, **samples(),
            "gbs": fp / (wall * 1e-3) / 1e9, "kernel_gbs": fp / (gpu * 1e-3) / 1e9}


def asym_case(qc, m, k, steps, warmup):
    import torch
    dev = torch.device("cuda:0")
    fp = 4 * m * k + m * k + 8 * m
    copies = rotation(fp)
    xs = [torch.randn((m, k), device=dev) for _ in range(copies)]
    codes = torch.empty((m, k), dtype=torch.int8, device=dev)
    scales = torch.empty(m, dtype=torch.float32, device=dev)
    zps = torch.empty(m, dtype=torch.int32, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev)

    def launch(i):
        st = qc.quantize_int8_asymmetric_raw(xs[i % copies], codes, scales, zps, m, k, status)
        if st:
            raise RuntimeError(f"quantize_int8_asymmetric status {st}")

    wall, gpu = time_steps(launch, steps, warmup)
    return {"m": m, "k": k, "bytes": fp, "wall_ms": wall, "gpu_ms": gpu, **samples(),
            "gbs": fp / (wall * 1e-3) / 1e9, "kernel_gbs": fp / (gpu * 1e-3) / 1e9}


def w8a8_operands(qc, m, n, k, seed=7):
    """BASELINE config 3's operands: weights f32 ~N(0, 0.02) quantized per
    output channel (absmax / 127), activations f32 ~N(0, 1) with 0.1% of the
    elements scaled by 20, quantized per row -- both with quantize_int8."""
    import torch
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed)
    wf = torch.randn((n, k), generator=g, device=dev) * 0.02
    w, ws = qc.quantize_int8(wf)
    del wf
    xf = torch.randn((m, k), generator=g, device=dev)
    xf = torch.where(torch.rand((m, k), generator=g, device=dev) < 1e-3, xf * 20.0, xf)
    x, as_ = qc.quantize_int8(xf)
    return w, x, ws.reshape(-1), as_.reshape(-1)


def w8a8_case(qc, m, n, k, steps, warmup, keep=False, gate=False):
    """int8_gemm over config 3's operand distribution.  With `gate`, 64
    output rows spread over every m-tile of one launch are checked bit for
    bit before timing."""
    import torch
    dev = torch.device("cuda:0")
    w, x, ws, as_ = w8a8_operands(qc, m, n, k)
    y = torch.empty((m, n), dtype=torch.float32, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev)

    def launch(i):
        st = qc.int8_gemm_raw(w, x, ws, as_, None, None, y, m, n, k, False, status)
        if st:
            raise RuntimeError(f"int8_gemm status {st}")

    check = None
    if gate:
        launch(0)
        rows = torch.linspace(0, m - 1, 64, device=dev).round().long().unique()
        check = w8a8_gate(w, x, ws, as_, y, rows)
    wall, gpu = time_steps(launch, steps, warmup)
    ops = 2.0 * m * n * k
    r = {"m": m, "n": n, "k": k, "ops": ops, "wall_ms": wall, "gpu_ms": gpu, **samples(),
         "tops": ops / (wall * 1e-3) / 1e12, "kernel_tops": ops / (gpu * 1e-3) / 1e12}
    if gate:
        r["check"] = check
    return (r, (w, x, ws, as_, y)) if keep else r


# the matmuls of one layer of a synthetic 32-layer,
# 4096-hidden / 14336-FFN decoder, as (count, N, K).
LAYER = [(4, 4096, 4096), (2, 14336, 4096), (1, 4096, 14336)]


def layer_sweep(qc, steps, warmup):
    """Per-layer sum of kernel times for each regime of config 4: q4_0 weights
    at M=1 (GEMV), M=8 (small-batch GEMM) and M=512 (prefill, the 2-D GEMM);
    W8A8 at M=512 and M=2048
    (per-token activation quantization + int8 GEMM).  Each matmul is timed on
    its own (same graph discipline, rotated weight copies), after one launch
    of it passed its correctness gate (f64 contract for q4_0 rows, bit-exact
    int8 GEMM rows); every regime reports its gates' outcome in `check`."""
    out = {}

    def gates(parts):
        return {"pass": all(p["pass"] for p in parts), "matmuls_checked": len(parts)}

    for m in (1, 8, 512):
        us, wbytes, checks = 0.0, 0, []
        for cnt, n, k in LAYER:
            if m == 1:
                r, *_ = gemv_case(qc, 1, n, k, steps, warmup, seed=100 + n + k, gate=True)
            else:
                r = qgemm_case(qc, n, k, m, steps, warmup, seed=200 + n + k, fmt=1, gate=True)
            checks.append(r["check"])
            us += cnt * r["gpu_ms"] * 1e3
            wbytes += cnt * n * (k // 32) * 18
        flops = sum(cnt * 2.0 * m * n * k for cnt, n, k in LAYER)
        out[f"q4_0_m{m}"] = {"layer_us": us, "model_ms_32_layers": 32 * us / 1e3,
                             "weight_gbs": wbytes / (us * 1e-6) / 1e9,
                             "tflops": flops / (us * 1e-6) / 1e12, "check": gates(checks)}
    # M = 1 with the fused decode seams: Q/K/V in one launch (4096 x 3 rows),
    # O alone, gate/up in one launch, down alone.
    us, checks = 0.0, []
    r = fused_case(qc, "qkv", 1, (4096, 4096, 4096), 4096, steps, warmup, seed=301, gate=True)
    us += r["gpu_ms"] * 1e3
    checks.append(r["check"])
    r, *_ = gemv_case(qc, 1, 4096, 4096, steps, warmup, seed=302, gate=True)
    us += r["gpu_ms"] * 1e3
    checks.append(r["check"])
    r = fused_case(qc, "up_gate", 1, (14336, 14336), 4096, steps, warmup, seed=303, gate=True)
    us += r["gpu_ms"] * 1e3
    checks.append(r["check"])
    r, *_ = gemv_case(qc, 1, 4096, 14336, steps, warmup, seed=304, gate=True)
    us += r["gpu_ms"] * 1e3
    checks.append(r["check"])
    wbytes = sum(cnt * n * (k // 32) * 18 for cnt, n, k in LAYER)
    out["q4_0_m1_fused"] = {"layer_us": us, "model_ms_32_layers": 32 * us / 1e3,
                            "weight_gbs": wbytes / (us * 1e-6) / 1e9, "check": gates(checks)}
    for m in (512, 2048):
        us, ops, checks = 0.0, 0.0, []
        for cnt, n, k in LAYER:
            q = quant_case(qc, m, k, steps, warmup)
            g = w8a8_case(qc, m, n, k, max(10, steps // 4), warmup, gate=True)
            checks.append(g["check"])
            us += cnt * (q["gpu_ms"] + g["gpu_ms"]) * 1e3
            ops += cnt * 2.0 * m * n * k
        out[f"w8a8_m{m}"] = {"layer_us": us, "model_ms_32_layers": 32 * us / 1e3,
                             "tops": ops / (us * 1e-6) / 1e12, "check": gates(checks)}
    return out


def profiled_traffic(name):
    """HBM bytes per launch measured by rocprofv3 FETCH_SIZE + WRITE_SIZE runs,
    scaled by the copy-kernel calibration, from the committed summary
    profiles/<name>.txt (None if absent).  Not measured in this run: the
    counters need their own profiler passes."""
    import re
    path = os.path.join(ROOT, "profiles", name + ".txt")
    if not os.path.exists(path):
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.]+)", open(path).read())
    return float(m.group(1)) if m else None


def traffic_source(name):
    """Where roofline.traffic comes from (it is read, not measured here)."""
    if profiled_traffic(name) is None:
        return None
    return (f"profiles/{name}.txt: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes of the same "
            "kernel, copy-calibrated; read from the committed summary, not measured in this run")


def host_cpu():
    """The host's CPU as the CPU baselines use it: model, the ISA features the
    reference's dispatch looks at, and the thread count -- the physical cores
    of NUMA node 0 that this process may run on, capped by its cgroup CPU
    quota (the GPU box's share of the host)."""
    info = {"model": None, "isa": [], "numa_node0_physical_cores": None,
            "allowed_cpus": len(os.sched_getaffinity(0)), "cgroup_cpu_quota": None}
    try:
        flags = set()
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name") and info["model"] is None:
                info["model"] = line.split(":", 1)[1].strip()
            elif line.startswith("flags") and not flags:
                flags = set(line.split(":", 1)[1].split())
        info["isa"] = [f for f in ("avx2", "fma", "f16c", "avx512f", "avx512bw", "avx512vl",
                                   "avx512dq", "avx512_vnni", "avx_vnni", "amx_int8")
                       if f in flags]
    except OSError:
        pass
    allowed = os.sched_getaffinity(0)
    try:
        node0 = set()
        for part in open("/sys/devices/system/node/node0/cpulist").read().strip().split(","):
            a, _, b = part.partition("-")
            node0.update(range(int(a), int(b or a) + 1))
        cores = set()
        for c in sorted(node0 & allowed):
            topo = f"/sys/devices/system/cpu/cpu{c}/topology/"
            cores.add((open(topo + "physical_package_id").read().strip(),
                       open(topo + "core_id").read().strip()))
        info["numa_node0_physical_cores"] = len(cores)
    except (OSError, ValueError):
        pass
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()
        if quota != "max":
            info["cgroup_cpu_quota"] = int(quota) / int(period)
    except (OSError, ValueError):
        pass
    threads = info["numa_node0_physical_cores"] or info["allowed_cpus"]
    if info["cgroup_cpu_quota"]:
        threads = min(threads, max(1, int(info["cgroup_cpu_quota"])))
    info["threads"] = max(1, threads)
    return info


def time_cpu(call, budget):
    """The reference harness's discipline (benchmarks/harness/timing.cpp:19-85):
    warmup >= 3 calls and >= 50 ms, then >= 20 samples of batches >= 2 ms until
    the budget is spent; returns (median seconds per call, samples)."""
    import numpy as np
    t_end = time.perf_counter() + 0.05
    calls = 0
    while calls < 3 or time.perf_counter() < t_end:
        call()
        calls += 1
    samples = []
    deadline = time.perf_counter() + budget
    while len(samples) < 20 or time.perf_counter() < deadline:
        t0 = time.perf_counter()
        reps = 0
        while True:
            call()
            reps += 1
            if time.perf_counter() - t0 >= 2e-3:
                break
        samples.append((time.perf_counter() - t0) / reps)
    return float(np.median(samples)), len(samples)


def reference():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    if not oracle.Reference.available():
        return None, oracle
    return oracle.Reference(), oracle


def cpu_legs(ref, oracle, cpu, seconds, work, unit, describe):
    """One CPU baseline: `work(threads)` returns (call, units per call); timed
    at the chosen thread count and at 1 thread, the reference's thread pool
    set explicitly (its default is 1, include/quixicore_cpu/threading.h:6-11)."""
    threads = cpu["threads"]
    ref.set_threads(threads)
    call, units = work()
    t_all, s_all = time_cpu(call, seconds * 0.7)
    ref.set_threads(1)
    t_one, s_one = time_cpu(call, seconds * 0.3)
    scale = 1e9 if unit == "GB/s" else 1e12
    return {"value": units / t_all / scale, "unit": unit, "cores": threads, "kind": "reference",
            "sample": (f"{describe}; median of {s_all} samples (>=2 ms batches, "
                       f"~{seconds * 0.7:.0f} s) at {threads} threads"),
            "value_1thread": units / t_one / scale, "ms_per_call": t_all * 1e3,
            "ms_per_call_1thread": t_one * 1e3,
            "cpu": {"model": cpu["model"], "isa": cpu["isa"],
                    "numa_node0_physical_cores": cpu["numa_node0_physical_cores"],
                    "cgroup_cpu_quota": cpu["cgroup_cpu_quota"]}}


def gemv_baseline(ref, oracle, cpu, fmt, packed_dev, x_dev, y_dev, n, k, seconds):
    """The reference's x86 GEMV route on this host (q4_0: gguf_gemv_avx2's
    q4_rows; q8_0: q8_0_gemv_ref, its only x86 route) on the same packed
    bytes, plus the correctness gate of one fresh GPU step: f64 contract
    oracle and the reference's own f32 output, both at 1e-4 normalised."""
    import numpy as np
    import quixicore_hip as qc
    packed = packed_dev.cpu().numpy()
    x = x_dev.cpu().numpy()
    st = qc.qgemv_raw(fmt, packed_dev, x_dev, y_dev, n, k)
    if st:
        raise RuntimeError(f"qgemv status {st}")
    y_gpu = y_dev.cpu().numpy()
    y64, wn = oracle.gemv_f64(fmt, packed, x, n, k)
    ok, worst = oracle.within_contract(y_gpu, y64, wn, x, 1e-4)
    y_ref = ref.gemv(fmt, packed, x, n, k)
    ok_ref, worst_ref = oracle.within_contract(y_gpu, y_ref.astype(np.float64), wn, x, 1e-4)
    gate = {"pass": bool(ok and ok_ref), "max_norm_err_vs_f64": worst,
            "max_norm_err_vs_reference": worst_ref}
    y = np.empty(n, dtype=np.float32)
    fn = ref.lib.qcref_q8_0_gemv if fmt == 0 else ref.lib.qcref_q4_0_gemv_avx2
    args = (oracle._ptr(packed), oracle._ptr(x), oracle._ptr(y), n, k)
    alg = n * (k // 32) * (34 if fmt == 0 else 18) + 4 * k + 4 * n
    name = "q8_0_gemv_ref" if fmt == 0 else "gguf_gemv_avx2 (q4_rows)"
    base = cpu_legs(ref, oracle, cpu, seconds, lambda: (lambda: fn(*args), alg), "GB/s",
                    f"reference {name} {'q8_0' if fmt == 0 else 'q4_0'} GEMV K={k} N={n} on the "
                    "same packed bytes")
    return base, gate


def w8a8_baseline(ref, oracle, cpu, w_dev, x_dev, ws_dev, as_dev, y_dev, sample_rows, seconds):
    """The reference's dispatched int8_gemm (src/dispatch/int8_gemm.cpp:20-63:
    AVX-512 VNNI where avx512f/bw/vl/dq + vnni are present) on the first
    `sample_rows` activation rows of the same operands, plus the bit-exact
    gate of the GPU output on those rows."""
    import numpy as np
    w = w_dev.cpu().numpy()
    x = np.ascontiguousarray(x_dev[:sample_rows].cpu().numpy())
    ws = ws_dev.cpu().numpy()
    as_ = np.ascontiguousarray(as_dev[:sample_rows].cpu().numpy())
    n, k = w.shape
    st, y_ref = ref.int8_gemm(w, x, ws, as_)
    gpu = y_dev[:sample_rows].cpu().numpy()
    gate = {"pass": bool(st == 0 and np.array_equal(gpu.view(np.uint32), y_ref.view(np.uint32))),
            "rows_checked": sample_rows, "bit_exact": True}
    y = np.empty((sample_rows, n), dtype=np.float32)
    args = (oracle._ptr(w), oracle._ptr(x), oracle._ptr(ws), oracle._ptr(as_), None, None,
            oracle._ptr(y), sample_rows, n, k, 0)
    ops = 2.0 * sample_rows * n * k
    base = cpu_legs(ref, oracle, cpu, seconds,
                    lambda: (lambda: ref.lib.qcref_int8_gemm(*args), ops), "TOPS",
                    f"reference int8_gemm ({ref.variant()} route) M={sample_rows} of the 2048 "
                    f"rows, N={n} K={k}, same int8 operands")
    return base, gate


def quant_baseline(ref, oracle, cpu, m, k, seconds):
    """The reference's quantize_int8 (kernels/quantization/quantization_ref.cpp:
    143-168, scalar per row) over config 3's whole M x K activation matrix,
    plus the bit-exact gate of the GPU quantizer on the same matrix (codes
    and scale bits against the reference's)."""
    import numpy as np
    import torch
    import quixicore_hip as qc
    from quixicore_hip import synth
    x = synth.activations_outliers_fast(3, m, k)
    codes_gpu, scales_gpu = qc.quantize_int8(torch.from_numpy(x).to("cuda:0"))
    st, codes_ref, scales_ref = ref.quantize_int8(x)
    gate = {"pass": bool(st == 0
                         and np.array_equal(codes_gpu.cpu().numpy(), codes_ref)
                         and np.array_equal(scales_gpu.cpu().numpy().view(np.uint32),
                                            scales_ref.view(np.uint32))),
            "rows_checked": m, "bit_exact": True}
    codes = np.empty((m, k), dtype=np.int8)
    scales = np.empty(m, dtype=np.float32)
    args = (oracle._ptr(x), oracle._ptr(codes), oracle._ptr(scales), m, k, 0)
    fp = 4 * m * k + m * k + 4 * m
    base = cpu_legs(ref, oracle, cpu, seconds,
                    lambda: (lambda: ref.lib.qcref_quantize_int8(*args), fp), "GB/s",
                    f"reference quantize_int8 M={m} K={k} (config 3 activations)")
    return base, gate


def median_fields(r):
    """The median (p20, p80) per-step kernel time over the 20 replays that
    follow a case's timed replay, in microseconds."""
    if "gpu_ms_median" not in r:
        return {}
    return {"kernel_us_median": round(r["gpu_ms_median"] * 1e3, 3),
            "kernel_us_p20_p80": [round(r["gpu_ms_p20"] * 1e3, 3), round(r["gpu_ms_p80"] * 1e3, 3)],
            "samples": r["samples"]}


def print_cases(cases):
    for key, r in cases.items():
        print(f"# {key}: " + ", ".join(f"{a}={b:.4g}" if isinstance(b, float) else f"{a}={b}"
                                      for a, b in r.items()), file=sys.stderr, flush=True)


def main():
    args = parse()
    global EAGER, RESIDENT
    EAGER = args.eager
    if args.gpus != 1:
        print(f"bench.py: this build runs on exactly one GPU (asked for --gpus {args.gpus}); "
              "sharding N across GPUs (replicated x, one all-gather of y) is designed, not "
              "built.", file=sys.stderr)
        sys.exit(2)
    import torch
    import quixicore_hip as qc
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    if args.rows_per_wave:
        qc.set_gemv_rows_per_wave(args.rows_per_wave)
    if args.only == "copy":
        # the plain 64 MiB copy that calibrates rocprofv3's FETCH_SIZE / WRITE_SIZE
        src = torch.randint(0, 255, (64 << 20,), dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(args.warmup + args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": 64 << 20, "launches": args.warmup + args.steps}))
        return
    if args.only == "stream":
        print_cases(stream_ceiling(qc, args.steps, args.warmup))
        return
    K, W = args.steps, args.warmup
    if args.only in ("w8a8", "qgemm", "prefill", "legs", "cint8", "decode", "layer"):
        s = {}
        if args.only == "decode":
            s["q4_0_gemv_w8a8_k4096_n14336"] = gemv_w8a8_case(qc, 1, 14336, 4096, K, W, seed=11)
            s["q8_0_gemv_w8a8_k4096_n4096"] = gemv_w8a8_case(qc, 0, 4096, 4096, K, W, seed=12)
            s["q4_0_up_gate_k4096_n2x14336"] = fused_case(qc, "up_gate", 1, (14336, 14336), 4096,
                                                          K, W, seed=13, gate=True)
            s["q4_0_qkv_k4096_n3x4096"] = fused_case(qc, "qkv", 1, (4096, 4096, 4096), 4096, K, W,
                                                     seed=14, gate=True)
        elif args.only == "layer":
            for key, r in layer_sweep(qc, K, W).items():
                s[f"decoder_layer_{key}"] = r
        elif args.only == "legs":
            # the metric's legs in the order the JSON line lists them
            s["q4_0_gemv_k4096_n14336"], *_ = gemv_case(qc, 1, 14336, 4096, K, W, seed=1)
            s["q8_0_gemv_k4096_n14336"], *_ = gemv_case(qc, 0, 14336, 4096, K, W, seed=5)
            s["w8a8_m2048_k4096_n4096"] = w8a8_case(qc, 2048, 4096, 4096, K, W)
            s["w8a8_m2048_k4096_n14336"] = w8a8_case(qc, 2048, 14336, 4096, K, W)
            s["quantize_int8_m2048_k4096"] = quant_case(qc, 2048, 4096, K, W)
        elif args.only == "prefill":
            # the 2-D GEMM route (M >= 64) at a 4096 / 14336 layer's FFN shape
            for fmt, name in ((1, "q4_0"), (0, "q8_0")):
                for m in (512, 2048):
                    s[f"{name}_qgemm_m{m}_k4096_n14336"] = qgemm_case(qc, 14336, 4096, m, K, W,
                                                                     seed=8 + m, fmt=fmt)
        elif args.only == "cint8":
            s["cint8_channel_m1_k4096_n14336"] = cint8_case(qc, 14336, 4096, 1, K, W)
            s["cint8_group128_m1_k4096_n14336"] = cint8_case(qc, 14336, 4096, 1, K, W, groups=32)
            s["cint8_channel_m4_k4096_n14336"] = cint8_case(qc, 14336, 4096, 4, K, W)
            s["cint8_swiglu_m1_k4096_n2x14336"] = cint8_case(qc, 14336, 4096, 1, K, W, mode=1)
            s["cint8_channel_m2_k4096_n14336"] = cint8_case(qc, 14336, 4096, 2, K, W)
            s["cint8_channel_m16_k4096_n14336"] = cint8_case(qc, 14336, 4096, 16, K, W)
            s["cint8_swiglu_m16_k4096_n2x14336"] = cint8_case(qc, 14336, 4096, 16, K, W, mode=1)
            s["cint8_channel_m64_k4096_n14336"] = cint8_case(qc, 14336, 4096, 64, K, W)
            s["cint8_channel_m512_k4096_n14336"] = cint8_case(qc, 14336, 4096, 512, max(5, K // 4), W)
            s["cint8_group128_m16_k4096_n14336"] = cint8_case(qc, 14336, 4096, 16, K, W, groups=32)
            s["cint8_group128_m64_k4096_n14336"] = cint8_case(qc, 14336, 4096, 64, K, W, groups=32)
            s["cint8_group128_m512_k4096_n14336"] = cint8_case(qc, 14336, 4096, 512, max(5, K // 4),
                                                               W, groups=32)
            s["cint8_group64_m16_k4096_n14336"] = cint8_case(qc, 14336, 4096, 16, K, W, groups=64)
            s["cint8_group64_m64_k4096_n14336"] = cint8_case(qc, 14336, 4096, 64, K, W, groups=64)
            s["cint8_group32_m16_k4096_n14336"] = cint8_case(qc, 14336, 4096, 16, K, W, groups=128)
            s["cint8_group32_m64_k4096_n14336"] = cint8_case(qc, 14336, 4096, 64, K, W, groups=128)
        elif args.only == "w8a8":
            s["quantize_int8_m2048_k4096"] = quant_case(qc, 2048, 4096, K, W)
            s["rms_norm_add_quant_int8_m2048_k4096"] = norm_quant_case(qc, 2048, 4096, K, W)
            s["quantize_int8_asymmetric_m2048_k4096"] = asym_case(qc, 2048, 4096, K, W)
            s["w8a8_m2048_k4096_n4096"] = w8a8_case(qc, 2048, 4096, 4096, K, W)
            s["w8a8_m2048_k4096_n14336"] = w8a8_case(qc, 2048, 14336, 4096, K, W)
        else:
            for fmt, name in ((0, "q8_0"), (1, "q4_0")):
                for n_ in (4096, 14336):
                    for m in (4, 8, 16, 32):
                        s[f"{name}_qgemm_m{m}_k4096_n{n_}"] = qgemm_case(qc, n_, 4096, m, K, W,
                                                                        seed=4 + m, fmt=fmt)
        print_cases(s)
        return
    n, k = 14336, 4096
    head, packed, x, y = gemv_case(qc, 1, n, k, K, W, seed=1)
    print(f"# headline q4_0 GEMV K={k} N={n}: {head['gbs']:.1f} GB/s wall, "
          f"{head['kernel_gbs']:.1f} GB/s kernel ({head['gpu_ms'] * 1e3:.2f} us)",
          file=sys.stderr, flush=True)
    # the other legs of BASELINE.json's metric
    q8, packed8, x8, y8 = gemv_case(qc, 0, n, k, K, W, seed=5)
    w8, w8ops = {}, {}
    for n_ in (4096, 14336):
        w8[n_], w8ops[n_] = w8a8_case(qc, 2048, n_, 4096, max(20, K // 4), W, keep=True)
    quant = quant_case(qc, 2048, 4096, K, W)
    # the streaming-read ceiling of the same footprints, measured in this process
    ceil = stream_ceiling(qc, K, W, sizes=STREAM_SIZES[1:3], wpcs=(2, 4))
    print_cases(ceil)
    print_cases({"q8_0_gemv_k4096_n14336": q8, "w8a8_m2048_k4096_n4096": w8[4096],
                 "w8a8_m2048_k4096_n14336": w8[14336], "quantize_int8_m2048_k4096": quant})
    secondary = {}
    if args.only == "all":
        s = {}
        r, *_ = gemv_case(qc, 0, 4096, 4096, K, W, seed=2)
        s["q8_0_gemv_k4096_n4096"] = r
        r, *_ = gemv_case(qc, 1, 4096, 14336, K, W, seed=3)
        s["q4_0_gemv_k14336_n4096"] = r
        s["q4_0_gemv_w8a8_k4096_n14336"] = gemv_w8a8_case(qc, 1, 14336, 4096, K, W, seed=11)
        s["q8_0_gemv_w8a8_k4096_n4096"] = gemv_w8a8_case(qc, 0, 4096, 4096, K, W, seed=12)
        s["q4_0_up_gate_k4096_n2x14336"] = fused_case(qc, "up_gate", 1, (14336, 14336), 4096, K, W,
                                                      seed=13)
        for n_ in (4096, 14336):
            for m in (4, 8, 16, 32):
                s[f"q8_0_qgemm_m{m}_k4096_n{n_}"] = qgemm_case(qc, n_, 4096, m, K, W, seed=4 + m)
        s["rms_norm_add_quant_int8_m2048_k4096"] = norm_quant_case(qc, 2048, 4096, K, W)
        s["quantize_int8_asymmetric_m2048_k4096"] = asym_case(qc, 2048, 4096, K, W)
        # prepared storage projections over canonical int8 weights (f32 x and y)
        s["cint8_channel_m1_k4096_n14336"] = cint8_case(qc, 14336, 4096, 1, K, W)
        s["cint8_group128_m1_k4096_n14336"] = cint8_case(qc, 14336, 4096, 1, K, W, groups=32)
        s["cint8_channel_m4_k4096_n14336"] = cint8_case(qc, 14336, 4096, 4, K, W)
        s["cint8_swiglu_m1_k4096_n2x14336"] = cint8_case(qc, 14336, 4096, 1, K, W, mode=1)
        s["cint8_channel_m16_k4096_n14336"] = cint8_case(qc, 14336, 4096, 16, K, W)
        for key, r in layer_sweep(qc, max(20, K // 4), W).items():
            s[f"decoder_layer_{key}"] = r
        # the same GEMV legs with one weight copy: cache-resident (Infinity
        # Cache) figures beside the rotated, HBM-streaming ones above
        RESIDENT = True
        try:
            for fmt, name, n_, k_ in ((1, "q4_0", 14336, 4096), (0, "q8_0", 14336, 4096),
                                      (0, "q8_0", 4096, 4096), (1, "q4_0", 4096, 14336)):
                r, *_ = gemv_case(qc, fmt, n_, k_, K, W, seed=21)
                s[f"{name}_gemv_k{k_}_n{n_}_cache_resident"] = r
        finally:
            RESIDENT = False
        print_cases(s)
        secondary = s

    cpu = host_cpu()
    ref, oracle = (None, None) if args.no_cpu else reference()
    bases = {}
    if ref is not None:
        sec = args.cpu_seconds
        bases["q4_0"] = gemv_baseline(ref, oracle, cpu, 1, packed, x, y, n, k, sec)
        bases["q8_0"] = gemv_baseline(ref, oracle, cpu, 0, packed8, x8, y8, n, k, sec * 0.5)
        for n_ in (4096, 14336):
            bases[n_] = w8a8_baseline(ref, oracle, cpu, w8ops[n_][0], w8ops[n_][1], w8ops[n_][2],
                                      w8ops[n_][3], w8ops[n_][4], 64, sec * 0.5)
        bases["quant"] = quant_baseline(ref, oracle, cpu, 2048, 4096, sec * 0.3)
        ref.set_threads(1)
    del w8ops

    def gemv_leg(r, key, name, ceiling=None):
        base, gate = bases.get(key, (None, None))
        extra = {}
        if ceiling is not None:
            extra = {"stream_read_us": round(ceiling["gpu_ms"] * 1e3, 3),
                     "pct_of_stream_read": round(100.0 * ceiling["gpu_ms"] / r["gpu_ms"], 1)}
        return {"value": round(r["gbs"], 2), "unit": "GB/s", **extra,
                "pct_hbm_peak": round(100.0 * r["gbs"] / HBM_PEAK_GBS, 2),
                "kernel_us": round(r["gpu_ms"] * 1e3, 3), "bytes_per_step": r["bytes"],
                **median_fields(r),
                "roofline": {"bound": "hbm", "achieved": round(r["kernel_gbs"], 2),
                             "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(r["kernel_gbs"] / HBM_PEAK_GBS, 4),
                             "traffic": profiled_traffic(name),
                             "traffic_source": traffic_source(name)},
                "cpu_baseline": base, "check": gate}

    def w8a8_leg(r, key, name):
        base, gate = bases.get(key, (None, None))
        return {"value": round(r["tops"], 2), "unit": "TOPS",
                "kernel_us": round(r["gpu_ms"] * 1e3, 3), "ops_per_step": r["ops"],
                **median_fields(r),
                "roofline": {"bound": "mfma", "achieved": round(r["kernel_tops"], 2),
                             "peak": INT8_PEAK_TOPS, "unit": "TOP/s",
                             "frac": round(r["kernel_tops"] / INT8_PEAK_TOPS, 4),
                             "traffic": profiled_traffic(name),
                             "traffic_source": traffic_source(name)},
                "cpu_baseline": base, "check": gate}

    legs = {
        "q4_0_gemv_k4096_n14336": gemv_leg(head, "q4_0", "q4_0_gemv_k4096_n14336",
                                           ceil["stream_read_33.1MB_q4_0_k4096_n14336"]),
        "q8_0_gemv_k4096_n14336": gemv_leg(q8, "q8_0", "q8_0_gemv_k4096_n14336",
                                           ceil["stream_read_62.5MB_q8_0_k4096_n14336"]),
        "w8a8_gemm_m2048_k4096_n4096": w8a8_leg(w8[4096], 4096, "w8a8_int8_gemm_m2048_k4096_n4096"),
        "w8a8_gemm_m2048_k4096_n14336": w8a8_leg(w8[14336], 14336,
                                                 "w8a8_int8_gemm_m2048_k4096_n14336"),
        "quantize_int8_m2048_k4096": gemv_leg(quant, "quant", "quantize_int8_m2048_k4096"),
    }
    head_leg = legs["q4_0_gemv_k4096_n14336"]
    line = {
        "metric": "q4_0 GEMV GB/s (% HBM peak) at K4096xN14336",
        "value": round(head["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": head["wall_ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int32 (exact int8 dot4 block sums) + f32",
        "dtype_note": ("q4_0 weights (4-bit codes, fp16 block scales); each 32-element block of "
                       "the f32 activations is encoded as 22-bit fixed point (three int8 digit "
                       "planes), block dots are exact int32 v_dot4_i32_i8 sums, scaled and "
                       "accumulated in f32"),
        "data": ("synthetic: torch-seeded N(0,0.02) f32 weights packed to q4_0 on the GPU, "
                 f"{head['copies']} rotated copies (HBM-resident, > Infinity Cache); x ~ N(0,1)"),
        "config": {"workload": "qgemv q4_0 M=1 K=4096 N=14336 (BASELINE config 1, up/gate)",
                   "m": 1, "k": k, "n": n, "bytes_per_step": head["bytes"],
                   "weight_bytes_per_step": head["weight_bytes"],
                   "parallelism": "single GPU"},
        "pct_hbm_peak": round(100.0 * head["gbs"] / HBM_PEAK_GBS, 2),
        # a pure 16-byte-load read of the same 33.1 MB in this process (qc_hip_stream_read)
        "stream_read_us": head_leg["stream_read_us"],
        "pct_of_stream_read": head_leg["pct_of_stream_read"],
        "roofline": dict(head_leg["roofline"], kernel_us=round(head["gpu_ms"] * 1e3, 3)),
        "cpu_baseline": head_leg["cpu_baseline"],
        "check": head_leg["check"],
        "legs": legs,
        "host_cpu": cpu,
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
