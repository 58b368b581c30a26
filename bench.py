#!/usr/bin/env python3
"""Benchmark of the quantized linear hot path on one MI355X.

A step is one pass of the hot path over one batch of synthetic input: the
Q4_G64 M=1 GEMV (K=2560, N=10240: the north-star shape) over each of the
weight copies in turn (40 copies, 557 MB: more than the 256 MB MALL, so every
weight byte comes from HBM); x, y and the copies are resident in HBM before
the timed region.

Exactly K steps are timed (K * 40 dispatches, so K >= 5 gives the >= 200
dispatches a measurement needs), after W warm-up steps run eagerly: HIP graphs
of up to 25 steps (1000 launches) each, every graph replayed once untimed and
then back to back in the timed region, bracketed by HIP events on the replay
stream, so the host never throttles the stream.  value = algorithmic bytes *
dispatches / elapsed; the roofline's achieved bandwidth uses the same average
dispatch duration (us_per_gemv).  Every other line is timed over one graph of
>= 200 calls.  The CPU baseline is the oracle's C restatement of the same GEMV
(same semantics, seeded inputs), timed on this host with 1 and all threads.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
       python bench.py --read-sweep | --dispatch-floor | --clock-period | --timeline [q4|q5|q6|w8]
                       | --timeline-rc M | --only LINE   (measurement modes)
"""
import argparse
import ctypes as C
import json
import math
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q4_G64 GEMV µs + achieved HBM GB/s (% of peak) at M=1; M=16 verify µs"
PEAK_GBS = 8000.0
ROTATE_BYTES = 512 * 1024 * 1024
MIN_STEPS = 200  # calls per line for the lines other than the headline
GRAPH_STEPS = 25  # headline steps per captured graph


def algorithmic_bytes(qtype_bytes_per_row, N, K, M, G=64):
    """packed weights + 16-bit scales + x (bf16, once) + y (bf16)."""
    return N * qtype_bytes_per_row + N * (K // G) * 2 + M * K * 2 + M * N * 2


def make_weights(torch, copies, N, K, gen, row_bytes=None, G=64):
    """Uniform bytes = uniform codes over each format's range (Q4 nibbles in [-8, 7], the Q5/Q6 low
    and high planes, W8 bytes; W8's -128 code is the only value outside its stated range and does not
    change the timing); fp16 scales log-uniform in [1e-3, 1e-2]."""
    rb = K // 2 if row_bytes is None else row_bytes
    w = torch.randint(0, 256, (copies, N * rb), dtype=torch.uint8, device="cuda", generator=gen)
    u = torch.rand((copies, N * (K // G)), device="cuda", generator=gen, dtype=torch.float32)
    s = torch.exp(math.log(1e-3) + u * math.log(10.0)).to(torch.float16)
    return w, s


# bytes per weight row and group size of each format: Q4 K/2 nibbles; Q5/Q6 the nibble plane plus a
# 1- or 2-bit high plane; W8 one byte per weight (the layouts viper_qlinear.h documents)
ROW_BYTES = {4: lambda K: K // 2, 5: lambda K: K * 5 // 8, 6: lambda K: K * 6 // 8, 8: lambda K: K}
GROUP = {4: 64, 5: 64, 6: 64, 8: 32}


def time_linear(torch, L, gen, qtype, N, K, M, steps=400, outliers=False, prequantized=False, frag=False):
    """us per call of viper_hip_qlinear (bf16 x, fused or separate quantize) over rotating weights;
    outliers: 5% of the activation channels (a fixed seeded set) scaled x20, as config 4 states;
    prequantized: x quantized once (viper_hip_quantize_act) outside the timed calls, each call
    viper_hip_qlinear_prequantized (int8 rows and their fp32 group scales in, bf16 y out);
    frag: the same with the rows in the matrix-core fragment order (viper_hip_rmsnorm_quantize_frag of
    x with gamma = 1 outside the timed calls, each call viper_hip_qlinear_prequantized_frag with a
    workspace of viper_hip_qlinear_frag_workspace_bytes, so long K splits over workgroups)."""
    G = GROUP[qtype]
    rb = ROW_BYTES[qtype](K)
    copy_bytes = N * rb + N * (K // G) * 2
    copies = max(2, -(-ROTATE_BYTES // copy_bytes) + 1)
    W, S = make_weights(torch, copies, N, K, gen, row_bytes=rb, G=G)
    xf = torch.randn((M, K), device="cuda", generator=gen)
    if outliers:
        ch = torch.randperm(K, device="cuda", generator=gen)[: K // 20]
        xf[:, ch] *= 20.0
    x = xf.to(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    nws = L.viper_hip_qlinear_frag_workspace_bytes(qtype, N, K, M) if frag else \
        L.viper_hip_qlinear_workspace_bytes(qtype, N, K, M)
    ws = torch.zeros(max(nws, 16), dtype=torch.uint8, device="cuda")   # zero before first use
    if prequantized:
        xq = torch.empty(M * K, dtype=torch.int8, device="cuda")
        xs = torch.empty(M * (K // G), dtype=torch.float32, device="cuda")
        if L.viper_hip_quantize_act(G, x.data_ptr(), M, K, xq.data_ptr(), xs.data_ptr(),
                                    torch.cuda.current_stream().cuda_stream) != 0:
            raise RuntimeError("quantize_act failed")
    if frag:
        xq = torch.empty(16 * K, dtype=torch.int8, device="cuda")
        xs = torch.empty(16 * (K // G), dtype=torch.float32, device="cuda")
        ones = torch.ones(K, dtype=torch.bfloat16, device="cuda")
        if L.viper_hip_rmsnorm_quantize_frag(x.data_ptr(), ones.data_ptr(), 1e-6, M, K, G, None, xq.data_ptr(),
                                             xs.data_ptr(), torch.cuda.current_stream().cuda_stream) != 0:
            raise RuntimeError("rmsnorm_quantize_frag failed")

    def launch(i):
        c = i % copies
        st = torch.cuda.current_stream().cuda_stream
        if frag:
            rc = L.viper_hip_qlinear_prequantized_frag(qtype, W[c].data_ptr(), S[c].data_ptr(), 0, G, N, K,
                                                       xq.data_ptr(), xs.data_ptr(), M, y.data_ptr(), None,
                                                       ws.data_ptr() if nws else None, nws, st)
        elif prequantized:
            rc = L.viper_hip_qlinear_prequantized(qtype, W[c].data_ptr(), S[c].data_ptr(), 0, G, N, K,
                                                  xq.data_ptr(), xs.data_ptr(), M, y.data_ptr(), None, st)
        else:
            rc = L.viper_hip_qlinear(qtype, W[c].data_ptr(), S[c].data_ptr(), 0, G, N, K, x.data_ptr(), M,
                                     y.data_ptr(), None, ws.data_ptr() if nws else None, nws, st)
        if rc != 0:
            raise RuntimeError(f"qlinear qtype={qtype} N={N} K={K} M={M} failed: {rc}")
    for i in range(20):
        launch(i)
    us = time_steps(torch, launch, max(steps, MIN_STEPS))
    del W, S
    alg = algorithmic_bytes(rb, N, K, M, G)
    if prequantized or frag:  # int8 rows + fp32 group scales in place of the bf16 rows
        alg += M * K + M * (K // G) * 4 - 2 * M * K
    return round(us, 3), round(alg / (us * 1e-6) / 1e9, 1)


def capture_n(torch, launch, n):
    """One HIP graph holding exactly n launches (launch(i) for i < n, i picks the weight copy)."""
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(n):
            launch(i)
    graph.replay()
    torch.cuda.synchronize()
    return graph


def time_steps(torch, launch, n):
    """us per call of launch(i) over one HIP graph of n calls (i = 0..n-1, cycling the weight copies),
    replayed once untimed and once timed."""
    g = capture_n(torch, launch, n)
    us = time_graph(torch, g, 1) * 1e3 / n
    del g
    return us


def time_graph(torch, graph, replays):
    """Elapsed ms of `replays` graph replays, events on the replay stream, after as many untimed
    replays: a line timed right after its weights were allocated read up to 0.8 us slower per launch
    without them (clocks and memory still settling)."""
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(replays):
        graph.replay()
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(replays):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1)


def clock_period(torch, L, launch, counts=(40, 120), replays=10):
    """us per launch of back-to-back launch(i) calls on the GPU's own 100 MHz clock, independent of
    HIP events and of a profiler: for each n in counts one HIP graph [clock stamp, launch(0..n-1),
    clock stamp] (viper_hip_clock_stamp), replayed once untimed and then `replays` times; span(n) =
    median of (second stamp - first stamp).  The least-squares slope of span over n is the period;
    the stamps' own launches and the graph's entry and exit fall into the intercept.  Returns
    (period_us, intercept_us, [(n, span_us), ...])."""
    stamps = torch.zeros(2, dtype=torch.int64, device="cuda")

    def stamp(k):
        if L.viper_hip_clock_stamp(stamps.data_ptr() + 8 * k, torch.cuda.current_stream().cuda_stream) != 0:
            raise RuntimeError("viper_hip_clock_stamp failed")
    rows = []
    for n in counts:
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            stamp(0)
            for i in range(n):
                launch(i)
            stamp(1)
        spans = []
        for r in range(replays + 1):
            g.replay()
            torch.cuda.synchronize()
            t = stamps.cpu().tolist()
            if r:
                spans.append((t[1] - t[0]) * 0.01)   # 100 MHz ticks -> us
        del g
        spans.sort()
        rows.append((n, spans[len(spans) // 2]))
    k = len(rows)
    mx = sum(n for n, _ in rows) / k
    my = sum(v for _, v in rows) / k
    sxx = sum((n - mx) ** 2 for n, _ in rows)
    slope = sum((n - mx) * (v - my) for n, v in rows) / sxx
    return slope, my - slope * mx, rows


def trace_summary(path, steps, warmup, copies=40):
    """Summary of a rocprofv3 kernel-trace CSV of `bench.py --no-cpu --no-extras --steps S --warmup W`:
    per kernel of this library and grid, dispatch count and mean / median / min / max duration (ns);
    then, for the north-star GEMV, the dispatches of the timed region (in dispatch order: W * copies
    eager warm-up launches, one untimed replay of the captured graphs, then the S * copies timed ones),
    their summed duration and the span from the first one's start to the last one's end."""
    import csv
    rows = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            name = r["Kernel_Name"]
            if "vq::" not in name:
                continue
            key = (name, int(r["Grid_Size_X"]) // max(1, int(r["Workgroup_Size_X"])), int(r["Workgroup_Size_X"]))
            rows.setdefault(key, []).append((int(r["Dispatch_Id"]), int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    for (name, wgs, nt), d in sorted(rows.items(), key=lambda kv: -len(kv[1])):
        d.sort()
        dur = sorted(e - b for _, b, e in d)
        print(json.dumps({"kernel": name[:120], "workgroups": wgs, "threads": nt, "dispatches": len(d),
                          "mean_ns": round(sum(dur) / len(dur), 1), "median_ns": dur[len(dur) // 2],
                          "min_ns": dur[0], "max_ns": dur[-1]}), flush=True)
    ns = [v for (n, wgs, nt), v in rows.items() if "qgemv_m1_kernel<4" in n and wgs == 512 and nt == 320]
    if ns:
        d = sorted(ns[0])
        lo = warmup * copies + steps * copies
        timed = d[lo:lo + steps * copies]
        dur = [e - b for _, b, e in timed]
        gaps = sorted(timed[i + 1][1] - timed[i][2] for i in range(len(timed) - 1))
        print(json.dumps({"timed_dispatches": len(timed), "sum_duration_us": round(sum(dur) / 1e3, 2),
                          "mean_duration_ns": round(sum(dur) / len(dur), 1),
                          "span_us": round((timed[-1][2] - timed[0][1]) / 1e3, 2),
                          "median_gap_ns": gaps[len(gaps) // 2] if gaps else None}), flush=True)


def cpu_baseline(N, K, reps_1t, reps_mt):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    packed, scales = O.gen_weights(O.Q4_G64, N, K, 0x5EED0000, O.SCALE_FP16)
    x = O.gen_act(1, K, 0x5EED0001)
    nthreads = O.omp_max_threads()
    O.qlinear_omp(O.Q4_G64, packed, scales, O.SCALE_FP16, N, K, x, 1)
    t0 = time.perf_counter()
    for _ in range(reps_1t):
        O.qlinear_omp(O.Q4_G64, packed, scales, O.SCALE_FP16, N, K, x, 1)
    t1 = (time.perf_counter() - t0) / reps_1t
    O.qlinear_omp(O.Q4_G64, packed, scales, O.SCALE_FP16, N, K, x, nthreads)
    t0 = time.perf_counter()
    for _ in range(reps_mt):
        O.qlinear_omp(O.Q4_G64, packed, scales, O.SCALE_FP16, N, K, x, nthreads)
    tm = (time.perf_counter() - t0) / reps_mt
    return t1, tm, nthreads


# ---- the streaming-read floor -----------------------------------------------------------

SWEEP_SHAPES = [(64, 16), (128, 10), (256, 5), (256, 10), (320, 5), (320, 10), (512, 5), (512, 8), (640, 5),
                (640, 10), (1024, 4), (1024, 8)]
SWEEP_MB = [13.1072, 28, 56, 112, 557]


def _time_probe(torch, L, pool, nbytes, threads, loads, y=None, launches=200, side_bytes=0):
    """us per dispatch of viper_hip_stream_read over rotating slices of pool (>= 512 MB of distinct
    data, or >= 2 slices for large sizes); with side_bytes, every workgroup also reads its own block of
    that many bytes, placed after the slice's nbytes."""
    wgs = nbytes // (threads * loads * 16)
    stride = (nbytes + wgs * side_bytes + 65535) // 65536 * 65536
    copies = max(2, min(40, pool.numel() // stride))
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    base = pool.data_ptr()
    yp = None if y is None else y.data_ptr()

    def launch(i):
        st = torch.cuda.current_stream().cuda_stream   # the capture stream while a graph is captured
        a = base + (i % copies) * stride
        rc = L.viper_hip_stream_read(a, nbytes, threads, loads, a + nbytes if side_bytes else None, side_bytes, yp,
                                     sink.data_ptr(), st)
        if rc != 0:
            raise RuntimeError(f"stream_read {threads}x{loads} {nbytes} failed: {rc}")
    n = max(launches, 2 * copies)
    for i in range(2 * copies):
        launch(i)
    g = capture_n(torch, launch, n)
    us = time_graph(torch, g, 1) * 1e3 / n
    del g
    return us


def dispatch_floor(torch, L, launches=400):
    """us per launch of viper_hip_empty_dispatch, back to back in one HIP graph (time_steps): one
    64-thread workgroup; the north-star GEMV's grid (512 x 320) without stores; the same grid storing one
    bf16 per 16-lane team (10240 rows, the GEMV's output pattern); and the 16-row GEMM's grid
    (256 x 640)."""
    y = torch.zeros(65536, dtype=torch.bfloat16, device="cuda")
    for nm, wg, nt, store in (("one_workgroup", 1, 64, False), ("gemv_grid", 512, 320, False),
                              ("gemv_grid_row_stores", 512, 320, True), ("gemm16_grid", 256, 640, False)):
        def launch(i, wg=wg, nt=nt, store=store):
            rc = L.viper_hip_empty_dispatch(wg, nt, y.data_ptr() if store else None,
                                            torch.cuda.current_stream().cuda_stream)
            if rc != 0:
                raise RuntimeError(f"viper_hip_empty_dispatch failed: {rc}")
        for i in range(50):
            launch(i)
        us = min(time_steps(torch, launch, launches) for _ in range(3))
        print(json.dumps({"dispatch": nm, "workgroups": wg, "threads": nt, "row_stores": store,
                          "us_per_launch": round(us, 3)}), flush=True)


def read_sweep(torch, L, gen):
    """Launch shapes x sizes of the GEMV-pattern streaming read; per shape a least-squares fit
    t = fixed + bytes / bandwidth over the sizes; then the north-star I/O ladder at the GEMV's shape."""
    pool = torch.randint(0, 256, (1200 << 20,), dtype=torch.uint8, device="cuda", generator=gen)
    best13 = None
    for threads, loads in SWEEP_SHAPES:
        per_wg = threads * loads * 16
        pts = []
        for mb in SWEEP_MB:
            nbytes = max(1, round(mb * 1e6 / per_wg)) * per_wg
            us = _time_probe(torch, L, pool, nbytes, threads, loads, launches=200 if mb < 100 else 40)
            pts.append((nbytes, us))
        xs = [b / 1e6 for b, _ in pts]
        ys = [u for _, u in pts]
        n = len(xs)
        mx, my = sum(xs) / n, sum(ys) / n
        slope = sum((a - mx) * (b - my) for a, b in zip(xs, ys)) / sum((a - mx) ** 2 for a in xs)
        fixed = my - slope * mx
        line = {"probe": "stream_read", "threads": threads, "loads_per_lane": loads,
                "points_bytes_us": [[b, round(u, 3)] for b, u in pts],
                "fit_fixed_us": round(fixed, 3), "fit_gbs": round(1e3 / slope, 1)}
        print(json.dumps(line), flush=True)
        if best13 is None or pts[0][1] < best13[1]:
            best13 = ((threads, loads), pts[0][1], pts[0][0])
    print(json.dumps({"probe": "best_13MB_shape", "threads": best13[0][0], "loads_per_lane": best13[0][1],
                      "bytes": best13[2], "us": round(best13[1], 3)}), flush=True)
    # the north-star GEMV's I/O at its own launch shape (320 threads, 5 loads per lane, 512 workgroups of
    # 20 rows): the weights; the weights and each workgroup's 1600-byte block of scales (13,926,400 bytes,
    # as the GEMV reads them); the same with one bf16 store per row
    y = torch.empty(512 * 20, dtype=torch.int16, device="cuda")
    ladder = {"probe": "north_star_io_ladder"}
    ladder["read_13107200_us"] = round(_time_probe(torch, L, pool, 13107200, 320, 5), 3)
    ladder["read_weights_scale_blocks_us"] = round(_time_probe(torch, L, pool, 13107200, 320, 5, side_bytes=1600), 3)
    ladder["read_weights_scale_blocks_store_rows_us"] = round(
        _time_probe(torch, L, pool, 13107200, 320, 5, y=y, side_bytes=1600), 3)
    print(json.dumps(ladder), flush=True)
    del pool


def timeline(torch, L, gen, N, K, qt=4):
    """Per-wave timeline of the M=1 GEMV of format qt at shape (K, N): percentiles of each
    stamp over all waves of one dispatch (the last of a back-to-back sequence over rotating weights),
    in us from the first wave's start."""
    G = GROUP[qt]
    copy_bytes = N * ROW_BYTES[qt](K) + N * (K // G) * 2
    copies = max(2, -(-ROTATE_BYTES // copy_bytes) + 1)
    W, S = make_weights(torch, copies, N, K, gen, row_bytes=ROW_BYTES[qt](K), G=G)
    x = torch.randn((1, K), device="cuda", generator=gen).to(torch.bfloat16)
    y = torch.empty((1, N), dtype=torch.bfloat16, device="cuda")
    stamps = torch.zeros(1 << 20, dtype=torch.int64, device="cuda")
    grid, waves = C.c_int(0), C.c_int(0)

    def launch(i):
        c = i % copies
        st = torch.cuda.current_stream().cuda_stream   # the capture stream while a graph is captured
        rc = L.viper_hip_qlinear_timeline(qt, W[c].data_ptr(), S[c].data_ptr(), 0, G, N, K, x.data_ptr(),
                                          y.data_ptr(), stamps.data_ptr(), stamps.numel() * 8, C.byref(grid),
                                          C.byref(waves), st)
        if rc != 0:
            raise RuntimeError(f"timeline failed: {rc}")
    for i in range(50):
        launch(i)
    g = capture_n(torch, launch, 400)
    us = time_graph(torch, g, 1) * 1e3 / 400
    g.replay()
    torch.cuda.synchronize()
    nw = grid.value * waves.value
    t = stamps[: nw * 8].view(nw, 8).cpu().numpy()
    t = (t - t[:, 0].min()) * 0.01       # 100 MHz ticks -> us
    names = ["wave start", "activation + scale loads issued", "weight loads issued", "activation quantized",
             "barrier passed", "first chunk dotted", "last chunk dotted", "output stored"]
    import numpy as np
    rows = {}
    for i, nm in enumerate(names):
        v = np.sort(t[:, i])
        rows[nm] = [round(float(np.percentile(v, p)), 3) for p in (10, 50, 90)] + [round(float(v[-1]), 3)]
    name = {4: "Q4_G64", 5: "Q5_G64", 6: "Q6_G64", 8: "W8_G32"}[qt]
    print(json.dumps({"timeline": f"qgemv_m1 {name} K={K} N={N}", "workgroups": grid.value,
                      "waves_per_workgroup": waves.value, "us_per_launch_stamped": round(us, 3),
                      "percentiles_us_p10_p50_p90_max": rows}), flush=True)


def timeline_rc(torch, L, gen, N, K, M, qt=4):
    """Per-wave timeline of the M-row matrix-core GEMM (Q4_G64 or W8_G32 by qt, fragment input:
    viper_hip_qlinear_frag_timeline; long K on the K split, with its workspace) at shape (K, N):
    percentiles of each stamp over all waves of one dispatch (the last of a back-to-back sequence over
    rotating weights), in us from the first wave's start; with the split, the last parts' output
    stamps separately."""
    G = GROUP[qt]
    rb = ROW_BYTES[qt](K)
    copy_bytes = N * rb + N * (K // G) * 2
    copies = max(2, -(-ROTATE_BYTES // copy_bytes) + 1)
    W, S = make_weights(torch, copies, N, K, gen, row_bytes=rb, G=G)
    x = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16)
    xf = torch.empty(16 * K, dtype=torch.int8, device="cuda")
    xs = torch.empty(16 * (K // G), dtype=torch.float32, device="cuda")
    ones = torch.ones(K, dtype=torch.bfloat16, device="cuda")
    st0 = torch.cuda.current_stream().cuda_stream
    if L.viper_hip_rmsnorm_quantize_frag(x.data_ptr(), ones.data_ptr(), 1e-6, M, K, G, None, xf.data_ptr(),
                                         xs.data_ptr(), st0) != 0:
        raise RuntimeError("rmsnorm_quantize_frag failed")
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    stamps = torch.zeros(1 << 20, dtype=torch.int64, device="cuda")
    grid, waves = C.c_int(0), C.c_int(0)
    nws = L.viper_hip_qlinear_frag_workspace_bytes(qt, N, K, M)
    ws = torch.zeros(max(nws, 16), dtype=torch.uint8, device="cuda")

    def launch(i):
        c = i % copies
        st = torch.cuda.current_stream().cuda_stream
        rc = L.viper_hip_qlinear_frag_timeline(qt, W[c].data_ptr(), S[c].data_ptr(), 0, G, N, K, xf.data_ptr(),
                                               xs.data_ptr(), M, y.data_ptr(), stamps.data_ptr(), stamps.numel() * 8,
                                               C.byref(grid), C.byref(waves), ws.data_ptr() if nws else None, nws,
                                               st)
        if rc != 0:
            raise RuntimeError(f"frag timeline failed: {rc}")
    for i in range(50):
        launch(i)
    g = capture_n(torch, launch, 400)
    us = time_graph(torch, g, 1) * 1e3 / 400
    g.replay()
    torch.cuda.synchronize()
    nw = grid.value * waves.value
    t = stamps[: nw * 10].view(nw, 10).cpu().numpy()
    t = (t - t[:, 0].min()) * 0.01       # 100 MHz ticks -> us
    names = ["wave start", "activation + scale loads issued", "weight loads issued", "staged scales in LDS",
             "first group scaled", "last group scaled", "cross-wave barrier passed",
             "sums stored" if nws else "outputs stored"]
    if nws:
        names += ["counted"]
    import numpy as np
    rows = {}

    def pct(v):
        v = np.sort(v)
        return [round(float(np.percentile(v, p)), 3) for p in (10, 50, 90)] + [round(float(v[-1]), 3)]
    for i, nm in enumerate(names):
        rows[nm] = pct(t[:, i])
    if nws:   # the blocks' last parts: their outputs stored after the other parts' sums arrived
        last = t[:, 9] > t[:, 8]
        if last.any():
            rows["outputs stored (last parts)"] = pct(t[last, 9])
            rows["last parts: counted -> outputs stored"] = pct(t[last, 9] - t[last, 8])
    print(json.dumps({"timeline": f"qgemm_rc {'W8_G32' if qt == 8 else 'Q4_G64'} M={M} K={K} N={N} (fragment input"
                      + (", K split)" if nws else ")"), "workgroups": grid.value,
                      "waves_per_workgroup": waves.value, "us_per_launch_stamped": round(us, 3),
                      "percentiles_us_p10_p50_p90_max": rows}), flush=True)


def time_config3(torch, stk, fused, replays=10, prefetch=0):
    """us per config-3 decode step (one graph of the whole step, replayed), its weight + head GB/s,
    and the launches per step (prefetch > 0: the fused step with the next slot's weights warmed from a
    second stream by that many workgroups)."""
    run = (lambda: stk.step_fused(prefetch)) if fused else stk.step
    run()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    # ~0.1 s of untimed replays first: the first graph timed right after the stack's weights were
    # initialised ran ~2% slower than every later one
    for _ in range(100):
        g.replay()
    torch.cuda.synchronize()
    ms = time_graph(torch, g, replays) / replays
    del g
    # the step's algorithmic bytes as the benchmark table counts them: weights of the 44 slots and the
    # head, the slots' activations (4,595,712 B) and the head's x and logits (337,408 B)
    nbytes = stk.weight_bytes_per_step() + 4_595_712 + 337_408
    launches = (4 if fused else 9) * stk.layers * stk.passes + 3
    return round(ms * 1e3, 1), round(nbytes / (ms * 1e-3) / 1e9, 1), launches


def time_mlp(torch, L, gen, qtype=4, G=64, forms=("ref", "2launch")):
    """Config 1 (M = 1 MLP: gate+up K=2560 -> 2x10240, SwiGLU, down K=10240 -> 2560, all Q4_G64, weights
    rotating over >= 512 MB): the reference's launch sequence (gate+up as one concatenated matrix,
    swiglu + quantize, prequantized down + residual) and the 2-launch form (gate/up pair with the swiglu
    epilogue, down quantizing h in its prologue + residual).  Returns {line: value} for the forms asked
    for."""
    N, K = 10240, 2560
    extras = {}
    H, I = 2560, 10240
    step_bytes = 3 * (N * K // 2 + N * (K // G) * 2)
    mcopies = max(2, -(-ROTATE_BYTES // step_bytes) + 1)
    # gate and up concatenated (config 1: one K=2560, N=2x10240 matrix per copy, gate rows first):
    # the reference sequence launches it as one matrix, the 2-launch form pairs its two halves
    Wgu, Sgu = make_weights(torch, mcopies, 2 * I, H, gen)
    up_w, up_s = I * H // 2, I * (H // G) * 2   # byte offsets of the up half
    Wdn, Sdn = make_weights(torch, mcopies, H, I, gen)
    xm = torch.randn((1, H), device="cuda", generator=gen).to(torch.bfloat16)
    rm = torch.randn((1, H), device="cuda", generator=gen).to(torch.bfloat16)
    gum = torch.empty((1, 2 * I), dtype=torch.bfloat16, device="cuda")
    gm, um = gum[:, :I], gum[:, I:]
    ym = torch.empty((1, H), dtype=torch.bfloat16, device="cuda")
    xqm = torch.empty((1, I), dtype=torch.int8, device="cuda")
    xsm = torch.empty((1, I // G), dtype=torch.float32, device="cuda")

    def launch_mlp(i):
        c = i % mcopies
        st = torch.cuda.current_stream().cuda_stream
        rc = L.viper_hip_qlinear(qtype, Wgu[c].data_ptr(), Sgu[c].data_ptr(), 0, G, 2 * I, H, xm.data_ptr(), 1,
                                 gum.data_ptr(), None, None, 0, st)
        rc = rc or L.viper_hip_swiglu_quantize(gm.data_ptr(), um.data_ptr(), 1, I, G, gm.data_ptr(),
                                               xqm.data_ptr(), xsm.data_ptr(), st)
        rc = rc or L.viper_hip_qlinear_prequantized(qtype, Wdn[c].data_ptr(), Sdn[c].data_ptr(), 0, G, H, I,
                                                    xqm.data_ptr(), xsm.data_ptr(), 1, ym.data_ptr(),
                                                    rm.data_ptr(), st)
        if rc != 0:
            raise RuntimeError(f"MLP step failed: {rc}")
    if "ref" in forms:
        for i in range(20):
            launch_mlp(i)
        mlp_us = time_steps(torch, launch_mlp, 200)
    # weights + scales of the three matrices, x and the residual in, gate/up
    # out and back in, int8 activation + scales out and back in, y out
    mlp_bytes = (step_bytes + H * 2 * 2 + 2 * I * 2 * 2 + (I + I // G * 4) * 2 + H * 2)
    if "ref" in forms:
        extras["mlp_config1_us"] = round(mlp_us, 3)
        extras["mlp_config1_gbs"] = round(mlp_bytes / (mlp_us * 1e-6) / 1e9, 1)

    # the same MLP in 2 launches: gate/up pair with the swiglu epilogue (h bf16), then
    # down + residual quantizing h in its prologue
    def launch_mlp2(i):
        c = i % mcopies
        st = torch.cuda.current_stream().cuda_stream
        rc = L.viper_hip_qlinear_m1_swiglu(qtype, 0, G, H, 0, xm.data_ptr(), None, 0.0, None,
                                           Wgu[c].data_ptr(), Sgu[c].data_ptr(), Wgu[c].data_ptr() + up_w,
                                           Sgu[c].data_ptr() + up_s, I, gm.data_ptr(), None, None, st)
        rc = rc or L.viper_hip_qlinear(qtype, Wdn[c].data_ptr(), Sdn[c].data_ptr(), 0, G, H, I, gm.data_ptr(),
                                       1, ym.data_ptr(), rm.data_ptr(), None, 0, st)
        if rc != 0:
            raise RuntimeError(f"MLP (2 launches) failed: {rc}")
    if "2launch" in forms:
        for i in range(20):
            launch_mlp2(i)
        mlp2_us = time_steps(torch, launch_mlp2, 200)
        # weights + scales, x and the residual in, h out and back in, y out
        mlp2_bytes = step_bytes + H * 2 * 2 + I * 2 * 2 + H * 2
        extras["mlp_config1_2launch_us"] = round(mlp2_us, 3)
        extras["mlp_config1_2launch_gbs"] = round(mlp2_bytes / (mlp2_us * 1e-6) / 1e9, 1)
    del Wgu, Sgu, Wdn, Sdn
    return extras


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100, help="timed steps (one GEMV over each weight copy)")
    ap.add_argument("--warmup", type=int, default=10, help="eager warm-up steps")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 256 MiB device copy (FETCH_SIZE/WRITE_SIZE calibration under rocprofv3)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extras", action="store_true", help="skip the M=16 and down-shape lines")
    ap.add_argument("--m16-only", action="store_true",
                    help="only time the M=16 verify (K=2560, N=10240) line (rocprofv3 counter runs)")
    ap.add_argument("--read-sweep", action="store_true",
                    help="only the streaming-read floor: launch shapes x sizes, fixed cost + bandwidth fit, and "
                         "the north-star I/O ladder (JSON lines)")
    ap.add_argument("--timeline", nargs="?", const="q4", default=None, choices=("q4", "q5", "q6", "w8"),
                    help="only the per-wave timeline of the M=1 GEMV at the north-star shape, Q4_G64 unless a "
                         "format is named (viper_hip_qlinear_timeline)")
    ap.add_argument("--timeline-rc", type=int, default=0, metavar="M",
                    help="only the per-wave timeline of the M-row matrix-core GEMM (Q4_G64, or W8_G32 with "
                         "--timeline w8; fragment input) at the north-star shape (viper_hip_qlinear_frag_timeline)")
    ap.add_argument("--shape", type=int, nargs=2, default=None, metavar=("K", "N"),
                    help="with --timeline / --timeline-rc: another shape than the north star's")
    ap.add_argument("--only", default="", metavar="LINE",
                    help="only one line (rocprofv3 runs): config0[_pre], down, verify_mM (K=2560 N=10240) or "
                         "verify_mM_down (K=10240 N=2560), pre_mM[_down] (the same through the prequantized "
                         "entry, x quantized once outside the timed calls), frag_mM[_down] (the same from "
                         "fragment-order rows), q5_m1 / q6_m8 / w8_m1 ... "
                         "(config 4), FMT_kK_nN_mM[_pre|_frag] (any shape, e.g. q4_k3072_n6144_m1), config1 / "
                         "config1_2launch (MLP), config3 (fused step), config3_prefetchW (the fused step with the next slot's "
                         "weights warmed from a second stream by W workgroups) or config3_ref (reference launch "
                         "sequence)")
    ap.add_argument("--clock-period", action="store_true",
                    help="only the north-star dispatch period on the device clock: back-to-back sequences of "
                         "10..200 launches between two clock stamps, span per length and the fitted slope "
                         "(JSON lines)")
    ap.add_argument("--trace-summary", default="", metavar="CSV",
                    help="only summarise a rocprofv3 kernel-trace CSV of this bench run with the same --steps "
                         "and --warmup (no GPU needed)")
    ap.add_argument("--dispatch-floor", action="store_true",
                    help="only the fixed cost of a dispatch: back-to-back launches of a kernel that reads nothing "
                         "(viper_hip_empty_dispatch) on one workgroup and on the north-star GEMV's grid, with and "
                         "without its row stores (JSON lines)")
    ap.add_argument("--verify-only", type=int, default=0, metavar="M",
                    help="only time the M-row verify (K=2560, N=10240) line (rocprofv3 runs)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (the GEMV would shard by "
              "output rows, each GPU running the same kernel on its share of N). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    if args.trace_summary:
        trace_summary(args.trace_summary, max(1, args.steps), max(0, args.warmup))
        return

    import torch
    import viper_amd as va

    if args.copy_calibration:
        torch.cuda.set_device(0)
        a = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": a.numel(), "launches": 5}), flush=True)
        return

    L = va.lib()
    torch.cuda.set_device(0)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x5EED0000)

    N, K, M = 10240, 2560, 1
    qtype, G = int(va.QType.Q4_G64), 64
    if args.only:
        one = args.only
        if one in ("config0", "config0_pre"):
            res = time_linear(torch, L, gen, qtype, 2560, 2560, 1, steps=args.steps,
                              prequantized=one == "config0_pre")
        elif one == "down":
            res = time_linear(torch, L, gen, qtype, 2560, 10240, 1, steps=args.steps)
        elif one.startswith("verify_m") or one.startswith("pre_m") or one.startswith("frag_m"):
            Mv = int(one.split("_m")[1].split("_")[0])
            shape = (2560, 10240) if one.endswith("_down") else (10240, 2560)
            res = time_linear(torch, L, gen, qtype, shape[0], shape[1], Mv, steps=args.steps,
                              prequantized=one.startswith("pre_m"), frag=one.startswith("frag_m"))
        elif re.fullmatch(r"(q4|q5|q6|w8)_k\d+_n\d+_m\d+(_pre|_frag)?", one):
            fmt, kk, nn, mm = one.split("_")[:4]
            qt = {"q4": 4, "q5": 5, "q6": 6, "w8": 8}[fmt]
            res = time_linear(torch, L, gen, qt, int(nn[1:]), int(kk[1:]), int(mm[1:]), steps=args.steps,
                              outliers=qt != 4, prequantized=one.endswith("_pre"), frag=one.endswith("_frag"))
        elif one[:1] in "qw" and "_m" in one:
            fmt, mpart = one.split("_m")
            qt = {"q5": 5, "q6": 6, "w8": 8}[fmt]
            res = time_linear(torch, L, gen, qt, N, K, int(mpart), steps=args.steps, outliers=True)
        elif one in ("config1", "config1_2launch"):
            r = time_mlp(torch, L, gen, qtype, G, ("ref",) if one == "config1" else ("2launch",))
            key = "mlp_config1_us" if one == "config1" else "mlp_config1_2launch_us"
            res = (r[key], r[key.replace("_us", "_gbs")])
        elif one in ("config3", "config3_ref") or one.startswith("config3_prefetch"):
            from viper_amd.stack import Stack
            pf = int(one.split("config3_prefetch")[1] or 128) if one.startswith("config3_prefetch") else 0
            us, gbs, _ = time_config3(torch, Stack(torch), one != "config3_ref", replays=max(10, args.steps // 100),
                                      prefetch=pf)
            res = (us, gbs)
        else:
            raise SystemExit(f"unknown --only line {one}")
        print(json.dumps({"line": one, "us": res[0], "gbs": res[1]}), flush=True)
        return
    if args.read_sweep:
        read_sweep(torch, L, gen)
        return
    if args.dispatch_floor:
        dispatch_floor(torch, L)
        return
    if args.timeline_rc:
        Kt, Nt = (args.shape[0], args.shape[1]) if args.shape else (K, N)
        timeline_rc(torch, L, gen, Nt, Kt, args.timeline_rc, 8 if args.timeline == "w8" else 4)
        return
    if args.timeline:
        Kt, Nt = (args.shape[0], args.shape[1]) if args.shape else (K, N)
        timeline(torch, L, gen, Nt, Kt, {"q4": 4, "q5": 5, "q6": 6, "w8": 8}[args.timeline])
        return
    if args.m16_only or args.verify_only:
        Mv = 16 if args.m16_only else args.verify_only
        us, gbs = time_linear(torch, L, gen, qtype, N, K, Mv, steps=args.steps)
        print(json.dumps({"workload": f"Q4_G64 M={Mv} verify K=2560 N=10240", "us": us, "gbs": gbs}), flush=True)
        return
    copy_bytes = N * K // 2 + N * (K // G) * 2
    copies = max(2, -(-ROTATE_BYTES // copy_bytes) + 1)
    W, S = make_weights(torch, copies, N, K, gen)
    x = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    alg = algorithmic_bytes(K // 2, N, K, M)
    wp = [W[i].data_ptr() for i in range(copies)]
    spp = [S[i].data_ptr() for i in range(copies)]

    def launch(i):
        c = i % copies
        rc = L.viper_hip_qlinear(qtype, wp[c], spp[c], 0, G, N, K, x.data_ptr(), M, y.data_ptr(),
                                 None, None, 0, torch.cuda.current_stream().cuda_stream)
        if rc != 0:
            raise RuntimeError(f"viper_hip_qlinear failed: {rc}")

    if args.clock_period:
        for i in range(20 * copies):
            launch(i)
        counts = (10, 20, 40, 80, 120, 160, 200)
        for rep in range(3):
            per, icpt, rows = clock_period(torch, L, launch, counts=counts, replays=20)
            for n, span in rows:
                print(json.dumps({"rep": rep, "launches": n, "span_us": round(span, 3)}), flush=True)
            print(json.dumps({"rep": rep, "fit": "span = intercept + period * launches",
                              "period_us": round(per, 4), "intercept_us": round(icpt, 3),
                              "gbs": round(alg / (per * 1e-6) / 1e9, 1),
                              "frac": round(alg / (per * 1e-6) / 1e9 / PEAK_GBS, 4)}), flush=True)
        return

    # exactly --steps steps of `copies` dispatches each, after --warmup eager steps
    steps, warmup = max(1, args.steps), max(0, args.warmup)
    for i in range(warmup * copies):
        launch(i)
    full, rest = divmod(steps, GRAPH_STEPS)
    graphs = []
    if full:
        graphs.append((capture_n(torch, launch, GRAPH_STEPS * copies), full))
    if rest:
        graphs.append((capture_n(torch, launch, rest * copies), 1))
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for g, reps in graphs:
        for _ in range(reps):
            g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    job_ms = e0.elapsed_time(e1)
    dispatches = steps * copies
    del graphs
    ms_per_step = job_ms / steps
    us_per_gemv = job_ms * 1e3 / dispatches
    value = alg * dispatches / (job_ms * 1e-3) / 1e9
    achieved = value
    # the same dispatch period on the device's clock (slope over back-to-back sequences of 40 and 120
    # launches): a cross-check of the events that no profiler perturbs
    clk_us, clk_icpt, _ = clock_period(torch, L, launch)

    extras = {}
    if not args.no_extras:
        # the floor of one dispatch streaming the same bytes: a read-only kernel with the GEMV's launch
        # shape over the same rotating copies (viper_hip_stream_read): the weights alone, then the GEMV's
        # whole I/O (weights, each workgroup's block of scales, one bf16 store per row)
        sink = torch.zeros(4, dtype=torch.int32, device="cuda")
        wbytes = N * K // 2
        sblock = (N // 512) * (K // G) * 2

        def launch_read(i, io=False):
            c = i % copies
            rc = L.viper_hip_stream_read(wp[c], wbytes, 320, 5, spp[c] if io else None, sblock if io else 0,
                                         y.data_ptr() if io else None, sink.data_ptr(),
                                         torch.cuda.current_stream().cuda_stream)
            if rc != 0:
                raise RuntimeError(f"viper_hip_stream_read failed: {rc}")
        for i in range(20):
            launch_read(i)
            launch_read(i, True)
        read_us = time_steps(torch, launch_read, max(10 * copies, MIN_STEPS))
        io_us = time_steps(torch, lambda i: launch_read(i, True), max(10 * copies, MIN_STEPS))
        extras["stream_read_weights_us"] = round(read_us, 3)
        extras["stream_read_weights_gbs"] = round(wbytes / (read_us * 1e-6) / 1e9, 1)
        extras["stream_read_gemv_io_us"] = round(io_us, 3)

        # M=16 speculative verify (K=2560, N=10240): quantize kernel + GEMM
        M16 = 16
        x16 = torch.randn((M16, K), device="cuda", generator=gen).to(torch.bfloat16)
        y16 = torch.empty((M16, N), dtype=torch.bfloat16, device="cuda")
        nws = va.workspace_bytes(qtype, N, K, M16)
        ws16 = torch.zeros(nws, dtype=torch.uint8, device="cuda")

        def launch16(i):
            c = i % copies
            rc = L.viper_hip_qlinear(qtype, wp[c], spp[c], 0, G, N, K, x16.data_ptr(), M16, y16.data_ptr(),
                                     None, ws16.data_ptr(), nws, torch.cuda.current_stream().cuda_stream)
            if rc != 0:
                raise RuntimeError(f"M=16 qlinear failed: {rc}")
        for i in range(50):
            launch16(i)
        m16_us = time_steps(torch, launch16, 400)
        alg16 = algorithmic_bytes(K // 2, N, K, M16)
        extras["m16_verify_us"] = round(m16_us, 3)
        extras["m16_verify_gbs"] = round(alg16 / (m16_us * 1e-6) / 1e9, 1)

        # config 2: the other speculative-verify row counts at the north-star shape, and M=16 at the
        # down-projection shape
        for Mv in (2, 4, 8):
            us_v, gbs_v = time_linear(torch, L, gen, qtype, N, K, Mv)
            extras[f"verify_m{Mv}_us"], extras[f"verify_m{Mv}_gbs"] = us_v, gbs_v
        for Mv in (2, 4, 8, 16):
            us_v, gbs_v = time_linear(torch, L, gen, qtype, 2560, 10240, Mv)
            extras[f"verify_m{Mv}_down_us"], extras[f"verify_m{Mv}_down_gbs"] = us_v, gbs_v
        # the engine's verify step: rows quantized by the producer in the matrix-core fragment order,
        # one launch per linear (the K split with its workspace at the down shape)
        for Mv in (8, 16):
            for nm, (Nf, Kf) in (("", (N, K)), ("_down", (2560, 10240))):
                us_v, gbs_v = time_linear(torch, L, gen, qtype, Nf, Kf, Mv, frag=True)
                extras[f"verify_m{Mv}{nm}_frag_us"], extras[f"verify_m{Mv}{nm}_frag_gbs"] = us_v, gbs_v

        # config 0: the attention q/o projection, Q4_G64 M=1, K=N=2560
        us_v, gbs_v = time_linear(torch, L, gen, qtype, 2560, 2560, 1)
        extras["config0_us"], extras["config0_gbs"] = us_v, gbs_v

        # the prequantized entry (the reference engine's dp4a_smem_gemv call sites: int8 rows quantized
        # by the producer kernel): M=1 at the three shapes, 2-4 rows at the down shape
        for nm, (Nq, Kq), Mv in (("pre_config0", (2560, 2560), 1), ("pre_m1", (N, K), 1),
                                 ("pre_m1_down", (2560, 10240), 1), ("pre_m2_down", (2560, 10240), 2),
                                 ("pre_m3_down", (2560, 10240), 3), ("pre_m4_down", (2560, 10240), 4)):
            us_v, gbs_v = time_linear(torch, L, gen, qtype, Nq, Kq, Mv, prequantized=True)
            extras[f"{nm}_us"], extras[f"{nm}_gbs"] = us_v, gbs_v

        # config 4: Q5_G64, Q6_G64 and W8_G32 at M=1 and M=8, K=2560, N=10240
        for qt, nm in ((5, "q5"), (6, "q6"), (8, "w8")):
            for Mv in (1, 8):
                us_v, gbs_v = time_linear(torch, L, gen, qt, N, K, Mv, outliers=True)
                extras[f"{nm}_m{Mv}_us"], extras[f"{nm}_m{Mv}_gbs"] = us_v, gbs_v

        # the reference engine's own linears (include/viper/model_impl.cuh:107-116: hidden 3072,
        # intermediate 10752, 48 x 128 query heads): q 3072 -> 6144, o 6144 -> 3072, gate (and up)
        # 3072 -> 10752, down 10752 -> 3072, one decode row and a 16-row verify
        for nm, (Ne, Ke) in (("engine_q", (6144, 3072)), ("engine_o", (3072, 6144)),
                             ("engine_gate", (10752, 3072)), ("engine_down", (3072, 10752))):
            for Mv in (1, 16):
                us_v, gbs_v = time_linear(torch, L, gen, qtype, Ne, Ke, Mv)
                extras[f"{nm}_m{Mv}_us"], extras[f"{nm}_m{Mv}_gbs"] = us_v, gbs_v

        # down projection shape (K=10240, N=2560), M=1, fused quantize
        Kd, Nd = 10240, 2560
        Wd, Sd = make_weights(torch, copies, Nd, Kd, gen)
        xd = torch.randn((1, Kd), device="cuda", generator=gen).to(torch.bfloat16)
        yd = torch.empty((1, Nd), dtype=torch.bfloat16, device="cuda")
        wdp = [Wd[i].data_ptr() for i in range(copies)]
        sdp = [Sd[i].data_ptr() for i in range(copies)]

        def launchd(i):
            c = i % copies
            rc = L.viper_hip_qlinear(qtype, wdp[c], sdp[c], 0, G, Nd, Kd, xd.data_ptr(), 1, yd.data_ptr(),
                                     None, None, 0, torch.cuda.current_stream().cuda_stream)
            if rc != 0:
                raise RuntimeError(f"down qlinear failed: {rc}")
        for i in range(50):
            launchd(i)
        d_us = time_steps(torch, launchd, 400)
        algd = algorithmic_bytes(Kd // 2, Nd, Kd, 1)
        extras["down_k10240_n2560_us"] = round(d_us, 3)
        extras["down_k10240_n2560_gbs"] = round(algd / (d_us * 1e-6) / 1e9, 1)
        del Wd, Sd

        # config 1: gate+up (one fused2 launch, K=2560, N=2x10240) -> swiglu +
        # quantize -> down (K=10240, N=2560) + residual; one step = 3 launches
        extras.update(time_mlp(torch, L, gen, qtype, G))

        # LM head (config 3's head): bf16 GEMV K=2560, N=166144 (850 MB, larger
        # than the MALL, so one copy streams from HBM every call) + greedy argmax
        Nv = 166144
        Wh = (0.02 * torch.randn((Nv, K), device="cuda", generator=gen)).to(torch.bfloat16)
        xh = torch.randn((1, K), device="cuda", generator=gen).to(torch.bfloat16)
        yh = torch.empty((1, Nv), dtype=torch.bfloat16, device="cuda")
        th = torch.empty(1, dtype=torch.int32, device="cuda")

        def launch_head(i):
            st = torch.cuda.current_stream().cuda_stream
            rc = L.viper_hip_linear_bf16(Wh.data_ptr(), xh.data_ptr(), yh.data_ptr(), 1, Nv, K, st)
            if rc != 0:
                raise RuntimeError(f"LM head failed: {rc}")

        gws = torch.zeros(16, dtype=torch.uint8, device="cuda")

        def launch_greedy(i, split=False):
            st = torch.cuda.current_stream().cuda_stream
            if split:
                rc = L.viper_hip_sampling_greedy_split(yh.data_ptr(), th.data_ptr(), 1, Nv, gws.data_ptr(), 16, st)
            else:
                rc = L.viper_hip_sampling_greedy(yh.data_ptr(), th.data_ptr(), 1, Nv, st)
            if rc != 0:
                raise RuntimeError(f"greedy failed: {rc}")
        for i in range(5):
            launch_head(i)
            launch_greedy(i)
            launch_greedy(i, True)
        head_us = time_steps(torch, launch_head, 50)
        greedy_us = time_steps(torch, launch_greedy, 200)
        greedy_split_us = time_steps(torch, lambda i: launch_greedy(i, True), 200)
        head_bytes = Nv * K * 2 + K * 2 + Nv * 2
        extras["lm_head_us"] = round(head_us, 3)
        extras["lm_head_gbs"] = round(head_bytes / (head_us * 1e-6) / 1e9, 1)
        extras["greedy_argmax_us"] = round(greedy_us, 3)
        extras["greedy_argmax_split_us"] = round(greedy_split_us, 3)
        del Wh

        # config 3: 22 weight sets x 2 passes (44 slots) of the linear path +
        # final norm + bf16 LM head + greedy token, one step = one graph replay;
        # the reference launch sequence, then the producers folded into the
        # GEMVs (4 launches per slot)
        from viper_amd.stack import Stack
        stk = Stack(torch)
        for fused, key in ((False, "config3"), (True, "config3_fused")):
            us, gbs, launches = time_config3(torch, stk, fused)
            extras[f"{key}_step_us"] = us
            extras[f"{key}_step_gbs"] = gbs
            extras[f"{key}_launches_per_step"] = launches
        del stk

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic_q4_m1_k2560_n10240.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    cpu = None
    if not args.no_cpu:
        t1, tm, nth = cpu_baseline(N, K, reps_1t=10, reps_mt=40)
        cpu = {"value": round(alg / tm / 1e9, 3), "unit": "GB/s", "cores": nth, "kind": "port",
               "sample": (f"oracle C restatement (vo_qlinear_omp), Q4_G64 M=1 K={K} N={N}, seeded inputs; "
                          f"{nth} threads: {tm * 1e3:.2f} ms/GEMV over 40 runs; "
                          f"1 thread: {t1 * 1e3:.2f} ms/GEMV ({alg / t1 / 1e9:.3f} GB/s) over 10 runs")}

    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded: uniform int4 weights, fp16 log-uniform scales, bf16 N(0,1) x)",
        "config": {"workload": "Q4_G64 GEMV M=1 K=2560 N=10240 (north star), fused bf16->int8 quantize",
                   "qtype": "Q4_G64", "M": M, "K": K, "N": N, "weight_copies": copies,
                   "rotation_bytes": copies * copy_bytes, "algorithmic_bytes_per_gemv": alg,
                   "algorithmic_bytes_per_step": alg * copies,
                   "step": f"one GEMV over each of the {copies} weight copies ({copies} dispatches)",
                   "timed_region": (f"{steps} steps = {dispatches} dispatches: HIP graphs of up to {GRAPH_STEPS} steps, "
                                    f"each replayed once untimed, then back to back between events on the stream, "
                                    f"after {warmup} eager warm-up steps")},
        "us_per_gemv": round(us_per_gemv, 3),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_GBS, 4), "traffic": traffic,
                     "us_per_launch": round(us_per_gemv, 3), "device_clock_us_per_launch": round(clk_us, 3),
                     "device_clock_frac": round(alg / (clk_us * 1e-6) / 1e9 / PEAK_GBS, 4)},
        "cpu_baseline": cpu,
    }
    out.update(extras)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
