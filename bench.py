#!/usr/bin/env python3
"""Benchmark of the quantized decode hot path on one MI355X.

Headline workload (the metric's isolated-matvec configuration): y = W x with
fp32 x ~ N(0,1) of length 4096 and weights N(0, 0.02) quantized to Q8_0 and
Q4_0, shapes 4096x4096 and 11008x4096, batch 1.  One step = one matvec of
each of the four (format, shape) cases.  Each case cycles through a pool of
distinct weight copies larger than the 256 MB Infinity Cache, so every launch
streams its weights from HBM.  The K timed steps are captured in one HIP
graph (step by step, each step the four launches in order) and bracketed by
HIP events on the stream they run on; `value` is the total algorithmic bytes
of all K steps over the timed time.  Per-case figures (and the roofline's
kernel time) come from a second timing, each case's max(K, 200) launches in
a graph of their own between events.
Algorithmic bytes per launch = weight bytes + 4*K (x) + 4*N (y).

The same JSON line also reports the other configurations of the metric:
  decode_b1    SmolLM2-135M architecture, Q8_0, batch 1: seeded 32-token
               prompt, 128 greedy tokens (decode-only and prefill+decode tok/s)
  decode_b128  Qwen2.5-3B architecture, Q4_0, tied head, QKV bias, f32 KV
               pages (the reference's KVCache): 128 concurrent sequences,
               prompts U[16,512], outputs U[64,256], new requests admitted as
               others finish; aggregate generated tok/s; fp16 and int8 pages
               reported beside it with their streams' agreement with the f32
               run
  gemm         batched Q-GEMM, B in {8,32,64,128}, Qwen2.5-3B projection shapes
  gemm_library (not in the default run) hipBLASLt's bf16 GEMM (torch.mm) at the
               same shapes: one bf16 product, no dequantisation, a yardstick
  attention    ragged paged decode attention: 128 sequences, context U[128,4096],
               16 q / 2 kv heads, head_dim 128, fp16 K/V
  sampler      the device sampler on 128 rows x 151936 logits (penalty,
               temperature, top-k, top-p); the reference's Sampler per row on
               the host beside it
  load         QRAF file -> HBM (qraf_engine_create_from_file) of the
               Qwen2.5-3B-architecture Q4 model, from a file this leg writes
  steady_b128  (not in the default run) the steady 128-sequence decode of
               decode_b128 alone, in its own engine, for a profile whose every
               GEMM runs at 128 rows
All weights are synthetic (N(0,0.02), generated and quantized on the GPU).

    python bench.py [--gpus 1] [--steps 1000] [--warmup 50] [--cpu-seconds 12] [--only matvec,gemm,...]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q4/Q8 decode tok/s at batch 1 & 128; qmatvec achieved HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0      # MI355X published HBM3E bandwidth
MFMA_BF16_TFLOPS = 2500.0  # MI355X published dense bf16 matrix peak (the GEMM issues 2 MFMAs per product: hi + lo)
POOL_BYTES = 320 << 20     # > 256 MB MALL
Q8, Q4, F32, F16, I8 = 10, 20, 0, 1, 102
MV_CASES = [("q8_0", Q8, 4096, 4096), ("q8_0", Q8, 11008, 4096), ("q4_0", Q4, 4096, 4096), ("q4_0", Q4, 11008, 4096)]
GEMM_SHAPES = [(2048, 2048), (256, 2048), (11008, 2048), (2048, 11008)]


def row_bytes(dt, k):
    return (k // 32) * (36 if dt == Q8 else 18)


def mv_bytes(dt, n, k, b=1):
    return n * row_bytes(dt, k) + 4 * b * k + 4 * b * n


def host_cpu():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def graph_time_us(rt, body, iters):
    """Capture `iters` calls of body(i) in one graph; replay once untimed, then
    time one replay with events on the stream; microseconds per call.  With
    rt["eager"] (--no-graphs): the calls are launched directly, once untimed
    and once between the events."""
    stream, Graph, Event = rt["stream"], rt["Graph"], rt["Event"]
    if rt.get("eager"):
        for i in range(iters):
            body(i)
        stream.synchronize()
        e0, e1 = Event(), Event()
        e0.record(stream)
        for i in range(iters):
            body(i)
        e1.record(stream)
        return e0.elapsed_ms(e1) * 1e3 / iters
    g = Graph(stream)
    with g:
        for i in range(iters):
            body(i)
    g.launch()
    stream.synchronize()
    e0, e1 = Event(), Event()
    e0.record(stream)
    g.launch()
    e1.record(stream)
    us = e0.elapsed_ms(e1) * 1e3 / iters
    g.destroy()
    return us


# --------------------------------------------------------------------------- matvec (headline)

# HBM bytes per launch from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs of this
# bench (scaled by the counters' reading for a copy kernel of known size);
# reported only for the kernel they were measured on.
MEASURED_TRAFFIC = {("qmv_ring_kernel<8, 1, 2, 2, 8>", "q8_0 11008x4096"): 50937856}


def ring_kernel_name(case):
    """Template name of the ring kernel the automatic choice runs for a C2 case
    ('q8_0 11008x4096'): <format, rows per wave, x loads per thread, depth, waves per workgroup>."""
    fmt, shape = case.split()
    n, k = (int(v) for v in shape.split("x"))
    q8 = fmt == "q8_0"
    nw = 4 if (not q8 and n >= 8192) else 8
    r = 2 if (not q8 and n >= 8192 and n % 2 == 0) else 1
    per = 64 * nw * (4 if q8 else 8)
    xj = -(-k // per)
    xj = next(v for v in (1, 2, 4, 8, 12) if v >= xj)
    return f"qmv_ring_kernel<{8 if q8 else 4}, {r}, {xj}, 2, {nw}>"


def bench_matvec(args, rt):
    call, DeviceBuffer, Event, Graph, stream, lib = (rt[k] for k in ("call", "DeviceBuffer", "Event", "Graph", "stream",
                                                                     "lib"))
    rng = np.random.default_rng(2024)
    x_host = rng.standard_normal(4096).astype(np.float32)
    cases = []
    wanted = [c.strip() for c in args.cases.split(",") if c.strip()] if args.cases else None
    for (name, dt, n, k) in MV_CASES:
        if wanted is not None and f"{name} {n}x{k}" not in wanted:
            continue
        wbytes = n * row_bytes(dt, k)
        copies = max(2, math.ceil(POOL_BYTES / wbytes))
        pool = DeviceBuffer(copies * wbytes)
        sid = lib.qraf_hip_name_hash(f"bench.{name}.{n}x{k}".encode())
        call("qraf_hip_gen_weights_dev", pool.ptr, dt, n * k, 2024, sid, 0.02, stream.h)
        for c in range(1, copies):
            call("qraf_hip_memcpy_d2d", pool.ptr + c * wbytes, pool.ptr, wbytes, stream.h)
        cases.append(dict(name=name, dt=dt, n=n, k=k, wbytes=wbytes, copies=copies, pool=pool,
                          x=DeviceBuffer.from_array(x_host), y=DeviceBuffer(n * 4)))
    stream.synchronize()

    def launch(c, i):
        call("qraf_hip_matvec_q_dev", c["pool"].ptr + (i % c["copies"]) * c["wbytes"], c["dt"], 32, c["n"], c["k"],
             c["x"].ptr, c["y"].ptr, stream.h)

    for i in range(args.warmup):
        for c in cases:
            launch(c, i)
    stream.synchronize()
    # per-case launches: at least 200, so that one graph launch's fixed cost
    # (10-13 us of GPU time) stays within about 1% of a launch's figure
    kc = max(args.steps, 200)
    graphs = []
    if not rt.get("eager"):
        for c in cases:
            g = Graph(stream)
            with g:
                for i in range(kc):
                    launch(c, args.warmup + i)
            graphs.append(g)
        for g in graphs:  # one untimed replay: graph upload stays out of the timed region
            g.launch()
        stream.synchronize()
    # the K timed steps: one graph of K steps, each step the four matvecs in order
    step_graph = None
    if not rt.get("eager"):
        step_graph = Graph(stream)
        with step_graph:
            for i in range(args.steps):
                for c in cases:
                    launch(c, args.warmup + i)
        step_graph.launch()  # untimed: graph upload stays out of the timed region
        stream.synchronize()
    e0, e1 = Event(), Event()
    call("qraf_hip_device_synchronize")
    e0.record(stream)
    if step_graph:
        step_graph.launch()
    else:
        for i in range(args.steps):
            for c in cases:
                launch(c, args.warmup + i)
    e1.record(stream)
    stream.synchronize()
    call("qraf_hip_device_synchronize")
    total_ms = e0.elapsed_ms(e1)
    total_bytes = sum(mv_bytes(c["dt"], c["n"], c["k"]) for c in cases) * args.steps
    if step_graph:
        step_graph.destroy()
    # per case: each case's kc launches in a graph of their own, between events
    ev = [Event() for _ in range(len(cases) + 1)]
    call("qraf_hip_device_synchronize")
    ev[0].record(stream)
    for i, c in enumerate(cases):
        if graphs:
            graphs[i].launch()
        else:
            for j in range(kc):
                launch(c, args.warmup + j)
        ev[i + 1].record(stream)
    stream.synchronize()
    call("qraf_hip_device_synchronize")
    per_case = []
    for i, c in enumerate(cases):
        ms = ev[i].elapsed_ms(ev[i + 1])
        b = mv_bytes(c["dt"], c["n"], c["k"])
        us = ms * 1e3 / kc
        per_case.append({"case": f"{c['name']} {c['n']}x{c['k']}", "us_per_launch": round(us, 3), "alg_bytes": b,
                         "GB_s": round(b / (us * 1e-6) / 1e9, 1),
                         "frac_hbm_peak": round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "pool_copies": c["copies"]})
    for g in graphs:
        g.destroy()
    # plain-read ceiling: a streaming read of the same bytes from the same rotated pool copies
    rp_out = DeviceBuffer(lib.qraf_hip_read_probe_out_bytes())
    for c, p in zip(cases, per_case):
        b = mv_bytes(c["dt"], c["n"], c["k"])
        us = graph_time_us(rt, lambda i: call("qraf_hip_read_probe_dev", c["pool"].ptr + (i % c["copies"]) * c["wbytes"],
                                              c["wbytes"], rp_out.ptr, stream.h), kc)
        p["plain_read_us"] = round(us, 3)
        p["plain_read_GB_s"] = round(c["wbytes"] / (us * 1e-6) / 1e9, 1)
        p["frac_of_plain_read"] = round(us / p["us_per_launch"], 4)  # plain-read time / matvec time
    rp_out.free()
    # cache-resident reference point (same weight copy every launch), labelled as such
    cache_res = []
    for c in cases:
        us = graph_time_us(rt, lambda i: call("qraf_hip_matvec_q_dev", c["pool"].ptr, c["dt"], 32, c["n"], c["k"],
                                              c["x"].ptr, c["y"].ptr, stream.h), 200)
        cache_res.append({"case": f"{c['name']} {c['n']}x{c['k']}",
                          "GB_s": round(mv_bytes(c["dt"], c["n"], c["k"]) / (us * 1e-6) / 1e9, 1)})
    hosts = [(c["name"], c["dt"], c["n"], c["k"], c["pool"].download(np.uint8, c["wbytes"]), x_host) for c in cases]
    for c in cases:
        c["pool"].free()
    return total_bytes / (total_ms * 1e-3) / 1e9, total_ms, per_case, cache_res, hosts


def cpu_baseline_matvec(cases_host, budget_s):
    """The reference's own scalar matvec (oracle/_ref, compiled from the
    reference sources) on this host, one thread; the oracle's restatement
    when the reference build is absent."""
    from oracle import pyoracle as po
    R = po.ref()
    kind = "reference" if R is not None else "port"
    per = budget_s / len(cases_host)
    tot_bytes, tot_time, parts = 0, 0.0, []
    for (name, dt, n, k, wq, x) in cases_host:
        y = np.zeros(n, np.float32)
        it, t0 = 0, time.perf_counter()
        while True:
            if R is not None:
                R.ref_matvec_q(wq.ctypes.data, dt, 32, n, k, x.ctypes.data_as(po._fp), y.ctypes.data_as(po._fp))
            else:
                po.lib().or_matvec_q(wq.ctypes.data, dt, 32, n, k, x.ctypes.data_as(po._fp), y.ctypes.data_as(po._fp))
            it += 1
            el = time.perf_counter() - t0
            if el >= per:
                break
        tot_bytes += it * mv_bytes(dt, n, k)
        tot_time += el
        parts.append(f"{name} {n}x{k}: {it} iters")
    return {"value": round(tot_bytes / tot_time / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": kind,
            "sample": "; ".join(parts) + f" of dispatch_matvec_q (the scalar x86 path), one thread, {tot_time:.1f} s, "
                      f"host CPU {host_cpu()}"}


# --------------------------------------------------------------------------- batched GEMM

def batch_matvec_covered(dt, k, nv):
    """qraf_hip_matvec_q_batch_dev's coverage: K a multiple of 32 (64 for
    Q4_0), the batch rounded up to 2/4/8/16 vectors staged in 144 KB."""
    if k % (32 if dt == Q8 else 64):
        return False
    nvr = 2 if nv <= 2 else 4 if nv <= 4 else 8 if nv <= 8 else 16
    per = (k // 32) * 36 * 4 if dt == Q8 else (k // 64) * 76 * 4
    return nvr * per <= 144 * 1024


def bench_gemm(args, rt):
    call, DeviceBuffer, stream, lib = rt["call"], rt["DeviceBuffer"], rt["stream"], rt["lib"]
    rng = np.random.default_rng(7)
    out = []
    want = [c.strip() for c in args.gemm_cases.split(",") if c.strip()]
    for dt, fmt in ((Q8, "q8_0"), (Q4, "q4_0")):
        for (n, k) in GEMM_SHAPES:
            batches = [b for b in (8, 32, 64, 128) if not want or f"{fmt} {n}x{k} B={b}" in want]
            if not batches:
                continue
            wbytes = n * row_bytes(dt, k)
            copies = max(2, math.ceil(POOL_BYTES / wbytes))
            pool = DeviceBuffer(copies * wbytes)
            call("qraf_hip_gen_weights_dev", pool.ptr, dt, n * k, 7, lib.qraf_hip_name_hash(b"bench.gemm"), 0.02,
                 stream.h)
            for c in range(1, copies):
                call("qraf_hip_memcpy_d2d", pool.ptr + c * wbytes, pool.ptr, wbytes, stream.h)
            # the engine's form: a tile-major copy (same bytes, reordered at load time)
            tbytes = lib.qraf_hip_tiled_weight_bytes(dt, n, k)
            tcopies = max(2, math.ceil(POOL_BYTES / tbytes))
            tpool = DeviceBuffer(tcopies * tbytes)
            for c in range(tcopies):
                call("qraf_hip_repack_tiles_dev", pool.ptr + (c % copies) * wbytes, dt, n, k, tpool.ptr + c * tbytes,
                     stream.h)
            for b in batches:
                dx = DeviceBuffer.from_array(rng.standard_normal((b, k)).astype(np.float32))
                xh, xl, y = DeviceBuffer(b * k * 2), DeviceBuffer(b * k * 2), DeviceBuffer(b * n * 4)
                call("qraf_hip_split_bf16_dev", dx.ptr, xh.ptr, xl.ptr, b, k, stream.h)
                wsb = lib.qraf_hip_qgemm_workspace_bytes(dt, n, k, b)
                ws = DeviceBuffer(wsb) if wsb else None
                us_ref = graph_time_us(rt, lambda i: call("qraf_hip_qgemm_dev", pool.ptr + (i % copies) * wbytes, dt,
                                                          32, n, k, xh.ptr, xl.ptr, b, y.ptr, None,
                                                          ws.ptr if ws else None, wsb, stream.h), 100)
                wsbt = lib.qraf_hip_qgemm_tiled_workspace_bytes(dt, n, k, b)
                wst = DeviceBuffer(wsbt) if wsbt else None
                us = graph_time_us(rt, lambda i: call("qraf_hip_qgemm_tiled_dev", tpool.ptr + (i % tcopies) * tbytes,
                                                      dt, n, k, xh.ptr, xl.ptr, b, y.ptr, None,
                                                      wst.ptr if wst else None, wsbt, stream.h), 100)
                by, fl = mv_bytes(dt, n, k, b), 2.0 * b * n * k
                rec = {"case": f"{fmt} {n}x{k} B={b}", "us": round(us, 2),
                       "GB_s": round(by / (us * 1e-6) / 1e9, 1), "TFLOPs": round(fl / (us * 1e-6) / 1e12, 2),
                       "mfma_frac": round(2 * fl / (us * 1e-6) / 1e12 / MFMA_BF16_TFLOPS, 4),
                       "us_reference_layout": round(us_ref, 2)}
                rec["engine_form"] = ("batch matvec" if 2 <= b <= 8 and batch_matvec_covered(dt, k, b)
                                      and b * n * k <= 96 << 20 else "GEMM")
                if b <= 8 and batch_matvec_covered(dt, k, b):
                    # below the matrix cores' batch: the multi-vector matvec on the
                    # reference layout, fp32 x as is (the engine's form for 2-8 rows)
                    us_mv = graph_time_us(rt, lambda i: call("qraf_hip_matvec_q_batch_dev",
                                                             pool.ptr + (i % copies) * wbytes, dt, n, k, dx.ptr, b,
                                                             y.ptr, stream.h), 100)
                    rec.update({"us_batch_matvec": round(us_mv, 2),
                                "GB_s_batch_matvec": round(by / (us_mv * 1e-6) / 1e9, 1),
                                "frac_hbm_batch_matvec": round(by / (us_mv * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
                out.append(rec)
                for d in (dx, xh, xl, y):
                    d.free()
            pool.free()
            tpool.free()
    return out


def bench_gemm_library(args, rt):
    """Yardstick for the tiled Q-GEMM: the platform's tuned bf16 GEMM
    (torch.mm, which runs hipBLASLt) at the same shapes, y[B,N] = x[B,K] W^T
    with bf16 W[N,K] in the weights' row-major layout: ONE bf16 product per
    output (the Q-GEMM issues two, hi and lo planes), no dequantisation, 2 bytes
    per weight (Q4_0: 0.5625).  Weights rotate through >320 MB so they stream
    from HBM; 20 calls captured in one torch CUDA graph, one replay timed with
    events (the results are not read).  Not in the default run.  Measured in a
    child process: torch's own HIP runtime does not find the device in a
    process where this library's runtime already holds it."""
    import subprocess
    r = subprocess.run([sys.executable, os.path.abspath(__file__), "--gemm-library-child"], capture_output=True,
                       text=True, timeout=600)
    if r.returncode != 0:
        raise RuntimeError(f"gemm_library child failed ({r.returncode}):\n{r.stderr[-3000:]}")
    return json.loads(r.stdout.strip().split("\n")[-1])


def gemm_library_child():
    import torch
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    shapes = [(n, k, b) for (n, k) in GEMM_SHAPES for b in (8, 32, 64, 128)]
    shapes += [(22016, 2048, 128), (2560, 2048, 128), (151936, 2048, 128)]  # gate/up, QKV, tied head at 128 rows
    out, iters = [], 20
    for (n, k, b) in shapes:
        copies = max(2, math.ceil(POOL_BYTES / (n * k * 2)))
        pool = torch.empty((copies, n, k), dtype=torch.bfloat16, device=dev).normal_(0.0, 0.02, generator=gen)
        x = torch.empty((b, k), dtype=torch.bfloat16, device=dev).normal_(generator=gen)
        y = torch.empty((b, n), dtype=torch.bfloat16, device=dev)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for i in range(3):
                torch.mm(x, pool[i % copies].t(), out=y)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(iters):
                torch.mm(x, pool[i % copies].t(), out=y)
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / iters
        fl = 2.0 * b * n * k
        out.append({"case": f"bf16 {n}x{k} B={b}", "us": round(us, 2), "TFLOPs": round(fl / (us * 1e-6) / 1e12, 1),
                    "frac_bf16_peak": round(fl / (us * 1e-6) / 1e12 / MFMA_BF16_TFLOPS, 4)})
        del graph, pool, x, y
        torch.cuda.empty_cache()
    print(json.dumps(out), flush=True)


# --------------------------------------------------------------------------- attention

def bench_attention(args, rt):
    call, DeviceBuffer, stream, lib = rt["call"], rt["DeviceBuffer"], rt["stream"], rt["lib"]
    rng = np.random.default_rng(2024)
    n, H, Hkv, hd, ps, max_ctx = 128, 16, 2, 128, 16, 4096
    ctxs = rng.integers(128, max_ctx + 1, n).astype(np.int32)
    max_pages = max_ctx // ps
    num_pages = int(sum((c + ps - 1) // ps for c in ctxs))
    table = np.zeros((n, max_pages), np.int32)
    perm = rng.permutation(num_pages).astype(np.int32)
    k = 0
    for s, c in enumerate(ctxs):
        m = (c + ps - 1) // ps
        table[s, :m] = perm[k:k + m]
        k += m
    q = DeviceBuffer.from_array(rng.standard_normal((n, H * hd)).astype(np.float32))
    dt_, dc = DeviceBuffer.from_array(table), DeviceBuffer.from_array(ctxs)
    out = DeviceBuffer(n * H * hd * 4)
    wsb = lib.qraf_hip_attention_workspace_bytes(n, H, Hkv, hd, max_ctx)
    ws = DeviceBuffer(wsb)
    ws.zero()

    def timed(kv, K, V):
        return graph_time_us(rt, lambda i: call("qraf_hip_paged_attention_dev", q.ptr, K.ptr, V.ptr, kv, dt_.ptr,
                                                max_pages, dc.ptr, n, H, Hkv, hd, ps, np.float32(1 / math.sqrt(hd)),
                                                max_ctx, out.ptr, ws.ptr, wsb, stream.h), 50)

    def leg(kv, K, V, pos_bytes, valu=False):
        us = timed(kv, K, V)  # balanced split (the default form)
        forms = {"us_chunk_grid_form": 1}  # one workgroup per (sequence, 256-position chunk)
        if valu:
            forms["us_valu_kernel"] = 3  # the plain fp32 VALU kernel
        other = {}
        try:
            for name, f in forms.items():
                call("qraf_hip_set_attention_tuning", f)
                other[name] = round(timed(kv, K, V), 2)
        finally:
            call("qraf_hip_set_attention_tuning", rt["attn_form"])
        by = int(ctxs.sum()) * Hkv * pos_bytes * 2 + 2 * n * H * hd * 4
        return {"us": round(us, 2), "sum_ctx": int(ctxs.sum()), "alg_bytes": by,
                "GB_s": round(by / (us * 1e-6) / 1e9, 1), "frac_hbm_peak": round(by / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                **other}

    # fp16 pages, N(0,1)
    kv_half = num_pages * Hkv * ps * hd
    K, V = DeviceBuffer(kv_half * 2), DeviceBuffer(kv_half * 2)
    K.upload(rng.standard_normal(kv_half).astype(np.float16))
    V.upload(rng.standard_normal(kv_half).astype(np.float16))
    res = leg(F16, K, V, hd * 2)
    del K, V
    # int8 pages (a position of one KV head: hd bytes + a f32 scale), bytes ~ N(0, 40), scales 0.02
    blocks = np.empty((num_pages * Hkv, ps * (hd + 4)), np.uint8)
    K8, V8 = DeviceBuffer(blocks.size), DeviceBuffer(blocks.size)
    for buf in (K8, V8):
        blocks[:, :ps * hd] = np.clip(np.rint(rng.standard_normal((num_pages * Hkv, ps * hd)) * 40), -127,
                                      127).astype(np.int8).view(np.uint8)
        blocks[:, ps * hd:] = np.full((num_pages * Hkv, ps), 0.02, np.float32).view(np.uint8)
        buf.upload(blocks)
    res["int8_pages"] = leg(I8, K8, V8, hd + 4)
    del K8, V8
    # f32 pages (the reference's own KV precision), N(0,1)
    K, V = DeviceBuffer(kv_half * 4), DeviceBuffer(kv_half * 4)
    K.upload(rng.standard_normal(kv_half, dtype=np.float32))
    V.upload(rng.standard_normal(kv_half, dtype=np.float32))
    res["f32_pages"] = leg(F32, K, V, hd * 4, valu=True)
    return res


# --------------------------------------------------------------------------- decode, batch 1

SMOL = dict(vocab=49152, hidden=576, layers=30, heads=9, kv_heads=3, inter=1536, max_seq=2048, rope_theta=1e5,
            eps=1e-5)


def smol_bytes_per_token(ctx):
    """Weights + KV read per decode token of the SmolLM2-135M architecture in Q8_0."""
    D, F, L, V, kvd = 576, 1536, 30, 49152, 192
    layer = (D + 2 * kvd) * row_bytes(Q8, D) + D * row_bytes(Q8, D) + 2 * F * row_bytes(Q8, D) + D * row_bytes(Q8, F)
    return L * layer + V * row_bytes(Q8, D) + int(ctx * L * 2 * kvd * 4)


def c1_prompt():
    """The batch-1 workload's prompt: 32 tokens uniform over the vocabulary,
    numpy's default generator seeded with 1; the GPU legs and the reference's
    CPU leg decode this same prompt."""
    return np.random.default_rng(1).integers(0, SMOL["vocab"], 32).tolist()


def bench_decode_b1(args, rt):
    from qraf_amd.engine import Engine, model_config
    cfg = model_config(*(SMOL[k] for k in ("vocab", "hidden", "layers", "heads", "kv_heads", "inter", "max_seq",
                                           "rope_theta", "eps")))
    # 32 rows per step (the prompt as one batched step), KV pages for two sequences
    e = Engine(cfg, kv_dtype=F32, max_batch=32, num_pages=2 * (-(-SMOL["max_seq"] // 16)))
    e.generate_weights(Q8, Q8, Q8, False, False, 1)
    e.finalize()
    e.set_graphs(not args.no_graphs)
    if args.fusion >= 0:
        e.set_fusion(args.fusion)
    prompt = c1_prompt()
    n_gen = 128

    def run(batched_prefill=False, pipeline=True):
        s = e.seq_create()
        t0 = time.perf_counter()
        nx = None
        if batched_prefill:  # the whole prompt in one step, logits of its last row only
            _, nx = e.step([s] * len(prompt), prompt, list(range(len(prompt))),
                           want_logits=[0] * (len(prompt) - 1) + [1])
        else:  # token by token, as inference.cpp:90-99
            for i, t in enumerate(prompt):
                _, nx = e.step([s], [t], [i], want_logits=[1 if i == len(prompt) - 1 else 0])
        t1 = time.perf_counter()
        toks = [int(nx[0])]
        pos = len(prompt)
        if pipeline:
            # step k+1 issued before step k's token reaches the host: it takes that
            # token from step k's argmax on the device (no EOS stop here)
            e.step_async([s], [toks[0]], [pos])
            pos += 1
            known = 2  # tokens collected or in flight
            while known < n_gen:
                e.step_async([s], [0], [pos], token_src=[0])
                pos += 1
                known += 1
                toks.append(int(e.collect()[0]))
            toks.append(int(e.collect()[0]))
        else:  # each token read back before the next step is issued
            while len(toks) < n_gen:
                _, nx = e.step([s], [toks[-1]], [pos])
                toks.append(int(nx[0]))
                pos += 1
        t2 = time.perf_counter()
        e.seq_release(s)
        return t1 - t0, t2 - t1, toks

    # the per-launch floor: empty kernels back to back in one graph, as a step's
    # 150 layer kernels run (1 workgroup, and 256 as the decode matvecs launch)
    floor = {f"{w}_wg": round(graph_time_us(rt, lambda i, w=w: rt["call"]("qraf_hip_launch_floor_dev", w,
                                                                          rt["stream"].h), 150), 3)
             for w in (1, 256)}
    run()  # warm-up
    pre, dec, toks = run()
    _, dec_u, toks_u = run(pipeline=False)
    run(True)
    run(True)  # a step shape is captured into a graph the second time it comes
    pre_b, dec_b, toks_b = run(True)
    steps = n_gen - 1  # the first token comes from the prefill's logits
    gbs = steps * smol_bytes_per_token(len(prompt) + steps / 2) / dec / 1e9
    # the reference's defaults: InferenceEngine::generate_tokens with repetition penalty 1.1 (device sampler on the
    # step's logits) and EOS 2, prompt fed token by token
    from qraf_amd.engine import InferenceEngine, Transformer
    ie = InferenceEngine(Transformer(e), eos_token=2)
    ie.generate_tokens(prompt, n_gen, repetition_penalty=1.1)
    t0 = time.perf_counter()
    out_p = ie.generate_tokens(prompt, n_gen, repetition_penalty=1.1)
    el_p = time.perf_counter() - t0
    e.close()
    rt["c1_tokens"] = toks
    return {"model": "SmolLM2-135M architecture, Q8_0 weights, f32 KV pages, random init", "prompt": len(prompt),
            "generated": n_gen, "decode_tok_s": round(steps / dec, 1), "ms_per_token": round(dec / steps * 1e3, 3),
            "pipelined": True,
            "unpipelined": {"decode_tok_s": round(steps / dec_u, 1), "ms_per_token": round(dec_u / steps * 1e3, 3),
                            "same_tokens": toks_u == toks},
            "prefill_plus_decode_tok_s": round(n_gen / (pre + dec), 1), "prefill_ms_token_by_token": round(pre * 1e3, 2),
            "batched_prefill": {"prefill_ms": round(pre_b * 1e3, 2),
                                "prefill_plus_decode_tok_s": round(n_gen / (pre_b + dec_b), 1),
                                "same_tokens": toks_b == toks},
            "decode_GB_s": round(gbs, 1), "first_tokens": toks[:8],
            "launch_floor_us": floor, "launches_per_token": 5 * SMOL["layers"] + 3,
            "reference_defaults": {"repetition_penalty": 1.1, "eos": 2, "generated": len(out_p),
                                   "tok_s": round(len(out_p) / el_p, 1),
                                   "note": "generated / (prefill + decode) as inference.cpp:150-153; the penalty "
                                           "applied on the device from counts of the fed tokens, decode pipelined"}}


def cpu_decode_b1(gpu_tokens=None, n_tokens=128):
    """SmolLM2-135M-architecture Q8 decode with the reference's own
    InferenceEngine (oracle/_ref) on this host, the whole C1 run: the GPU
    legs' 32-token prompt fed token by token, then 128 greedy tokens (about
    15 s of one core), on the same weights (seed 1).  With the GPU leg's
    stream: whether it equals the reference's, the first position where they
    differ and the reference's own top-2 logit gap there (its forward replayed
    along its own stream)."""
    import tempfile
    from oracle import pyoracle as po
    if po.ref() is None:
        return None
    m = po.Model(po.make_config(wdtype=Q8, **SMOL), 1)
    path = os.path.join(tempfile.mkdtemp(), "smol.qraf")
    m.write_qraf(path)
    m.close()
    eng = po.RefEngine(path)
    prompt = c1_prompt()
    toks, ms = eng.generate(prompt, n_tokens, 1.0)
    eng.close()
    out = {"value": round(len(toks) / (ms / 1e3), 3),
           "unit": "tok/s, generated / (prefill + decode) as inference.cpp:150-153 reports", "cores": 1,
           "kind": "reference", "sample": f"{len(prompt)}-token prompt + {len(toks)} greedy tokens via "
                                          f"InferenceEngine::generate_tokens, {ms / 1e3:.1f} s, host CPU {host_cpu()}"}
    if gpu_tokens is not None:
        same = list(gpu_tokens) == list(toks)
        cmp = {"same_tokens_as_reference": same, "tokens_compared": len(toks),
               "same_first_32": list(gpu_tokens[:32]) == list(toks[:32])}
        if not same:
            d = next((i for i in range(min(len(toks), len(gpu_tokens))) if toks[i] != gpu_tokens[i]),
                     min(len(toks), len(gpu_tokens)))
            rm = po.RefModel(path, SMOL["vocab"])
            lg = None
            for i, t in enumerate(prompt + toks[:d]):
                lg = rm.forward(t, i)
            rm.close()
            s2 = np.sort(lg)
            cmp.update({"first_divergence": d, "reference_top2_gap_there": float(s2[-1] - s2[-2]),
                        "reference_top_logit_there": float(s2[-1])})
        out["stream_check"] = cmp
    os.remove(path)
    return out


# --------------------------------------------------------------------------- decode, batch 128

def cpu_decode_qwen(rt, n_prompt=4, n_gen=4):
    """The Qwen2.5-3B-architecture Q4 decode on the host with the reference's
    own QrafModel + Transformer (oracle/_ref), one core, on the same weights
    (written to a .qraf file from the device generator): one sequence, an
    n_prompt-token prompt fed token by token, then n_gen greedy tokens.  The
    reference decodes sequences one at a time (its scheduler calls forward
    per request), so its aggregate rate over 128 sequences is this rate."""
    import tempfile
    from oracle import pyoracle as po
    if po.ref() is None:
        return None
    tmp = tempfile.mkdtemp()
    path = os.path.join(tmp, "qwen3b_q4.qraf")
    try:
        write_qraf_synthetic(path, QWEN, Q4, 3, rt)
        ref = po.RefModel(path, QWEN["vocab"])
        try:
            toks = np.random.default_rng(9).integers(0, QWEN["vocab"], n_prompt).tolist()
            t0 = time.perf_counter()
            for pos in range(n_prompt + n_gen - 1):
                lg = ref.forward(toks[pos], pos)
                if pos >= n_prompt - 1:
                    toks.append(int(np.argmax(lg)))
            el = time.perf_counter() - t0
        finally:
            ref.close()
    finally:
        if os.path.exists(path):
            os.remove(path)
        os.rmdir(tmp)
    fwd = n_prompt + n_gen - 1
    return {"value": round(fwd / el, 4), "unit": "tok/s (forward passes per second, one sequence)", "cores": 1,
            "kind": "reference", "s_per_token": round(el / fwd, 3),
            "sample": f"Transformer::forward of the Qwen2.5-3B architecture (Q4_0, tied f32 head as the reference "
                      f"builds it): {n_prompt}-token prompt + {n_gen} greedy tokens, {fwd} forwards in {el:.1f} s, "
                      f"host CPU {host_cpu()}"}


QWEN = dict(vocab=151936, hidden=2048, layers=36, heads=16, kv_heads=2, inter=11008, max_seq=1024, rope_theta=1e6,
            eps=1e-6)


KV_NAMES = {F32: "f32", F16: "fp16", I8: "int8"}
KV_POS_BYTES = {F32: 2 * 36 * 2 * 128 * 4, F16: 2 * 36 * 2 * 128 * 2, I8: 2 * 36 * 2 * (128 + 4)}  # K+V, all layers


def qwen_engine(args, rows, kv=F32):
    """The Qwen2.5-3B-architecture engine of the batch-128 legs (random Q4_0
    weights; f32 KV pages by default, the reference's KVCache)."""
    from qraf_amd.engine import Engine, model_config
    cfg = model_config(*(QWEN[k] for k in ("vocab", "hidden", "layers", "heads", "kv_heads", "inter", "max_seq",
                                           "rope_theta", "eps")))
    pages = 128 * (-(-QWEN["max_seq"] // 16)) + 64
    e = Engine(cfg, kv_dtype=kv, max_batch=rows, num_pages=pages)
    e.generate_weights(Q4, Q4, Q4, True, True, 3)
    e.finalize()
    e.set_graphs(not args.no_graphs)
    e.set_row_padding(args.row_padding)
    return e


def bench_decode_b128(args, rt):
    """C5: 128 concurrent requests, continuous batching.  The headline run
    feeds prompts in chunks (up to --prefill-chunk tokens of one request per
    step, within a --rows row budget, decode rows first); the token-by-token
    run (every active request one row per step) is reported beside it."""
    from qraf_amd.engine import BatchScheduler
    rows = max(128, args.rows)
    e = qwen_engine(args, rows)
    rng = np.random.default_rng(3)
    warm = BatchScheduler(e, max_batch=128, max_rows=rows, prefill_chunk=args.prefill_chunk)
    for _ in range(8):
        warm.submit(rng.integers(0, QWEN["vocab"], 300).tolist(), 4)
    warm.run()
    work = []
    for _ in range(args.requests):
        plen, olen = int(rng.integers(16, 513)), int(rng.integers(64, 257))
        work.append((rng.integers(0, QWEN["vocab"], plen).tolist(), olen))

    pipe = not args.no_pipeline

    keep = args.keep_logits

    def run(max_rows, chunk, pipeline=pipe, keep_logits=keep):
        return run_schedule(e, work, max_rows, chunk, pipeline, keep_logits)

    e.stats(reset=True)
    chunked, streams_c = run(rows, args.prefill_chunk)
    unpiped, streams_u = run(rows, args.prefill_chunk, False)
    tbt, streams_t = run(128, 1)
    other, streams_o = run(rows, args.prefill_chunk, pipe, not keep)  # the other head form, same schedule
    other["streams_equal"] = streams_o == streams_c
    steady = steady_decode_b128(e, np.random.default_rng(3), args.decode_steps, F32, pipe, keep)
    e.close()
    extras = {}
    for kv in (F16, I8):  # narrower pages: not the reference's values; agreement with the f32 streams beside them
        ek = qwen_engine(args, rows, kv)
        res, streams_k = run_schedule(ek, work, rows, args.prefill_chunk, pipe, keep)
        res["stream_agreement_with_f32_pages"] = stream_agreement(streams_c, streams_k)
        res["steady_decode"] = steady_decode_b128(ek, np.random.default_rng(3), args.decode_steps, kv, pipe, keep)
        ek.close()
        extras[f"{KV_NAMES[kv]}_pages"] = res
    out = {"model": "Qwen2.5-3B architecture, Q4_0 weights, tied head, QKV bias, f32 KV pages, random init",
           "requests": args.requests, "max_concurrent": 128}
    out.update(chunked)
    unpiped["streams_equal_pipelined"] = streams_u == streams_c
    out.update({"row_budget": rows, "prefill_chunk": args.prefill_chunk, "pipelined": pipe,
                "note": "continuous batching, requests admitted as others finish; each step feeds every decoding "
                        "request's last token, then prompt chunks within the row budget; f32 KV pages hold the "
                        "reference's KVCache values; pipelined: step N+1 is issued before step N's tokens reach "
                        "the host, its decode rows taking them from step N's argmax on the device",
                "unpipelined": unpiped, ("logits_kept" if not keep else "greedy_only_head"): other,
                "token_by_token": tbt, "stream_agreement": stream_agreement(streams_c, streams_t),
                "steady_decode": steady})
    out.update(extras)
    return out


def run_schedule(e, work, max_rows, chunk, pipeline=False, keep_logits=False):
    """One continuous-batching run of `work` [(prompt, max tokens)] through 128
    slots; aggregate generated tok/s, and the host's share of the wall time:
    the scheduler's own Python work plus the engine's host-side preparation of
    each step (unpipelined, the device idles meanwhile, as every step ends in a
    synchronisation; pipelined, that work overlaps the previous step's run and
    device_wait_ms_per_step is the time the host waited for the device).
    keep_logits False: the greedy requests keep no logits (the engine's
    greedy-only head, its argmax in the head GEMM's epilogue)."""
    from qraf_amd.engine import BatchScheduler
    sched = BatchScheduler(e, max_batch=128, max_rows=max_rows, prefill_chunk=chunk, pipeline=pipeline,
                           keep_logits=keep_logits)
    for p, o in work:
        sched.submit(p, o)
    e.stats(reset=True)
    t0 = time.perf_counter()
    done = sched.run()
    el = time.perf_counter() - t0
    st = e.stats(reset=True)
    gen = sum(len(r.generated) for r in done)
    host_ms = (sched.host_s * 1e3 + st["host_us"] * 1e-3) / sched.steps
    return {"generated_tokens": gen, "steps": sched.steps, "rows_processed": sched.rows, "wall_s": round(el, 3),
            "generated_tok_s": round(gen / el, 1), "rows_per_s": round(sched.rows / el, 1),
            "ms_per_step": round(el / sched.steps * 1e3, 3),
            "host_ms_per_step": round(host_ms, 3), "host_share": round(host_ms / (el / sched.steps * 1e3), 4),
            "scheduler_python_ms_per_step": round(sched.host_s * 1e3 / sched.steps, 3),
            "engine_host_prep_ms_per_step": round(st["host_us"] * 1e-3 / sched.steps, 3),
            "device_wait_ms_per_step": round(st["wait_us"] * 1e-3 / sched.steps, 3),
            "step_launches": {"eager": st["eager_steps"], "graph_captures": st["graph_captures"],
                              "graph_launches": st["graph_launches"]},
            "pad_rows": st["pad_rows"], "logits_kept": keep_logits}, \
        [r.generated for r in sorted(done, key=lambda r: r.id)]


def fnv1a(name: str) -> int:
    h = 14695981039346656037
    for ch in name.encode():
        h = ((h ^ ch) * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return h


def write_qraf_synthetic(path, q, wdt, seed, rt):
    """A .qraf file (include/qraf/format.h:26-132 layout) holding exactly the
    weights Engine.generate_weights(wdt, wdt, wdt, tied=True, qkv_bias=True,
    seed) makes on the device: each tensor from qraf_hip_gen_weights_dev with
    stream = FNV-1a(name), norms 1, f32 q/k/v biases, no lm_head (tied).
    Returns the file size."""
    import struct
    call, DeviceBuffer, stream = rt["call"], rt["DeviceBuffer"], rt["stream"]
    D, F, V, nl, H, Hkv = q["hidden"], q["inter"], q["vocab"], q["layers"], q["heads"], q["kv_heads"]
    hd = D // H
    qd, kvd = H * hd, Hkv * hd
    ts = [("model.embed_tokens.weight", wdt, (V, D))]
    for layer in range(nl):
        p = f"model.layers.{layer}."
        ts += [(p + "self_attn.q_proj.weight", wdt, (qd, D)), (p + "self_attn.k_proj.weight", wdt, (kvd, D)),
               (p + "self_attn.v_proj.weight", wdt, (kvd, D)), (p + "self_attn.o_proj.weight", wdt, (D, qd)),
               (p + "self_attn.q_proj.bias", F32, (qd,)), (p + "self_attn.k_proj.bias", F32, (kvd,)),
               (p + "self_attn.v_proj.bias", F32, (kvd,)), (p + "mlp.gate_proj.weight", wdt, (F, D)),
               (p + "mlp.up_proj.weight", wdt, (F, D)), (p + "mlp.down_proj.weight", wdt, (D, F)),
               (p + "input_layernorm.weight", F32, (D,)), (p + "post_attention_layernorm.weight", F32, (D,))]
    ts.append(("model.norm.weight", F32, (D,)))
    nbytes = lambda dt, sh: sh[0] * row_bytes(dt, sh[1]) if len(sh) == 2 else 4 * sh[0]
    cfg = [("architecture", 2, "qwen2")] + [(k, 0, q[n]) for k, n in (
        ("vocab_size", "vocab"), ("hidden_size", "hidden"), ("num_layers", "layers"), ("num_heads", "heads"),
        ("num_kv_heads", "kv_heads"), ("intermediate_size", "inter"), ("max_seq_len", "max_seq"))] + [
        ("rope_theta", 1, q["rope_theta"]), ("rms_norm_eps", 1, q["eps"])]
    strtab, soff = bytearray(), {}

    def sref(x):
        if x not in soff:
            soff[x] = len(strtab)
            strtab.extend(x.encode() + b"\0")
        return soff[x]
    for k, ty, v in cfg:
        sref(k)
        if ty == 2:
            sref(v)
    for n, _, _ in ts:
        sref(n)
    cfg_off = 128
    cfg_blk = struct.pack("<I", len(cfg)) + b"".join(
        struct.pack("<III", sref(k), ty, sref(v) if ty == 2 else
                    (struct.unpack("<I", struct.pack("<f", v))[0] if ty == 1 else v)) for k, ty, v in cfg)
    dir_off = cfg_off + len(cfg_blk)
    qdir_off = dir_off + 80 * len(ts)
    str_off = qdir_off + 32
    off = (str_off + len(strtab) + 63) // 64 * 64
    data_off, offs = off, []
    for n, dt, sh in ts:
        offs.append(off)
        off = (off + nbytes(dt, sh) + 63) // 64 * 64
    size = off
    tdir = b"".join(struct.pack("<QII8IIIQQII", fnv1a(n), sref(n), len(sh), *(list(sh) + [0] * (8 - len(sh))), dt,
                                0 if dt in (Q8, Q4) else 0xFFFFFFFF, o, nbytes(dt, sh), 0, 0)
                    for (n, dt, sh), o in zip(ts, offs))
    qdir = struct.pack("<IIIIffII", 0, wdt, 32, 1, 0.0, 0.0, 1, 0)
    hdr = struct.pack("<IIQ" + "Q" * 11 + "IIII8s", 0x46415251, 1, size, cfg_off, len(cfg_blk), 0, 0, dir_off,
                      len(tdir), qdir_off, len(qdir), str_off, len(strtab), data_off, len(ts), 1, 0, 0, b"\0" * 8)
    big = max(nbytes(dt, sh) for _, dt, sh in ts)
    buf = DeviceBuffer(big)
    with open(path, "wb") as f:
        f.write(hdr + cfg_blk + tdir + qdir + bytes(strtab))
        for (n, dt, sh), o in zip(ts, offs):
            cnt = sh[0] * (sh[1] if len(sh) == 2 else 1)
            if n.endswith("layernorm.weight") or n == "model.norm.weight":
                data = np.ones(cnt, np.float32).tobytes()
            else:
                call("qraf_hip_gen_weights_dev", buf.ptr, dt, cnt, seed, fnv1a(n), 0.02, stream.h)
                stream.synchronize()  # the download is not ordered after work on this stream
                data = buf.download(np.uint8, nbytes(dt, sh)).tobytes()
            f.write(b"\0" * (o - f.tell()))
            f.write(data)
        f.write(b"\0" * (size - f.tell()))
    buf.free()
    return size


def bench_load(args, rt):
    """QRAF file -> HBM for the Qwen2.5-3B architecture in Q4_0 (tied head,
    QKV bias): qraf_engine_create_from_file on a file this leg writes (warm
    page cache), then one forward checked bit for bit against an engine whose
    weights were generated on the device with the same seed."""
    import tempfile
    from qraf_amd.engine import Engine, Transformer, model_config
    tmp = tempfile.mkdtemp()
    path = os.path.join(tmp, "qwen3b_q4.qraf")
    try:
        t0 = time.perf_counter()
        size = write_qraf_synthetic(path, QWEN, Q4, 3, rt)
        t_write = time.perf_counter() - t0
        loads = []
        for _ in range(2):
            t0 = time.perf_counter()
            e = Engine.from_file(path, kv_dtype=F16, max_batch=1)
            rt["call"]("qraf_hip_device_synchronize")
            loads.append(time.perf_counter() - t0)
            if len(loads) < 2:
                e.close()
        tf = Transformer(e)
        cfg = model_config(*(QWEN[k] for k in ("vocab", "hidden", "layers", "heads", "kv_heads", "inter", "max_seq",
                                               "rope_theta", "eps")))
        g = Engine(cfg, kv_dtype=F16, max_batch=1)
        g.generate_weights(Q4, Q4, Q4, True, True, 3)
        g.finalize()
        same = bool(np.array_equal(tf.forward(17, 0), Transformer(g).forward(17, 0)))
        e.close()
        g.close()
    finally:
        if os.path.exists(path):
            os.remove(path)
        os.rmdir(tmp)
    best = min(loads)
    return {"model": "Qwen2.5-3B architecture, Q4_0, tied head, QKV bias", "file_bytes": size,
            "load_s": round(best, 3), "load_GB_s": round(size / best / 1e9, 2), "write_s": round(t_write, 2),
            "logits_equal_device_generated": same,
            "note": "qraf_engine_create_from_file: validate + map + copy every tensor to HBM + finalize (tile-major "
                    "repack on the device), file in the page cache; best of 2"}


def bench_sampler(args, rt):
    """The device sampler (qraf_hip_sample_dev) on 128 rows of Qwen2.5-3B-
    vocabulary logits with SamplingConfig's defaults (temperature 0.8, top-k
    40, top-p 0.9, repetition penalty 1.1 over 512 recent tokens per row),
    captured 20 calls to a graph."""
    import ctypes as C
    from qraf_amd._lib import SamplingParams
    call, DeviceBuffer = rt["call"], rt["DeviceBuffer"]
    rows, V, nrec = 128, QWEN["vocab"], 512
    rng = np.random.default_rng(5)
    dl = DeviceBuffer.from_array((rng.standard_normal((rows, V)) * 3).astype(np.float32))
    rec = DeviceBuffer.from_array(rng.integers(0, V, (rows, nrec)).astype(np.uint32))
    cnt = DeviceBuffer.from_array(np.full(rows, nrec, np.int32))
    uni = DeviceBuffer.from_array(rng.random(rows).astype(np.float32))
    out = DeviceBuffer(rows * 4)
    sp = SamplingParams(0.8, 40, 0.9, 1.1)
    us = graph_time_us(rt, lambda i: call("qraf_hip_sample_dev", dl.ptr, rows, V, C.byref(sp), rec.ptr, cnt.ptr, nrec,
                                          uni.ptr, out.ptr, rt["stream"].h), 20)
    sp1 = SamplingParams(0.8, 40, 0.9, 1.0)
    us_nopen = graph_time_us(rt, lambda i: call("qraf_hip_sample_dev", dl.ptr, rows, V, C.byref(sp1), None, None, 0,
                                                uni.ptr, out.ptr, rt["stream"].h), 20)
    for d in (dl, rec, cnt, uni, out):
        d.free()
    return {"rows": rows, "vocab": V, "recent_tokens": nrec, "config": "T 0.8, top_k 40, top_p 0.9, penalty 1.1",
            "us_per_call": round(us, 1), "us_per_call_without_penalty": round(us_nopen, 1),
            "logits_kept_in_hbm_MB": round(rows * V * 4 / 1e6, 1)}


def cpu_sampler():
    """The reference's Sampler::sample (std::sort over the vocabulary) on one
    row of the same shape, on the host: ms per draw."""
    import ctypes as C
    from oracle import pyoracle as po
    R = po.ref()
    if R is None:
        return None
    V = QWEN["vocab"]
    l = (np.random.default_rng(5).standard_normal(V) * 3).astype(np.float32)
    out = np.zeros(8, np.uint32)
    t0 = time.perf_counter()
    R.ref_sample(l.ctypes.data_as(C.POINTER(C.c_float)), V, 0.8, 40, 0.9, 7, 8,
                 out.ctypes.data_as(C.POINTER(C.c_uint32)))
    ms = (time.perf_counter() - t0) * 1e3 / 8
    return {"value": round(ms, 2), "unit": "ms per sampled token (one row)", "cores": 1, "kind": "reference",
            "sample": f"Sampler::sample on one {V}-logit row, 8 draws, host CPU {host_cpu()}"}


def bench_steady_b128(args, rt):
    """The steady 128-sequence decode alone (every GEMM at 128 rows), for profiling."""
    kv = {"f32": F32, "fp16": F16, "int8": I8}[args.kv]
    e = qwen_engine(args, 128, kv)
    out = steady_decode_b128(e, np.random.default_rng(3), args.decode_steps, kv, not args.no_pipeline,
                             args.keep_logits)
    e.close()
    return out


def stream_agreement(a, b):
    """How far two runs' greedy streams of the same requests agree.  Batch
    composition changes the GEMM's tiling and split, so fp32 rounding differs
    within the parity tolerance; random-init logits have near-ties, where a
    different rounding may pick the other token, after which a stream differs."""
    first = [next((i for i, (x, y) in enumerate(zip(s, t)) if x != y), min(len(s), len(t))) for s, t in zip(a, b)]
    return {"requests": len(first), "identical": sum(1 for s, t in zip(a, b) if s == t),
            "first_32_identical": sum(1 for f, s in zip(first, a) if f >= min(32, len(s))),
            "median_first_difference": int(np.median(first))}


QWEN_LAYER_WEIGHT_BYTES = 1560674304  # 36 layers of Q4_0 q/k/v/o/gate/up/down
QWEN_HEAD_BYTES = 175030272           # the tied Q4_0 embedding read as the head


def steady_decode_b128(e, rng, steps, kv, pipeline=False, keep_logits=False):
    """128 concurrent sequences at ragged contexts (prompt U[16,512] plus U[0,255] generated, the run above's
    distribution), prefilled in 128-row steps; then `steps` decode steps of 128 rows, every row generating
    (greedy, device argmax).  Timed: the decode steps only.  Pipelined: each step is issued before the previous
    one's tokens are collected, its rows taking them from the previous step's argmax on the device.
    keep_logits False: the decode steps keep no logits (the greedy-only head)."""
    n, V = 128, QWEN["vocab"]
    seqs = [e.seq_create() for _ in range(n)]
    ctx = rng.integers(16, 513, n) + rng.integers(0, 256, n)
    rows = [(s, p) for s, c in zip(seqs, ctx) for p in range(int(c))]
    for i in range(0, len(rows), 128):
        ch = rows[i:i + 128]
        e.step([s for s, _ in ch], rng.integers(0, V, len(ch)).tolist(), [p for _, p in ch],
               want_logits=np.zeros(len(ch), np.uint8), logits=False, argmax=False)
    toks = rng.integers(0, V, n).tolist()
    pos = ctx.astype(np.int64).copy()
    e.set_keep_logits(keep_logits)
    for _ in range(3):  # warm-up decode steps
        _, nx = e.step(seqs, toks, pos.tolist())
        toks, pos = nx.tolist(), pos + 1
    t0 = time.perf_counter()
    if pipeline:
        src = np.arange(n, dtype=np.int32)
        e.step_async(seqs, toks, pos.tolist())
        pos = pos + 1
        for _ in range(steps - 1):
            e.step_async(seqs, toks, pos.tolist(), token_src=src)
            pos = pos + 1
            e.collect()
        nx = e.collect()
    else:
        for _ in range(steps):
            _, nx = e.step(seqs, toks, pos.tolist())
            toks, pos = nx.tolist(), pos + 1
    el = time.perf_counter() - t0
    e.set_keep_logits(True)
    for s in seqs:
        e.seq_release(s)
    # HBM bytes per step: every layer weight, the head, and every cached K/V position read once
    mean_ctx = float(ctx.mean()) + 3 + (steps + 1) / 2
    by = QWEN_LAYER_WEIGHT_BYTES + QWEN_HEAD_BYTES + KV_POS_BYTES[kv] * mean_ctx * n
    ms = el / steps * 1e3
    return {"kv_pages": KV_NAMES[kv], "sequences": n, "context_mean_at_start": round(float(ctx.mean()) + 3, 1),
            "context_max_at_end": int(pos.max()), "decode_steps": steps, "ms_per_step": round(ms, 3),
            "decode_tok_s": round(n * steps / el, 1), "pipelined": pipeline, "logits_kept": keep_logits,
            "alg_bytes_per_step": int(by),
            "GB_s": round(by / (ms * 1e-3) / 1e9, 1), "frac_hbm_peak": round(by / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


# --------------------------------------------------------------------------- main

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="matvec,gemm,attention,decode_b1,decode_b128,load,sampler")
    ap.add_argument("--requests", type=int, default=256, help="requests in the batch-128 decode run")
    ap.add_argument("--decode-steps", type=int, default=64, help="timed steps of the steady 128-sequence decode")
    ap.add_argument("--rows", type=int, default=512, help="row budget per step of the continuous-batch run")
    ap.add_argument("--prefill-chunk", type=int, default=512, help="prompt tokens of one request per step at most")
    ap.add_argument("--keep-logits", action="store_true",
                    help="batch-128 legs: greedy steps keep their logits in HBM (default: the greedy-only head, "
                         "argmax in the head GEMM's epilogue; the other form is reported beside it)")
    ap.add_argument("--cases", default="",
                    help="restrict the matvec leg to these cases, e.g. 'q8_0 11008x4096' (comma-separated; "
                         "a profile of one case then has one shape per kernel)")
    ap.add_argument("--gemm-cases", default="",
                    help="restrict the GEMM leg to these cases, e.g. 'q4_0 11008x2048 B=128' (comma-separated)")
    ap.add_argument("--no-graphs", action="store_true",
                    help="launch every kernel eagerly (timed with events) instead of replaying captured graphs, "
                         "in every leg")
    ap.add_argument("--no-pipeline", action="store_true",
                    help="batch-128 legs: wait for every step's tokens before issuing the next")
    ap.add_argument("--kv", default="f32", choices=["f32", "fp16", "int8"], help="KV pages of the steady_b128 leg")
    ap.add_argument("--rows-per-wave", type=int, default=0)
    ap.add_argument("--kernel", type=int, default=0,
                    help="matvec kernel: 0 auto, 1 one-shot, 2 persistent, 3 ring (8-wave groups), 4 ring (4-wave groups)")
    ap.add_argument("--wgs-per-cu", type=int, default=0)
    ap.add_argument("--row-padding", type=int, default=16,
                    help="batched engine steps of more than 8 rows run padded to a multiple of this (1: off)")
    ap.add_argument("--gemm-form", default="auto", choices=["auto", "pipelined", "wave_split", "row_split"],
                    help="tiled batched-GEMM form for every leg (auto: the library's per-shape choice)")
    ap.add_argument("--fusion", type=int, default=-1,
                    help="engine fusion flags of the batch-1 decode leg (qraf_engine_set_fusion; -1: the defaults)")
    ap.add_argument("--attn-form", type=int, default=0,
                    help="attention work form for every leg: 0 auto, 1 chunk grid, 2 balanced split, 3 VALU kernel")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not supported "
              "(the decode path would shard by sequence across GPUs)", file=sys.stderr)
        sys.exit(2)
    only = set(args.only.split(","))

    import qraf_amd
    from qraf_amd._lib import call
    from qraf_amd.backend import DeviceBuffer, Event, Graph, Stream

    qraf_amd.backend.backend_init(0)
    call("qraf_hip_set_matvec_tuning", args.kernel, args.rows_per_wave, args.wgs_per_cu)
    call("qraf_hip_set_attention_tuning", args.attn_form)
    if args.gemm_form == "pipelined":  # the LDS-ring kernels everywhere over 32 rows
        call("qraf_hip_set_qgemm_kw", -1, 0)
    elif args.gemm_form == "wave_split":
        call("qraf_hip_set_qgemm_kw", 1, 0)
    elif args.gemm_form == "row_split":
        call("qraf_hip_set_qgemm_tuning", 0, 0, 3, 0)
    rt = dict(call=call, DeviceBuffer=DeviceBuffer, Event=Event, Graph=Graph, stream=Stream(), lib=qraf_amd.lib,
              eager=args.no_graphs, attn_form=args.attn_form)

    value, total_ms, per_case, cache_res, hosts = bench_matvec(args, rt)
    print(f"# matvec done: {value:.1f} GB/s", file=sys.stderr, flush=True)
    extra = {}
    for part, fn in (("gemm", bench_gemm), ("gemm_library", bench_gemm_library), ("attention", bench_attention),
                     ("decode_b1", bench_decode_b1),
                     ("decode_b128", bench_decode_b128), ("steady_b128", bench_steady_b128), ("load", bench_load),
                     ("sampler", bench_sampler)):
        if part in only:
            extra[part] = fn(args, rt)
            print(f"# {part} done", file=sys.stderr, flush=True)

    dom = max(per_case, key=lambda p: p["us_per_launch"])  # dominant kernel: longest launch
    kname = ring_kernel_name(dom["case"])
    traffic = MEASURED_TRAFFIC.get((kname, dom["case"]))
    roofline = {"bound": "hbm", "achieved": dom["GB_s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(dom["GB_s"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                "traffic_source": "profiles/qmv_matvec_isolated.md (FETCH_SIZE, WRITE_SIZE scaled by a copy kernel)"
                if traffic else None,
                "kernel": kname,
                "case": dom["case"], "alg_bytes_per_launch": dom["alg_bytes"],
                "plain_read_GB_s": dom.get("plain_read_GB_s"), "frac_of_plain_read": dom.get("frac_of_plain_read"),
                # every case of the step in brief: [case, us per launch, GB/s, fraction of HBM peak,
                # fraction of the same-size plain read]
                "per_case": [[p["case"], p["us_per_launch"], p["GB_s"], p["frac_hbm_peak"], p.get("frac_of_plain_read")]
                             for p in per_case]}
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline_matvec(hosts, args.cpu_seconds)
        if "decode_b1" in only:
            extra["cpu_decode_b1"] = cpu_decode_b1(rt.get("c1_tokens"))
            chk = (extra["cpu_decode_b1"] or {}).get("stream_check")
            if chk and "decode_b1" in extra:
                extra["decode_b1"]["same_tokens_as_reference"] = chk["same_tokens_as_reference"]
        if "sampler" in only:
            extra["cpu_sampler"] = cpu_sampler()
        if "decode_b128" in only:
            extra["cpu_decode_b128"] = cpu_decode_qwen(rt)
        print("# cpu baseline done", file=sys.stderr, flush=True)

    out = {"metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(total_ms / args.steps, 5), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
           "config": {"workload": "isolated quantized matvec, batch 1: fp32 x[4096] times Q8_0 and Q4_0 weights "
                                  "4096x4096 and 11008x4096 (N(0,0.02), repo quantizer), one launch per case per "
                                  "step, weights rotating through >320 MB pools per case",
                      "cases": [p["case"] for p in per_case]},
           "per_case": per_case, "cache_resident": cache_res, "roofline": roofline, "cpu_baseline": cpu}
    out.update(extra)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    if "--gemm-library-child" in sys.argv:  # the gemm_library leg's measuring process (torch only)
        gemm_library_child()
    else:
        main()
