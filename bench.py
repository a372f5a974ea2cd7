#!/usr/bin/env python3
"""Benchmark of the shipped gfx950 GEMM path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-decode]

One step is one launch of the shipped gemm_fp16 (kernels/shipped/gemm_fp16/gfx950, reached
through the C-ABI libtempo_gfx950.so) over configuration C1: C[4096,15360] = A[4096,3840] .
B[15360,3840]^T, fp16 inputs N(0,1)/sqrt(K) from PCG64 seeds 11 / 77, fp32 accumulation, fp16
output; inputs are resident in HBM before the timed region.  `value` is that kernel's TFLOP/s
(2MNK flops per step).  Before timing, the output passes a correctness gate (no 0x7f7f poison
left, fp64 dot products on 256 sampled cells within |got-ref|/(|ref|+1e-3) <= 3e-3, the rule of
the reference's kernels/shipped/gemm_fp16/sm_70/ship_probe.cu:70-79).

Extra fields of the one JSON line:
  roofline      the C1 kernel against the fp16 dense MFMA peak; `achieved` from HIP events on
                the launch stream; `traffic` (HBM bytes per launch) from the committed rocprofv3
                --pmc summary profiles/counters_gemm_fp16_configs.md (its C1 "bytes" line) when
                present, else null.
  settle        clock settling before warm-up: back-to-back C1 launches in timed batches of 20
                until two batches agree within 2 % (the engine clock ramps over the first few
                hundred ms of load); `warmup` and `steps` keep their meaning after it.
  cpu_baseline  the CPU restatement of the reference's naive kernel (oracle/, fp32 sequential-k
                FMA per output, OpenMP) timed on this host over a bounded row sample of C1, with
                the host's CPU model and a numpy fp32 BLAS arm over a row sample as a library bar.
  decode        HBM GB/s of the decode regime (M <= 32): gemm_w8a16 on both weight formats and
                gemm_fp16 on the two C2 shapes, weights rotated through > 512 MiB so no launch
                finds its weights in the 256 MiB Infinity Cache.  These launches (and the
                gate/up ones) go straight to the C entry points on parameter blocks built once
                per weight copy: a Python wrapper's checks per call take longer than a 20-40 us
                kernel and would time the host instead.
  fmha          the causal FMHA forward at configuration C5, TFLOP/s.
  card          the card passport before and after the run (tempo/plugins/gfx950/card.py):
                engine and memory clocks, socket power, temperature, clock lock, and the
                processes seen on the card other than this one (the reference's
                kernels/shipped/gemm_fp16/sm_70/manifest.json:107-113).
  roofline.sclk_mhz / peak_at_sclk / frac_at_sclk
                the engine clock the C1 kernel runs at -- GRBM_GUI_ACTIVE per dispatch over its
                duration, from the committed counter summary (the clock follows the matrix
                cores' load within microseconds, so only a counter read during the dispatch
                gives it) -- and the matrix-core peak at that clock (256 CUs x 4096 flop/clk x
                sclk), the reference's peak_tflops_1530 at its locked clock (manifest.json:119).
  roofline.sclk_live_mhz / peak_at_sclk_live / frac_at_sclk_live
                the same clock read on this box during the run: amd-smi's gfx clocks sampled
                while C1 runs back to back after the timed steps (a short-window average, so the
                load lasts across the reads), the median of the reads.
  decode[].hbm_frac_measured
                GB/s against the MEASURED pure-read HBM rate of the plugin's rate table
                (HBM.READ_PURE, taken by tempo.plugins.gfx950.calibrate on a clean card), next
                to hbm_frac against the 8 TB/s spec.
  cpu_baseline.w8a16_arm
                the W8A16 CPU path: the oracle's dequantisation followed by its fp32 GEMM, on a
                row sample of the (34816, 5120) decode shape, both weight formats.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

METRIC = ("GEMM TFLOP/s & % fp16 MFMA peak (prefill); HBM GB/s & % peak (decode M≤32)")
PEAK_FP16_TFLOPS = 2516.6   # 256 CUs x 2.4 GHz x 4096 flop/clk (AMD dense fp16 figure)
PEAK_HBM_GBPS = 8000.0      # MI355X HBM3E
TRAFFIC_FILE = os.path.join(HERE, "profiles", "counters_gemm_fp16_configs.md")

C1 = dict(M=4096, N=15360, K=3840)
# Each decode and gate/up line first runs its own launches for at least this long: the engine
# clock and power state take a few hundred ms of steady load to settle (measured on the M = 1
# W8A16 line at (34816, 5120): 31.5 us per launch after ~150 launches, 29.7 us after 0.3 s)
DECODE_SETTLE_S = 0.3
SEED_A, SEED_B = 11, 77


def randn_f16(shape, seed, scale):
    g = np.random.Generator(np.random.PCG64(seed))
    return (g.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float16)


def to_dev(x):
    import torch

    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0")


def time_launches(fn, steps, warmup, stream):
    """Average ms per launch of fn(i) on `stream`, HIP events recorded on that same stream."""
    import torch

    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(steps):
        fn(i)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def direct(entry, params, stream):
    """fn(i) launching the C entry point `entry` on prebuilt parameter blocks params[i % len]:
    a launch then costs the C-ABI call alone (a few microseconds), so a timed loop of kernels of
    ~20-40 us is not bound by the host.  The operands were checked once, when the blocks were
    built (capi's wrappers)."""
    from cuda_tempiler_amd import capi

    sp = capi._stream(stream)
    n = len(params)

    def fn(i):
        rc = entry(params[i % n], sp)
        if rc != 0:
            raise capi.TempoError(rc, entry.__name__)
    return fn


def gate_c1(A, B, C):
    """fp64 spot check of 256 sampled cells plus the poison count (numpy, independent of the
    kernel and of the CPU oracle)."""
    M, K = A.shape
    N = B.shape[0]
    Ch = C.view(np.uint16)
    poison = int(np.count_nonzero(Ch == 0x7f7f))
    t = np.arange(256)
    m, n = (t * 37) % M, (t * 53) % N
    ref = np.einsum("ik,ik->i", A[m].astype(np.float64), B[n].astype(np.float64))
    got = C[m, n].astype(np.float64)
    rel = np.abs(got - ref) / (np.abs(ref) + 1e-3)
    return {"poison": poison, "spot_cells": 256, "spot_max": float(rel.max()),
            "ok": bool(poison == 0 and rel.max() <= 3e-3)}


def read_traffic():
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, or None."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    with open(TRAFFIC_FILE, encoding="utf-8") as f:
        for line in f:  # "bytes M,N,K,fmt: fetch F write W traffic T algorithmic A"
            w = line.split()
            if w[:2] == ["bytes", "%d,%d,%d,0:" % (C1["M"], C1["N"], C1["K"])]:
                return int(w[w.index("traffic") + 1])
    return None


def settle_clocks(fn, stream, batch=20, tol=0.02, max_s=3.0, min_s=0.0):
    """Back-to-back launches in timed batches until two consecutive batches agree within `tol`
    (or `max_s` of launching), and at least `min_s` of launching has passed: the engine clock on
    this part ramps over the first few hundred milliseconds of sustained matrix-core load, and
    the timed region must not include the ramp (a slow ramp can look settled to two short
    batches).  Returns what it did (reported next to `warmup`, which keeps its meaning)."""
    import torch

    hist, t0, i = [], time.perf_counter(), 0
    while True:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(batch):
            fn(i)
            i += 1
        e1.record(stream)
        e1.synchronize()
        hist.append(e0.elapsed_time(e1) / batch)
        if (len(hist) >= 2 and abs(hist[-1] - hist[-2]) <= tol * hist[-1]
                and time.perf_counter() - t0 >= min_s):
            break
        if time.perf_counter() - t0 > max_s:
            break
    shown = hist if len(hist) <= 10 else hist[:5] + hist[-5:]  # the ramp and where it ended
    return {"launches": i, "batches": len(hist),
            "batches_ms_per_launch": [round(x, 4) for x in shown],
            "settled": len(hist) >= 2 and abs(hist[-1] - hist[-2]) <= tol * hist[-1]}


def cpu_model():
    """The host CPU as /proc/cpuinfo names it: model name, family / model / stepping, and the
    vector extensions the oracle's code paths use."""
    info = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if ":" not in line:
                    if info:
                        break  # the first processor's block is enough
                    continue
                k, v = (x.strip() for x in line.split(":", 1))
                info.setdefault(k, v)
    except OSError:
        return "unknown"
    flags = set(info.get("flags", "").split())
    ext = [f for f in ("avx2", "f16c", "fma", "avx512f", "avx512_bf16") if f in flags]
    return "%s (family %s model %s stepping %s; %s; %d logical CPUs on the host, %d usable)" % (
        info.get("model name", "unknown"), info.get("cpu family", "?"), info.get("model", "?"),
        info.get("stepping", "?"), " ".join(ext), os.cpu_count() or 0,
        len(os.sched_getaffinity(0)))


def cpu_library_arm(A, B, threads, budget_s=5.0):
    """numpy's fp32 BLAS matmul over a row sample of C1: a library bar next to the restatement
    (fp16 operands widened to fp32; the widening is outside the timed region)."""
    Bt = np.ascontiguousarray(B.astype(np.float32).T)
    N, K = B.shape
    A32 = A[:256].astype(np.float32)
    A32 @ Bt  # BLAS thread pool and page warm-up, not timed
    t = time.perf_counter()
    A32 @ Bt
    rate = 2 * 256 * N * K / (time.perf_counter() - t)
    rows = int(min(A.shape[0], max(256, budget_s * rate / (2 * N * K))))
    A32 = A[:rows].astype(np.float32)
    t = time.perf_counter()
    A32 @ Bt
    dt = time.perf_counter() - t
    return {"value": round(2 * rows * N * K / dt / 1e12, 5), "unit": "TFLOP/s",
            "kind": "library", "library": "numpy %s fp32 matmul (BLAS)" % np.__version__,
            "threads": threads,
            "sample": "C1 rows 0..%d (%dx%dx%d), %.2f s" % (rows - 1, rows, N, K, dt)}


def cpu_baseline(A, B, budget_s=12.0):
    """The oracle's fp32 sequential-k GEMM over C1 rows, repeated until about `budget_s` of
    CPU work (a bounded sample of the workload)."""
    from oracle import oracle as O

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))
    threads = min(threads, len(os.sched_getaffinity(0)))
    N, K = B.shape
    O.gemm_f16(A[:64], B, threads=threads)  # thread pool and page warm-up, not timed
    t = time.perf_counter()
    O.gemm_f16(A[:256], B, threads=threads)
    rate = 2 * 256 * N * K / (time.perf_counter() - t)
    rows = int(min(A.shape[0], max(256, budget_s * rate / (2 * N * K))))
    rows -= rows % 8
    reps = max(1, int(round(budget_s * rate / (2 * rows * N * K))))
    t = time.perf_counter()
    for _ in range(reps):
        O.gemm_f16(A[:rows], B, threads=threads)
    dt = time.perf_counter() - t
    out = {"value": round(2 * reps * rows * N * K / dt / 1e12, 5), "unit": "TFLOP/s",
            "cores": threads, "kind": "port", "cpu_model": cpu_model(),
            "sample": "C1 rows 0..%d (%dx%dx%d) x %d passes, %.1f s: oracle_gemm_f16, the C "
                      "restatement of kernels/naive/gemm_fp16.cu:60-68 (fp32 sequential-k FMA "
                      "per output, OpenMP over %d threads)" % (rows - 1, rows, N, K, reps, dt,
                                                               threads)}
    try:
        out["library_arm"] = cpu_library_arm(A, B, threads)
    except Exception as e:  # a missing BLAS is reported, not fatal
        out["library_arm"] = {"error": str(e)}
    out["w8a16_arm"] = cpu_w8a16_arm(threads)
    return out


def cpu_w8a16_arm(threads, budget_s=4.0):
    """The W8A16 CPU path (dequantise, then the fp32 sequential-k GEMM: oracle_gemm_w8a16) on a
    row sample of the (34816, 5120) decode shape, M = 16, both weight formats; reported as weight
    bytes streamed per second (the decode metric's unit) and TFLOP/s."""
    from oracle import oracle as O

    g = np.random.Generator(np.random.PCG64(5))
    K, M, G = 5120, 16, 128
    A = randn_f16((M, K), 6, 1.0 / np.sqrt(K))
    out = []
    for fmt in (1, 2):
        def make(n):
            if fmt == 1:
                q = g.integers(-127, 128, (n, K), dtype=np.int8)
                sc = (g.uniform(0.5, 1.5, n) / 127).astype(np.float16)
                return q, sc, None
            q = g.integers(0, 256, (n, K), dtype=np.uint8)
            sc = (g.uniform(0.5, 1.5, (n, K // G)) / 255).astype(np.float16)
            z = g.integers(100, 157, (n, K // G), dtype=np.uint8)
            return q, sc, z

        q, sc, z = make(1024)
        O.gemm_w8a16(A, q[:64], sc[:64], None if z is None else z[:64], G if fmt == 2 else 0,
                     fmt, threads)  # thread pool and page warm-up, not timed
        t = time.perf_counter()
        O.gemm_w8a16(A, q, sc, z, G if fmt == 2 else 0, fmt, threads)
        rate = 1024 / max(time.perf_counter() - t, 1e-6)
        n = int(min(34816, max(512, budget_s * rate)))
        n -= n % 64
        q, sc, z = make(n)
        t = time.perf_counter()
        O.gemm_w8a16(A, q, sc, z, G if fmt == 2 else 0, fmt, threads)
        dt = time.perf_counter() - t
        wbytes = n * K + (2 * n if fmt == 1 else 3 * n * K // G)
        out.append({"fmt": "sym_i8" if fmt == 1 else "asym_u8_g128", "M": M, "N": n, "K": K,
                    "s": round(dt, 2), "GBps": round(wbytes / dt / 1e9, 3),
                    "TFLOPs": round(2 * M * n * K / dt / 1e12, 5), "threads": threads,
                    "kind": "port", "what": "oracle_gemm_w8a16: dequantise (fp16_rn((q-z)*s)) "
                    "then fp32 sequential-k FMA per output"})
    return out


def measured_rate(kind):
    """A MEASURED rate of the plugin's table (GB/s or TFLOP/s) with its card date, or None."""
    try:
        from tempo.plugins.gfx950.machine import Gfx950Machine

        r = Gfx950Machine().peak(kind)
    except Exception:
        return None
    if r.status != "MEASURED":
        return None
    return {"value": r.value, "units": r.units, "symbol": r.symbol,
            "date": r.prov.card.date if r.prov and r.prov.card else None}


def read_sclk():
    """The engine clock the C1 kernel ran at, from the committed rocprofv3 --pmc summary
    (GRBM_GUI_ACTIVE / 8 XCDs / the dispatch's duration, its C1 row's "sclk GHz" column), or
    None.  The clock follows the matrix cores' load within microseconds -- a probe kernel queued
    right after a C1 launch already reads ~2.4 GHz, and amd-smi's per-XCD clock is not sampled
    fast enough -- so only a counter read during the dispatch itself gives it."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    with open(TRAFFIC_FILE, encoding="utf-8") as f:
        for line in f:
            c = [x.strip() for x in line.split("|")]
            if len(c) > 13 and c[1:5] == [str(C1["M"]), str(C1["N"]), str(C1["K"]), "0"]:
                try:
                    ghz = float(c[12])
                except ValueError:
                    return None
                return {"median_mhz": round(ghz * 1e3, 1),
                        "source": "profiles/counters_gemm_fp16_configs.md (C1 row): "
                                  "GRBM_GUI_ACTIVE / 8 XCDs / dispatch duration under "
                                  "rocprofv3 --pmc"}
    return None


def live_sclk(fn, stream, samples=5, settle_s=0.3, gap_s=0.1, budget_s=8.0):
    """The engine clock of this box under a sustained C1 load: C1 launched back to back while a
    second thread reads amd-smi's gfx clocks (`samples` reads, each the mean over the XCDs, after
    `settle_s` of load); the median read, or None when amd-smi gives nothing.  amd-smi's clock is
    a short-window average, so it is read under a load that lasts across the reads -- the timed
    run itself is too short for that -- and it complements the counter-derived clock of
    read_sclk, which is the dispatch's own but comes from the committed profile's box."""
    import threading

    from tempo.plugins.gfx950 import card

    vals = []

    def sampler():
        time.sleep(settle_s)
        for j in range(samples + 1):
            txt = card._run([card.AMD_SMI, "metric", "-g", "0", "--clock", "--json"], timeout=5)
            m = card.parse_metric(txt or "", 0)
            # the first read after the load starts still reports the idle clock: dropped
            if j > 0 and "gfx_clock_mhz" in m:
                vals.append(round(m["gfx_clock_mhz"], 1))
            time.sleep(gap_s)

    t = threading.Thread(target=sampler, daemon=True)
    t.start()
    t0 = time.time()
    i = 0
    while t.is_alive() and time.time() - t0 < budget_s:
        for _ in range(16):  # ~6 ms of C1 per batch; the host never runs far ahead
            fn(i)
            i += 1
        stream.synchronize()
    t.join(timeout=1.0)
    if not vals:
        return None
    return {"median_mhz": float(np.median(vals)), "samples_mhz": vals, "launches": i,
            "source": "amd-smi metric --clock (mean over XCDs) under back-to-back C1 launches"}


def decode_lines(steps):
    import torch
    from cuda_tempiler_amd import capi

    hbm = measured_rate("hbm_read_pure")

    out = []
    stream = torch.cuda.current_stream()
    g = np.random.Generator(np.random.PCG64(3))

    def rotate(nbytes):
        return max(2, -(-(512 << 20) // nbytes) + 1)

    # W8A16, both formats, shape (34816, 5120) and (5120, 17408)
    for (N, K) in ((34816, 5120), (5120, 17408)):
        for fmt in (1, 2):
            G = 128
            nb = N * K + (2 * N if fmt == 1 else 3 * N * K // G)
            copies = rotate(nb)
            W, S, Z = [], [], []
            for c in range(copies):
                if fmt == 1:
                    W.append(torch.randint(-127, 128, (N, K), dtype=torch.int8, device="cuda:0"))
                    S.append(torch.empty(N, dtype=torch.float16, device="cuda:0").uniform_(0.5, 1.5) / 127)
                    Z.append(None)
                else:
                    W.append(torch.randint(0, 256, (N, K), dtype=torch.uint8, device="cuda:0"))
                    S.append(torch.empty((N, K // G), dtype=torch.float16, device="cuda:0").uniform_(0.5, 1.5) / 255)
                    Z.append(torch.randint(100, 157, (N, K // G), dtype=torch.uint8, device="cuda:0"))
            for M in (1, 16, 32):
                A = to_dev((g.standard_normal((M, K), dtype=np.float32) / np.sqrt(K)).astype(np.float16))
                C = torch.empty((M, N), dtype=torch.float16, device="cuda:0")
                capi.gemm_w8a16(A, W[0], S[0], Z[0], fmt=fmt, group=G, C=C, stream=stream)
                ps = [capi.w8a16_params(A, W[c], S[c], Z[c], C, fmt, G) for c in range(copies)]
                fn = direct(capi.lib().tempo_gemm_w8a16_launch, ps, stream)
                settle_clocks(fn, stream, batch=50, min_s=DECODE_SETTLE_S)
                ms = time_launches(fn, steps, max(10, steps // 5), stream)
                byts = nb + 2 * M * K + 2 * M * N
                gbps = byts / (ms * 1e-3) / 1e9
                out.append({"op": "gemm_w8a16", "fmt": "sym_i8" if fmt == 1 else "asym_u8_g128",
                            "M": M, "N": N, "K": K, "us": round(ms * 1e3, 2),
                            "GBps": round(gbps, 1), "hbm_frac": round(gbps / PEAK_HBM_GBPS, 4),
                            "hbm_frac_measured": round(gbps / hbm["value"], 4) if hbm else None,
                            "route": capi.route(1 if fmt == 1 else 2, M, N, K)})
            del W, S, Z
    # fp16 decode (C2 shapes)
    for (N, K) in ((15360, 3840), (3840, 15360)):
        nb = 2 * N * K
        copies = rotate(nb)
        Bs = [torch.randn((N, K), dtype=torch.float16, device="cuda:0") for _ in range(copies)]
        for M in (1, 8, 16, 32):
            A = torch.randn((M, K), dtype=torch.float16, device="cuda:0")
            C = torch.empty((M, N), dtype=torch.float16, device="cuda:0")
            capi.gemm_fp16(A, Bs[0], C, stream=stream)
            ps = [capi.TempoGemmParams(capi._ptr(A), capi._ptr(Bs[c]), capi._ptr(C), M, N, K,
                                       K, K, N) for c in range(copies)]
            fn = direct(capi.lib().tempo_gemm_fp16_launch, ps, stream)
            settle_clocks(fn, stream, batch=50, min_s=DECODE_SETTLE_S)
            ms = time_launches(fn, steps, max(10, steps // 5), stream)
            byts = nb + 2 * M * K + 2 * M * N
            gbps = byts / (ms * 1e-3) / 1e9
            out.append({"op": "gemm_fp16", "M": M, "N": N, "K": K, "us": round(ms * 1e3, 2),
                        "GBps": round(gbps, 1), "hbm_frac": round(gbps / PEAK_HBM_GBPS, 4),
                        "hbm_frac_measured": round(gbps / hbm["value"], 4) if hbm else None,
                        "route": capi.route(0, M, N, K)})
        del Bs
    if hbm:
        out.append({"hbm_measured": hbm, "mode": "HBM.READ_PURE: nontemporal 16-byte loads, "
                    "4 GiB buffer (tempo.plugins.gfx950.calibrate)"})
    return out


def gate_up_lines(steps):
    """The fused gate/up epilogue on the production gate_up shape (2N = 34816, K = 5120; both
    W8A16 formats and fp16 weights) against the unfused chain on the same stream: the plain
    shipped GEMM into [M, 2N], then torch's silu and product.  Decode M (the streaming kernels)
    and prefill M (the interleaved kernels' fused epilogue)."""
    import torch
    import torch.nn.functional as F
    from cuda_tempiler_amd import capi

    out = []
    stream = torch.cuda.current_stream()
    N, K, G = 17408, 5120, 128
    for fmt in (1, 2, 0):
        wb = 2 if fmt == 0 else 1
        nb = 2 * N * K * wb + (4 * N if fmt == 1 else (6 * N * K // G if fmt == 2 else 0))
        copies = max(2, -(-(512 << 20) // nb) + 1)
        W, S, Z = [], [], []
        for c in range(copies):
            if fmt == 0:
                W.append(torch.randn((2 * N, K), dtype=torch.float16, device="cuda:0") / K ** 0.5)
                S.append(None)
                Z.append(None)
            elif fmt == 1:
                W.append(torch.randint(-127, 128, (2 * N, K), dtype=torch.int8, device="cuda:0"))
                S.append(torch.empty(2 * N, dtype=torch.float16, device="cuda:0").uniform_(0.5, 1.5) / 127)
                Z.append(None)
            else:
                W.append(torch.randint(0, 256, (2 * N, K), dtype=torch.uint8, device="cuda:0"))
                S.append(torch.empty((2 * N, K // G), dtype=torch.float16, device="cuda:0").uniform_(0.5, 1.5) / 255)
                Z.append(torch.randint(100, 157, (2 * N, K // G), dtype=torch.uint8, device="cuda:0"))
        for M in (1, 16, 32, 128, 2048):
            A = torch.randn((M, K), dtype=torch.float16, device="cuda:0") / K ** 0.5
            C = torch.empty((M, N), dtype=torch.float16, device="cuda:0")
            T = torch.empty((M, 2 * N), dtype=torch.float16, device="cuda:0")
            L = capi.lib()
            if fmt == 0:
                capi.gemm_fp16_gate_up(A, W[0], C, stream=stream)  # operand checks, once
                capi.gemm_fp16(A, W[0], T, stream=stream)
                pf = [capi.TempoGemmParams(capi._ptr(A), capi._ptr(W[c]), capi._ptr(C), M, N, K,
                                           K, K, N) for c in range(copies)]
                pp = [capi.TempoGemmParams(capi._ptr(A), capi._ptr(W[c]), capi._ptr(T), M, 2 * N,
                                           K, K, K, 2 * N) for c in range(copies)]
                fused = direct(L.tempo_gemm_fp16_gate_up_launch, pf, stream)
                plain = direct(L.tempo_gemm_fp16_launch, pp, stream)
            else:
                capi.gemm_w8a16_gate_up(A, W[0], S[0], Z[0], fmt=fmt, group=G, C=C, stream=stream)
                capi.gemm_w8a16(A, W[0], S[0], Z[0], fmt=fmt, group=G, C=T, stream=stream)
                pf = []
                for c in range(copies):
                    q = capi.w8a16_params(A, W[c], S[c], Z[c], C, fmt, G)
                    q.N = N  # the output width; the weights hold 2N rows
                    pf.append(q)
                pp = [capi.w8a16_params(A, W[c], S[c], Z[c], T, fmt, G) for c in range(copies)]
                fused = direct(L.tempo_gemm_w8a16_gate_up_launch, pf, stream)
                plain = direct(L.tempo_gemm_w8a16_launch, pp, stream)

            def unfused(i):
                plain(i)
                g, u = T.chunk(2, dim=-1)
                return F.silu(g) * u

            settle_clocks(fused, stream, batch=20, min_s=DECODE_SETTLE_S)
            ms_f = time_launches(fused, steps, max(10, steps // 5), stream)
            settle_clocks(unfused, stream, batch=20, min_s=DECODE_SETTLE_S)
            ms_u = time_launches(unfused, steps, max(10, steps // 5), stream)
            byts = nb + 2 * M * K + 2 * M * N
            gbps = byts / (ms_f * 1e-3) / 1e9
            tf = 2.0 * M * (2 * N) * K / (ms_f * 1e-3) / 1e12
            out.append({"op": "gate_up", "fmt": ["fp16", "sym_i8", "asym_u8_g128"][fmt],
                        "M": M, "N": N, "K": K, "us": round(ms_f * 1e3, 2),
                        "unfused_us": round(ms_u * 1e3, 2), "speedup": round(ms_u / ms_f, 3),
                        "GBps": round(gbps, 1), "hbm_frac": round(gbps / PEAK_HBM_GBPS, 4),
                        "TFLOPs": round(tf, 1), "mfma_frac": round(tf / PEAK_FP16_TFLOPS, 4),
                        "route": capi.route(3 + fmt, M, N, K)})
        del W, S, Z
    return out


def gptq_lines(steps):
    """Load-time GPTQ repack (checkpoint [K/4,N] int32 -> [N,K] bytes) on the model's two
    largest layers; algorithmic bytes = the checkpoint read once plus the repack written once."""
    import torch
    from cuda_tempiler_amd import capi

    out = []
    stream = torch.cuda.current_stream()
    for (K, N) in ((5120, 34816), (17408, 5120)):
        G = 128
        qw = torch.randint(-(2**31), 2**31 - 1, (K // 4, N), dtype=torch.int32, device="cuda:0")
        qz = torch.randint(-(2**31), 2**31 - 1, (K // G, N // 4), dtype=torch.int32, device="cuda:0")
        sc = torch.empty((K // G, N), dtype=torch.float16, device="cuda:0").uniform_(0.001, 0.021)
        wq = torch.empty((N, K), dtype=torch.uint8, device="cuda:0")
        so = torch.empty((N, K // G), dtype=torch.float16, device="cuda:0")
        zo = torch.empty((N, K // G), dtype=torch.uint8, device="cuda:0")
        lib = capi.lib()
        args = (capi._ptr(qw), capi._ptr(qz), capi._ptr(sc), K, N, G, capi._ptr(wq),
                capi._ptr(so), capi._ptr(zo), capi._stream(stream))
        fn = lambda i: capi._check(lib.tempo_gptq_repack_u8(*args), "tempo_gptq_repack_u8")
        ms = time_launches(fn, steps, max(5, steps // 5), stream)
        byts = 2 * (K * N + 3 * (K // G) * N)
        gbps = byts / (ms * 1e-3) / 1e9
        out.append({"op": "gptq_repack_u8", "K": K, "N": N, "us": round(ms * 1e3, 2),
                    "GBps": round(gbps, 1), "hbm_frac": round(gbps / PEAK_HBM_GBPS, 4)})
        del qw, qz, sc, wq, so, zo
    return out


def fmha_line(steps):
    import torch
    from cuda_tempiler_amd import capi

    B, S, H, Hkv, D = 1, 4096, 16, 8, 256
    Q = torch.randn((B, S, H, D), dtype=torch.float16, device="cuda:0")
    K = torch.randn((B, S, Hkv, D), dtype=torch.float16, device="cuda:0")
    V = torch.randn((B, S, Hkv, D), dtype=torch.float16, device="cuda:0")
    O = torch.empty_like(Q)
    L = torch.empty((B, H, S), dtype=torch.float32, device="cuda:0")
    stream = torch.cuda.current_stream()
    fn = lambda i: capi.fmha_fwd(Q, K, V, 1.0 / 16, True, O=O, LSE=L, stream=stream)
    # the decode lines before it leave the engine clock low: settle it as for C1, for at least
    # 0.3 s (the FMHA clock ramp is slow: 189 -> 163 us per launch over the first ~100 launches)
    settle = settle_clocks(fn, stream, batch=10, min_s=0.3)
    ms = time_launches(fn, steps, max(5, steps // 5), stream)
    flops = 4 * D * B * H * S * (S + 1) // 2
    tf = flops / (ms * 1e-3) / 1e12
    return {"op": "fmha_fwd", "config": "B=1 H=16 Hkv=8 S=4096 D=256 causal", "us": round(ms * 1e3, 1),
            "TFLOPs": round(tf, 1), "mfma_frac": round(tf / PEAK_FP16_TFLOPS, 4),
            "settle": settle}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-decode", action="store_true", help="skip the decode and FMHA lines")
    ap.add_argument("--no-settle", action="store_true",
                    help="skip the clock-settling launches before the warm-up and timed region")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="after the timed region, run a plain 1 GiB device copy three times (the "
                         "known-size kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (the GEMMs would "
              "shard by N with no exchange; see the sharding notes of the design document). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2

    from tempo.plugins.gfx950 import card

    card_before = card.wait_idle(0)  # before this process touches the GPU
    import torch
    from cuda_tempiler_amd import capi

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    capi.lib()  # loud failure if the HIP library is not built
    M, N, K = C1["M"], C1["N"], C1["K"]
    Ah = randn_f16((M, K), SEED_A, 1.0 / np.sqrt(K))
    Bh = randn_f16((N, K), SEED_B, 1.0 / np.sqrt(K))
    A, B = to_dev(Ah), to_dev(Bh)
    C = torch.empty((M, N), dtype=torch.int16, device="cuda:0").fill_(0x7f7f).view(torch.float16)
    stream = torch.cuda.Stream()  # default priority
    with torch.cuda.stream(stream):
        capi.gemm_fp16(A, B, C, stream=stream)
    torch.cuda.synchronize()
    gate = gate_c1(Ah, Bh, C.cpu().numpy())
    if not gate["ok"]:
        print(json.dumps({"error": "correctness gate failed", "gate": gate}), file=sys.stderr)
        return 1

    fn = lambda i: capi.gemm_fp16(A, B, C, stream=stream)
    torch.cuda.synchronize()
    settle = settle_clocks(fn, stream) if not args.no_settle else None
    ms = time_launches(fn, args.steps, args.warmup, stream)
    flops = 2 * M * N * K
    tflops = flops / (ms * 1e-3) / 1e12
    traffic = read_traffic()
    sclk = read_sclk()
    peak_sclk = 256 * 4096 * sclk["median_mhz"] * 1e6 / 1e12 if sclk else None
    live = live_sclk(fn, stream)
    peak_live = 256 * 4096 * live["median_mhz"] * 1e6 / 1e12 if live else None
    line = {
        "metric": METRIC, "value": round(tflops, 1), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "settle": settle,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic: A,B ~ N(0,1)/sqrt(K) fp16 from numpy PCG64 seeds 11/77",
        "config": {"workload": "C1 dense fp16 GEMM C=A.B^T M=4096 N=15360 K=3840, fp32 accumulate",
                   "kernel_row": capi.route(0, M, N, K), "parallelism": "single GPU"},
        "gate": gate,
        "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": PEAK_FP16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / PEAK_FP16_TFLOPS, 4),
                     "traffic": traffic,
                     "algorithmic_bytes": 2 * (M * K + N * K + M * N),
                     "sclk_mhz": sclk, "peak_at_sclk": round(peak_sclk, 1) if sclk else None,
                     "frac_at_sclk": round(tflops / peak_sclk, 4) if sclk else None,
                     "sclk_live_mhz": live,
                     "peak_at_sclk_live": round(peak_live, 1) if live else None,
                     "frac_at_sclk_live": round(tflops / peak_live, 4) if live else None,
                     "mfma_measured": measured_rate("tensor_measured")},
    }
    del C
    if args.copy_calibration:
        src = torch.empty(1 << 29, dtype=torch.float16, device="cuda:0").fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        line["copy_calibration_bytes"] = src.numel() * 2
        del src, dst
    if not args.no_decode:
        torch.cuda.empty_cache()
        line["decode"] = decode_lines(max(50, args.steps))
        torch.cuda.empty_cache()
        line["fmha"] = fmha_line(max(10, args.steps // 10))
        torch.cuda.empty_cache()
        line["gptq_repack"] = gptq_lines(max(20, args.steps // 4))
        torch.cuda.empty_cache()
        line["gate_up"] = gate_up_lines(max(50, args.steps // 2))
    torch.cuda.synchronize()
    card_after = card.snapshot(0)
    line["card"] = {"before": card_before, "after": card_after,
                    "clean": card.clean(card_before, card_after)}
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(Ah, Bh)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
