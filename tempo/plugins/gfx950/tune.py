"""The variant driver of the gfx950 plugin: enumerate -> prune -> build -> gate -> paired timing ->
rows.  Reference flow: bench/tempolate_gemm.py:5-11 (the tempolator loop), the harness's gate and
timer (tempo/plugins/sm70/skeletons/gemm_hmma884/harness.cu:92-103,161-268) and the report parse
(bench/tempolate_report.py:21-34).

Two phases, because the build runs on the CPU and the measurement on the GPU:

  plan (CPU)  python3 -m tempo.plugins.gfx950.tune plan gemm_w8a16 --shape 128 5120 17408 2 \\
                  [--shape ...] [--kinds ilv8 line] [--per-kind 6] [--out DIR]
      For each shape: the naive input of its weight format is recognised from its TEMPO-OP
      block (kernels/naive/*.hip), the plugin enumerates the space, the core prunes it without
      building (tempo/core/search/prune.py), and the kept hyperforms are ranked by the model
      bound, the first --per-kind of each kind becoming candidates.  Each candidate is written
      as a row of the delivery's own ladder language (launcher expression and fit predicate from
      the delivery's gen_dispatch.py), so it runs exactly the code a shipped row would.  The
      harness library (tune_harness.hip + the candidates) is compiled into DIR/libtune.so.
  run (GPU)   python3 -m tempo.plugins.gfx950.tune run DIR
      Per shape and candidate, in the reference's order (tempo/core/measure/correctness.py:21-27):
      poison the output (0x7f7f), launch, gate (no poison left, relL2 <= 3e-3 against the naive
      kernel on the GPU), and only then time it in paired rounds against the shipped row (the
      library's own dispatcher), the arms interleaved, weights rotated through > 512 MiB, the
      median of the per-round ratios reported (tempo/core/measure/ratio.py:63-73).  Rows go to
      DIR/rows.json: every candidate's gate and timing, and per shape the winner.
  report      python3 -m tempo.plugins.gfx950.tune report DIR
  peak (GPU)  python3 -m tempo.plugins.gfx950.tune peak DIR
      the MFMA-only throughput probe of the harness: the rate the matrix cores sustain on this
      part with no memory traffic (1 and 2 waves per SIMD).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import ctypes as ct
import importlib.util
import json
import os
import statistics
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.abspath(os.path.join(HERE, "..", "..", ".."))
SHIPPED = os.path.join(ROOT, "kernels", "shipped")
NAIVE = {0: "kernels/naive/gemm_fp16.hip", 1: "kernels/naive/gemm_w8a16_sym.hip",
         2: "kernels/naive/gemm_w8a16.hip"}
DELIVERY = {"gemm_fp16": ("gen", "GemmParams"), "gemm_w8a16": ("gen8", "W8A16Params")}
PREFILL_KIND = {"gemm_fp16": "ilv", "gemm_w8a16": "ilv8"}
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["-O3", "-std=c++17", "--offload-arch=gfx950", "-fPIC", "-Xclang", "-target-feature",
         "-Xclang", "-packed-fp32-ops", "-Wno-unused-result"]
PREFILL_FLAGS = ["-mllvm", "-amdgpu-sched-strategy=iterative-minreg"]
ROUNDS = 5


def _say(*a):
    print(*a, flush=True)


def _module(path, name):
    spec = importlib.util.spec_from_file_location(name, path)
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


def delivery_dir(op):
    return os.path.join(SHIPPED, op, "gfx950")


# ---- hyperform -> ladder row ------------------------------------------------------------------
def row_of(params: dict):
    """A hyperform of the plugin's space as a row of the delivery's ladder: (kind, row params), or
    None when no shipped launcher runs that hyperform (the launchers fix some axes: the dma
    launcher runs XT = 0 / MINB = 1, the line launcher its own thread bound, and the ring kind
    has no launcher at all).  Inverse of tempo.plugins.gfx950.manifest.hyper_params."""
    p = dict(params)
    kind = p.pop("kind")
    p.pop("BFMT", None)
    p.pop("SPLIT", None)
    p.pop("KSL", None)  # the phase kernel's k-sliced instantiation follows from KS
    if kind == "ring":
        return None
    if kind == "dma":
        if p.pop("XT", 0) or p.pop("MINB", 1) != 1:
            return None
    if kind == "stream":
        p["A"] = p.pop("ALDS", 0)
    if kind == "line" and p.get("MT"):
        return ("line", p) if p.pop("TPB", 0) == 64 * p["S"] else None
    if kind == "line":
        tpb = p.pop("TPB", 1024)
        if tpb != (512 if p["MB"] >= 4 else 1024):
            return None
        if p.get("SN", 1) == 1:
            p.pop("SN", None)
        if not p.get("TL"):
            p.pop("TL", None)
    if kind == "shared" and p.get("TPB", 1024) == 1024:
        p.pop("TPB", None)
    return ({"reg": "mfma"}.get(kind, kind), p)


def _match(params: dict, where) -> bool:
    """--where filters: KEY=VALUE pairs, each a hyperform's params must match; VALUE may list
    alternatives separated by commas (KEY=2,3,4).  Values compare as ints when they parse."""
    for cond in where or ():
        key, _, val = cond.partition("=")
        wants = [int(v) if v.lstrip("-").isdigit() else v for v in val.split(",")]
        if params.get(key, {"SW": 0, "SPLIT": 0, "SN": 1, "KS": 1, "TL": 0, "TAIL": 0}.get(key)) not in wants:
            return False
    return True


def plan(op, shapes, kinds=None, per_kind=6, out="gpurun_out/tune", where=()):
    sys.path.insert(0, ROOT)
    from tempo.core.op import recognize
    from tempo.core.search.prune import prune
    from tempo.plugins.gfx950 import load, space

    plug = load()
    gd = _module(os.path.join(delivery_dir(op), "gen_dispatch.py"), "tune_gd_" + op)
    sel = gd._select()
    cands, by_inst = [], {}
    plan_shapes = []
    for (M, N, K, fmt) in shapes:
        spec = recognize.from_file(os.path.join(ROOT, NAIVE[fmt]), {"M": M, "N": N, "K": K})
        hyps = list(plug.skeletons.variants(spec))
        pruned = prune(plug, spec, hyps)
        kept = [c for c in pruned if c.kept]
        groups = {}
        for c in kept:
            k = dict(c.hyper.params)["kind"]
            if kinds and k not in kinds:
                continue
            if not _match(dict(c.hyper.params), where):
                continue
            groups.setdefault(k, []).append(c)
        chosen = []
        for k, cs in sorted(groups.items()):
            cs.sort(key=lambda c: (c.bound is None or c.bound.silent,
                                   c.bound.T if c.bound is not None else 0.0, c.hyper.key))
            n = 0
            for c in cs:
                r = row_of(c.hyper.params)
                if r is None:
                    continue
                chosen.append((c, r))
                n += 1
                if n >= per_kind:
                    break
        ids = []
        for c, (kind, rp) in chosen:
            inst = gd.instantiation(kind, rp)
            if inst not in by_inst:
                _, fit = gd.condition(sel, kind, rp, 1 << 30)
                by_inst[inst] = len(cands)
                cands.append(dict(id=len(cands), tag=c.hyper.key, kind=kind, row=rp, inst=inst,
                                  fit=fit, bound=(None if c.bound is None or c.bound.silent
                                                  else c.bound.T)))
            ids.append(by_inst[inst])
        plan_shapes.append(dict(M=M, N=N, K=K, fmt=fmt, enumerated=len(hyps), kept=len(kept),
                                candidates=ids))
        _say("plan %s M=%d N=%d K=%d fmt=%d: %d hyperforms, %d kept, %d candidates"
             % (op, M, N, K, fmt, len(hyps), len(kept), len(ids)))
    os.makedirs(out, exist_ok=True)
    with open(os.path.join(out, "plan.json"), "w") as f:
        json.dump(dict(op=op, shapes=plan_shapes, candidates=cands), f, indent=1)
    build(op, cands, out)
    return out


def build(op, cands, out):
    """Compile the harness library of a plan: the candidate table (default scheduler) and, in a
    second translation unit, the prefill kind's launchers (its scheduler flag)."""
    ns, params = DELIVERY[op]
    pk = PREFILL_KIND[op]
    with open(os.path.join(out, "cands.inc"), "w") as f:
        for c in cands:
            f.write('TEMPO_CAND(%d, "%s", %s,\n           (%s))\n'
                    % (c["id"], c["tag"], c["fit"], c["inst"]))
    pre = [c for c in cands if c["kind"] == pk]
    with open(os.path.join(out, "prefill_tu.hip"), "w") as f:
        f.write("// generated by tempo.plugins.gfx950.tune: the plan's %s launchers\n"
                '#include "launch_prefill.h"\n\nnamespace tempo {\nnamespace %s {\n' % (pk, ns))
        for c in pre:
            f.write("template hipError_t %s(const %s&, hipStream_t, const Workspace&);\n"
                    % (c["inst"], params))
        f.write("}  // namespace %s\n}  // namespace tempo\n" % ns)
    inc = ["-I", out, "-I", delivery_dir(op)]
    defs = ["-DTEMPO_NS=%s" % ns, "-DTEMPO_PARAMS=%s" % params]
    jobs = [([HIPCC] + FLAGS + defs + inc + ["-c", os.path.join(HERE, "tune_harness.hip"), "-o",
                                            os.path.join(out, "harness.o")]),
            ([HIPCC] + FLAGS + PREFILL_FLAGS + inc + ["-c", os.path.join(out, "prefill_tu.hip"),
                                                      "-o", os.path.join(out, "prefill.o")])]

    def run(cmd):
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode:
            raise RuntimeError("harness build failed:\n%s\n%s" % (" ".join(cmd), r.stderr[-5000:]))

    with cf.ThreadPoolExecutor(2) as ex:
        list(ex.map(run, jobs))
    run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", os.path.join(out, "libtune.so"),
         os.path.join(out, "harness.o"), os.path.join(out, "prefill.o")])
    _say("built %s (%d candidates)" % (os.path.join(out, "libtune.so"), len(cands)))


# ---- GPU phase ----------------------------------------------------------------------------------
def _load(out):
    L = ct.CDLL(os.path.join(out, "libtune.so"))
    L.tempo_tune_count.restype = ct.c_int
    L.tempo_tune_id.restype = ct.c_int
    L.tempo_tune_id.argtypes = [ct.c_int]
    L.tempo_tune_tag.restype = ct.c_char_p
    L.tempo_tune_tag.argtypes = [ct.c_int]
    L.tempo_tune_fits.restype = ct.c_int
    L.tempo_tune_fits.argtypes = [ct.c_int, ct.c_void_p]
    L.tempo_tune_launch.restype = ct.c_int
    L.tempo_tune_launch.argtypes = [ct.c_int, ct.c_void_p, ct.c_void_p]
    L.tempo_tune_workspace.restype = ct.c_size_t
    L.tempo_tune_workspace.argtypes = [ct.c_int, ct.c_void_p]
    L.tempo_tune_mfma_peak.restype = ct.c_int
    L.tempo_tune_mfma_peak.argtypes = [ct.c_int, ct.c_int, ct.POINTER(ct.c_float), ct.c_void_p,
                                       ct.c_void_p]
    return L


def _events_ms(fn, iters, stream):
    import torch

    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(iters):
        fn(i)
    e1.record(stream)
    e1.synchronize()
    return e0.elapsed_time(e1) / iters


def _rel_l2(got, ref):
    import torch

    g, r = got.double(), ref.double()
    den = torch.sum(r * r).item()
    return float(torch.sqrt(torch.sum((g - r) ** 2) / den).item()) if den > 0 else 0.0


def run(out):
    import torch

    sys.path.insert(0, ROOT)
    from cuda_tempiler_amd import capi

    with open(os.path.join(out, "plan.json")) as f:
        pl = json.load(f)
    op = pl["op"]
    L = _load(out)
    index = {L.tempo_tune_id(i): i for i in range(L.tempo_tune_count())}
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    sp = ct.c_void_p(stream.cuda_stream)
    gen = torch.Generator(device=dev)
    rows = []
    for sh in pl["shapes"]:
        M, N, K, fmt = sh["M"], sh["N"], sh["K"], sh["fmt"]
        _say("shape %s M=%d N=%d K=%d fmt=%d" % (op, M, N, K, fmt))
        gen.manual_seed(7 * M + N + K + fmt)
        A = (torch.randn((M, K), generator=gen, device=dev) / K ** 0.5).half()
        wbytes = 2 * N * K if fmt == 0 else N * K + (2 * N if fmt == 1 else 3 * N * K // 128)
        copies = max(2, -(-(512 << 20) // wbytes) + 1)
        Ws, Ss, Zs = [], [], []
        for _ in range(copies):
            if fmt == 0:
                Ws.append((torch.randn((N, K), generator=gen, device=dev) / K ** 0.5).half())
                Ss.append(None)
                Zs.append(None)
            elif fmt == 1:
                Ws.append(torch.randint(-127, 128, (N, K), generator=gen, device=dev,
                                        dtype=torch.int8))
                Ss.append((torch.rand(N, generator=gen, device=dev) + 0.5).div(127).half())
                Zs.append(None)
            else:
                Ws.append(torch.randint(0, 256, (N, K), generator=gen, device=dev,
                                        dtype=torch.uint8))
                Ss.append((torch.rand((N, K // 128), generator=gen, device=dev) + 0.5)
                          .div(255).half())
                Zs.append(torch.randint(100, 157, (N, K // 128), generator=gen, device=dev,
                                        dtype=torch.uint8))
        F0 = Ws[0] if fmt == 0 else capi.dequant_tile(Ws[0], Ss[0], Zs[0], fmt, 0, 0, N, K)
        ref = capi.naive_gemm_fp16(A, F0)
        C = torch.empty((M, N), dtype=torch.float16, device=dev)
        torch.cuda.synchronize()

        def params(i, Cout):
            j = i % copies
            if fmt == 0:
                return capi.TempoGemmParams(capi._ptr(A), capi._ptr(Ws[j]), capi._ptr(Cout), M, N,
                                            K, A.stride(0), Ws[j].stride(0), Cout.stride(0))
            return capi.w8a16_params(A, Ws[j], Ss[j], Zs[j], Cout, fmt, 128)

        pars = [params(i, C) for i in range(copies)]

        def shipped(i):
            if fmt == 0:
                capi.gemm_fp16(A, Ws[i % copies], C, stream=stream)
            else:
                capi.gemm_w8a16(A, Ws[i % copies], Ss[i % copies], Zs[i % copies], fmt=fmt, C=C,
                                stream=stream)

        ship_route = capi.route(fmt, M, N, K)
        results = []
        for cid in sh["candidates"]:
            cand = pl["candidates"][cid]
            i = index[cid]
            res = dict(id=cid, tag=cand["tag"], kind=cand["kind"], row=cand["row"])
            p0 = pars[0]
            if not L.tempo_tune_fits(i, ct.byref(p0)):
                res["gate"] = "does not fit"
                results.append(res)
                continue
            C.view(torch.int16).fill_(0x7f7f)
            torch.cuda.synchronize()
            rc = L.tempo_tune_launch(i, ct.byref(p0), sp)
            torch.cuda.synchronize()
            if rc != 0:
                res["gate"] = "launch error %d" % rc
                results.append(res)
                continue
            poison = int((C.view(torch.int16) == 0x7f7f).sum().item())
            rel = _rel_l2(C, ref)
            res.update(poison=poison, rel_l2=rel, workspace=int(L.tempo_tune_workspace(
                i, ct.byref(p0))))
            if poison or not rel <= 3e-3:
                res["gate"] = "FAIL"
                results.append(res)
                _say("  GATE FAIL %s poison=%d rel=%.3e" % (cand["tag"], poison, rel))
                continue
            res["gate"] = "pass"

            def cand_fn(k, i=i):
                L.tempo_tune_launch(i, ct.byref(pars[k % copies]), sp)

            for f in (shipped, cand_fn):
                for k in range(3):
                    f(k)
            torch.cuda.synchronize()
            t0 = _events_ms(cand_fn, 3, stream)
            it = int(min(500, max(3, 60.0 / max(t0, 1e-3))))
            ratios, tc, ts = [], [], []
            for _ in range(ROUNDS):
                a = _events_ms(shipped, it, stream)
                b = _events_ms(cand_fn, it, stream)
                ts.append(a)
                tc.append(b)
                ratios.append(a / b)
            ms = statistics.median(tc)
            flops = 2.0 * M * N * K
            byts = wbytes + 2 * M * K + 2 * M * N
            res.update(us=ms * 1e3, shipped_us=statistics.median(ts) * 1e3,
                       speedup_vs_shipped=statistics.median(ratios), tflops=flops / ms / 1e9,
                       GBps=byts / ms / 1e6, iters=it, rounds=ROUNDS)
            results.append(res)
            _say("  %-44s %8.2f us  x%.3f vs shipped %s (%.2f us)"
                 % (cand["tag"], ms * 1e3, res["speedup_vs_shipped"], ship_route,
                    res["shipped_us"]))
        timed = [r for r in results if "us" in r]
        win = min(timed, key=lambda r: r["us"]) if timed else None
        rows.append(dict(M=M, N=N, K=K, fmt=fmt, shipped_route=ship_route,
                         enumerated=sh["enumerated"], kept=sh["kept"], candidates=results,
                         winner=(win["tag"] if win else None),
                         winner_us=(win["us"] if win else None),
                         winner_speedup_vs_shipped=(win["speedup_vs_shipped"] if win else None)))
        del Ws, Ss, Zs, F0, ref
        torch.cuda.empty_cache()
    path = os.path.join(out, "rows.json")
    with open(path, "w") as f:
        json.dump(dict(op=op, rows=rows), f, indent=1)
    _say("wrote %s" % path)
    return path


def report(out):
    with open(os.path.join(out, "rows.json")) as f:
        got = json.load(f)
    for r in got["rows"]:
        _say("%s M=%d N=%d K=%d fmt=%d  shipped %s  (%d hyperforms, %d kept)"
             % (got["op"], r["M"], r["N"], r["K"], r["fmt"], r["shipped_route"], r["enumerated"],
                r["kept"]))
        for c in sorted(r["candidates"], key=lambda c: c.get("us", 1e30)):
            if "us" in c:
                _say("   %-46s %9.2f us  %7.1f TFLOP/s  %7.0f GB/s  x%.3f"
                     % (c["tag"], c["us"], c["tflops"], c["GBps"], c["speedup_vs_shipped"]))
            else:
                _say("   %-46s %s" % (c["tag"], c["gate"]))


def peak(out):
    import torch

    L = _load(out)
    scratch = torch.empty(256 * 8 * 4 * 256, dtype=torch.float32, device="cuda:0")
    stream = torch.cuda.current_stream()
    res = []
    for w in (1, 2):
        us = ct.c_float(0)
        iters = 4000
        rc = L.tempo_tune_mfma_peak(w, iters, ct.byref(us), ct.c_void_p(scratch.data_ptr()),
                                    ct.c_void_p(stream.cuda_stream))
        if rc:
            raise RuntimeError("peak probe failed: %d" % rc)
        flop = 16 * 16 * 32 * 2 * 4.0 * iters * (256 * w * 4) * 4
        res.append(dict(waves_per_simd=w, us=us.value, tflops=flop / (us.value * 1e-6) / 1e12))
        _say("MFMA-only probe, %d wave(s) per SIMD: %.1f us, %.1f TFLOP/s" % (w, us.value,
                                                                              res[-1]["tflops"]))
    return res


def main():
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    a = sub.add_parser("plan")
    a.add_argument("op", choices=sorted(DELIVERY))
    a.add_argument("--shape", nargs=4, type=int, action="append", required=True,
                   metavar=("M", "N", "K", "FMT"))
    a.add_argument("--kinds", nargs="*")
    a.add_argument("--per-kind", type=int, default=6)
    a.add_argument("--where", nargs="*", default=[], metavar="KEY=VALUE",
                   help="keep only hyperforms whose params match (e.g. BM=128 SW=0,256)")
    a.add_argument("--out", default="gpurun_out/tune")
    for name in ("run", "report", "peak"):
        b = sub.add_parser(name)
        b.add_argument("out")
    args = ap.parse_args()
    if args.cmd == "plan":
        plan(args.op, [tuple(s) for s in args.shape], args.kinds, args.per_kind, args.out,
             args.where)
    elif args.cmd == "run":
        run(args.out)
    elif args.cmd == "report":
        report(args.out)
    else:
        peak(args.out)
    return 0


if __name__ == "__main__":
    sys.exit(main())
