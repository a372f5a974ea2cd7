"""manifest.json of a shipped delivery (schema tempo/shipped/1, the reference's
kernels/shipped/gemm_fp16/sm_70/manifest.json fields, written for gfx950).

    python3 -m tempo.plugins.gfx950.manifest [--rows gpurun_out/rows_<op>.json ...]

Static part, derived here on the CPU: the op, layout and predicate; the dispatch ladder (read
from the delivery's own select.py); per ladder row the build numbers of OUR compile (VGPRs,
AGPRs, spills, scratch, LDS from hipcc's resource remarks, MFMA count and LDS-DMA use from
llvm-objdump), obtained by rendering the row's hyperform through the plugin and compiling it;
and an md5 over EVERY file of the delivery (kernel.hip, launch.h, launch.hip, dispatch.inc,
select.py), so no file ships unsigned.  Measured part: the rows written by
tempo.plugins.gfx950.measure_shipped on an MI355X, with the card state before and after.
"""
from __future__ import annotations

import argparse
import hashlib
import importlib.util
import json
import os
import random
import sys
import tempfile
from concurrent.futures import ProcessPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.abspath(os.path.join(HERE, "..", "..", ".."))
SHIPPED = os.path.join(ROOT, "kernels", "shipped")
SIGNED = ("kernel.hip", "launch.h", "launch.hip", "dispatch.inc", "dispatch_gate_up.inc",
          "select.py")
# files only some deliveries have (gemm_fp16's prefill translation unit); signed when present
SIGNED_OPTIONAL = ("launch_prefill.hip", "launch_prefill.h", "prefill.inc", "ship_probe.hip")

OPS = {
    "gemm_fp16": dict(dtype="fp16 x fp16 -> fp16, fp32 accumulate",
                      dtypes=("fp16", "fp16"), fmts=(0,)),
    "gemm_w8a16": dict(dtype="fp16 x (int8 sym per-channel | uint8 asym group-128) -> fp16, "
                             "dequantised to fp16 on the way into the MFMA feed, fp32 accumulate",
                       dtypes=("fp16", "int8"), fmts=(1, 2)),
}


def _select(op):
    path = os.path.join(SHIPPED, op, "gfx950", "select.py")
    spec = importlib.util.spec_from_file_location("sel_" + op, path)
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


def md5_of(op):
    d = os.path.join(SHIPPED, op, "gfx950")
    h = hashlib.md5()
    for f in signed_files(op):
        with open(os.path.join(d, f), "rb") as fh:
            h.update(f.encode() + b"\0" + fh.read())
    return h.hexdigest()


def signed_files(op):
    d = os.path.join(SHIPPED, op, "gfx950")
    return list(SIGNED) + [f for f in SIGNED_OPTIONAL if os.path.exists(os.path.join(d, f))]


def ladder_rows(sel):
    """Both ladders of a delivery: (M_max, N_min, tag, kind, params, epi); epi = 1 for the fused
    gate/up ladder."""
    return ([row + (0,) for row in sel.LADDER]
            + [row + (1,) for row in getattr(sel, "LADDER_GATE_UP", [])])


def hyper_params(kind, p, fmt, epi=0):
    """A ladder row of select.py (kind, template params) -> the plugin's hyperform params: the
    same kernel, named the way space.variants() names it."""
    pk = {"stream": "stream", "mfma": "reg", "dma": "dma", "shared": "shared", "ilv": "ilv",
          "ilv8": "ilv8", "line": "line", "phase": "phase"}[kind]
    # NMAX / KMIN / KMAX / FILL are the row's dispatch conditions, not kernel parameters
    params = {k: v for k, v in p.items() if k not in ("fmts", "NMAX", "KMIN", "KMAX", "FILL")}
    params["kind"] = pk
    if pk == "shared":
        params.setdefault("TPB", 1024)
    if pk == "line" and params.get("MT"):  # row tiles: the launcher bounds at 64 S threads
        params["TPB"] = 64 * params["S"]
    elif pk == "line" and params["MB"] >= 4:  # the shipped launchers bound these at 512 threads
        params.setdefault("SN", 1)
        params["TPB"] = 512
    if pk not in ("dma", "ilv"):
        params["BFMT"] = fmt
    if pk == "stream":
        params["ALDS"] = params.pop("A", 0)
    if pk == "dma":
        params.setdefault("XT", 0)
        params.setdefault("MINB", 1)
        params.setdefault("MS", 32)
    if pk in ("ilv", "ilv8") and params.get("SW", 0):
        params["SPLIT"] = 1  # the split-K instantiation of the kernel
    if pk == "phase" and params.get("KS", 1) > 1:
        params["KSL"] = 1  # the k-sliced instantiation of the kernel
    if epi:
        params["EPI"] = 1
    return params


# The register gate's fixture (tests/test_prune_acceptance.py): bodies of the plugin's own
# skeletons, compiled here, whose compiler numbers the pruner's pre-build estimate is held to.  A
# seeded sample of every kind over the op's canonical shapes, plus bodies heavy enough to spill,
# so that "a spilled body is never called FITS" is tested on real spills.
GATE_SHAPES = {0: ((4096, 15360, 3840), (16, 15360, 3840), (1, 3840, 15360)),
               1: ((16, 34816, 5120), (1, 5120, 17408)),
               2: ((16, 34816, 5120), (1, 5120, 17408))}
GATE_HEAVY = (dict(kind="stream", MB=1, R=4, U=8, ALDS=0), dict(kind="stream", MB=2, R=4, U=4, ALDS=0),
              dict(kind="stream", MB=1, R=4, U=4, ALDS=0),
              dict(kind="shared", MB=2, R=2, U=4, SN=2, TPB=1024),
              dict(kind="shared", MB=1, R=2, U=4, SN=2, TPB=1024))
GATE_PER_KIND = 6


def _spec(fmt, shape):
    from tempo.plugins.base import OpSpec

    M, N, K = shape
    return OpSpec(kind="gemm", dtype_a="fp16", dtype_b={0: "fp16", 1: "int8", 2: "uint8"}[fmt],
                  dtype_c="fp16", dtype_acc="fp32", layout_a="k", layout_b="k", layout_c="n",
                  shapes={"M": M, "N": N, "K": K})


def gate_bodies(op):
    """[(fmt, shape, params)]: deterministic (seeded) per op."""
    sys.path.insert(0, ROOT)
    from tempo.plugins.gfx950 import load

    plug = load()
    out, seen = [], set()
    for fmt in OPS[op]["fmts"]:
        rng = random.Random(950 + fmt)
        for shape in GATE_SHAPES[fmt]:
            by = {}
            for h in plug.skeletons.variants(_spec(fmt, shape)):
                by.setdefault(h.params["kind"], []).append(dict(h.params))
            for kind in sorted(by):
                pool = sorted(by[kind], key=lambda p: json.dumps(sorted(p.items())))
                for p in rng.sample(pool, min(len(pool), GATE_PER_KIND)):
                    k = json.dumps(sorted(p.items()))
                    if k not in seen:
                        seen.add(k)
                        out.append((fmt, shape, p))
        for hv in GATE_HEAVY:
            p = dict(hv, BFMT=fmt)
            k = json.dumps(sorted(p.items()))
            if k not in seen:
                seen.add(k)
                out.append((fmt, GATE_SHAPES[fmt][0], p))
    return out


def _compile_body(job):
    fmt, shape, params = job
    sys.path.insert(0, ROOT)
    from tempo.plugins.base import Hyperform
    from tempo.plugins.gfx950 import load

    plug = load()
    spec = _spec(fmt, shape)
    r = plug.skeletons.render(spec, Hyperform(plugin="gfx950", params=params, key="gate"))
    with tempfile.TemporaryDirectory() as td:
        src = os.path.join(td, r.filename)
        with open(src, "w") as f:
            f.write(r.source)
        b = plug.toolchain.compile(src, os.path.join(td, "k.o"), mode="device")
    if not b.ok:
        raise RuntimeError("gate body %s does not compile:\n%s" % (params, b.log[-2000:]))
    return dict(fmt=fmt, shape=list(shape), params=params, regs=b.regs, vgpr_spill=b.spill_st,
                scratch_bytes_per_lane=b.stack_frame)


def gate_numbers(op, jobs=8):
    with ProcessPoolExecutor(jobs) as ex:
        return list(ex.map(_compile_body, gate_bodies(op)))


# Ladder-row kinds whose operand copies are global->LDS DMA (a build of one of them with no LDS-DMA
# instruction has fallen back to register-staged loads)
DMA_KINDS = ("ilv", "ilv8", "dma", "line", "phase")
# Shipped rows allowed to keep a spill, with the reason and the measured cost of removing it
# (none today: the gate below refuses every spill)
SPILL_WAIVERS = {}


def gate_build(numbers: dict, waivers: dict = None) -> list:
    """The build gate of the verify stage: every shipped row compiles with no spilled VGPR or
    SGPR, no scratch and no scratch instruction (reference: the spill and stack numbers read
    per build, tempo/plugins/sm70/toolchain.py:102-112, and the loop-spill field of the
    contract's BuildResult, tempo/plugins/base.py:534), and every LDS-DMA kind copies through
    LDS-DMA.  Returns the failures as "row: reason" lines; a waived row is listed as waived."""
    waivers = SPILL_WAIVERS if waivers is None else waivers
    bad = []
    for key, b in numbers.items():
        why = []
        if b.get("vgpr_spill") or b.get("sgpr_spill"):
            why.append("spills %d VGPRs, %d SGPRs" % (b.get("vgpr_spill", 0), b.get("sgpr_spill", 0)))
        if b.get("scratch_bytes_per_lane") or b.get("scratch_insts"):
            why.append("scratch %d B/lane, %d scratch instructions"
                       % (b.get("scratch_bytes_per_lane", 0), b.get("scratch_insts", 0)))
        if b.get("kind") in DMA_KINDS and not b.get("lds_dma"):
            why.append("kind %s without an LDS-DMA copy" % b.get("kind"))
        if why and key not in waivers and b.get("tag") not in waivers:
            bad.append("%s: %s" % (key, "; ".join(why)))
    return bad


def source_numbers(plug, src, kind, tag):
    """Compile one kernel source alone (device code object) and read the build's numbers and
    its instruction mix."""
    from tempo.plugins.gfx950.classifier import parse_disasm
    from tempo.plugins.gfx950.toolchain import isa_summary

    with tempfile.TemporaryDirectory() as td:
        obj = os.path.join(td, "k.o")
        b = plug.toolchain.compile(src, obj, mode="device")
        if not b.ok:
            raise RuntimeError("row %s does not compile:\n%s" % (tag, b.log[-3000:]))
        isa = isa_summary(sum(parse_disasm(plug.toolchain.disasm(obj), operands=True).values(),
                              []))
    return dict(tag=tag, kind=kind, regs=b.regs, vgpr_spill=b.spill_st, sgpr_spill=b.spill_ld,
                scratch_bytes_per_lane=b.stack_frame, lds_static=b.smem_static, mfma=isa["mfma"],
                lds_dma=isa["lds_dma"], lds_dma_buffer=isa["lds_dma_buffer"],
                buffer_load=isa["buffer_load"], ds_read_b128=isa["ds_read_b128"],
                scratch_insts=isa["scratch"])


def row_numbers(plug, spec, h, kind, tag):
    """A ladder row rendered by the plugin, compiled alone: source_numbers()."""
    r = plug.skeletons.render(spec, h)
    with tempfile.TemporaryDirectory() as td:
        src = os.path.join(td, r.filename)
        with open(src, "w") as f:
            f.write(r.source)
        return source_numbers(plug, src, kind, tag)


def build_numbers(op, gate: bool = True):
    """Compile each ladder row's kernel alone (rendered by the plugin) and read our numbers; with
    gate=True a row that fails gate_build() stops the manifest."""
    sys.path.insert(0, ROOT)
    from tempo.plugins.base import Hyperform, OpSpec
    from tempo.plugins.gfx950 import load

    plug = load()
    sel = _select(op)
    out = {}
    for fmt in OPS[op]["fmts"]:
        db = {0: "fp16", 1: "int8", 2: "uint8"}[fmt]
        spec = OpSpec(kind="gemm", dtype_a="fp16", dtype_b=db, dtype_c="fp16", dtype_acc="fp32",
                      layout_a="k", layout_b="k", layout_c="n",
                      shapes={"M": 4096, "N": 15360, "K": 3840})
        for m_max, n_min, tag, kind, p, epi in ladder_rows(sel):
            if fmt not in p.get("fmts", (fmt,)):
                continue
            params = hyper_params(kind, p, fmt, epi)
            h = Hyperform(plugin="gfx950", params=params, key="%s_f%d" % (tag, fmt))
            key = tag if len(OPS[op]["fmts"]) == 1 else "%s/fmt%d" % (tag, fmt)
            out[key] = row_numbers(plug, spec, h, kind, tag)
    if gate:
        bad = gate_build(out)
        if bad:
            raise RuntimeError("build gate failed for %s:\n  %s" % (op, "\n  ".join(bad)))
    return out


def card_passport(before, after):
    """The manifest's card block from the measure stage's card states (card.snapshot() taken
    before and after the run): the reference's passport keys (manifest.json:107-113) with the
    clocks observed instead of locked."""
    from tempo.plugins.gfx950 import card

    before, after = before or {}, after or {}
    out = card.passport(before, after, name=before.get("name", ""))
    out["gcn_arch"] = before.get("gcn_arch")
    out["clean"] = card.clean(before, after)
    return out


def fold_counters(rows, counter_files, op, md5=None):
    """Attach the counter step's per-launch figures (measure_shipped --counters) to the measured
    rows of the same shape and format; returns how many rows got them.  A counter file taken on
    other sources than md5 (the rows') is refused."""
    n = 0
    for cf_ in counter_files:
        with open(cf_) as f:
            got = json.load(f)
        if got.get("op") != op:
            continue
        if md5 is not None and got.get("source_md5") != md5:
            raise ValueError("%s was taken on other sources than the rows (%s vs %s)"
                             % (cf_, got.get("source_md5"), md5))
        by = {(r["M"], r["N"], r["K"], r["fmt"]): r for r in got["rows"]}
        for row in rows:
            c = by.get((row["M"], row["N"], row["K"], row["fmt"]))
            if c is not None:
                row["counters"] = dict(c["counters"], groups=got.get("groups"),
                                       route=c.get("route"))
                n += 1
    return n


def make(op, rows_files=(), counter_files=()):
    sel = _select(op)
    d = os.path.join(SHIPPED, op, "gfx950")
    path = os.path.join(d, "manifest.json")
    old = {}
    if os.path.exists(path):
        with open(path) as f:
            old = json.load(f)
    man = {
        "schema": "tempo/shipped/1",
        "op": "gemm" if op == "gemm_fp16" else "gemm_w8a16",
        "arch": "gfx950",
        "dtype": OPS[op]["dtype"],
        "layout": "C = A . B^T, both operands k-contiguous (row-major [M,K] and [N,K]), C [M,N]",
        "predicate": {
            "alignment": "A, B 16 B; C 8 B; lda, ldb multiples of 8 elements, ldc of 4",
            "M": "any (rows beyond M are predicated in the tiled kernels)",
            "per_row_fit": "see dispatch[].fit",
            "fallback": "hipErrorInvalidConfiguration (TEMPO_FALLBACK): the caller's own path",
        },
        "dispatch_rule": "rows in order; the first whose band holds (M, N) and whose kernel fits "
                         "the shape runs; none -> fallback",
        "dispatch": [],
        "dispatch_gate_up": [],
        "build": build_numbers(op),
        "gate": gate_numbers(op),
        "source_md5": md5_of(op),
        "source_md5_of": signed_files(op),
        "rows": old.get("rows", []),
        "card": old.get("card", None),
    }
    if "rows_source_md5" in old:
        man["rows_source_md5"] = old["rows_source_md5"]
    for m_max, n_min, tag, kind, p, epi in ladder_rows(sel):
        if kind == "stream":
            fit = "N %% %d == 0 and K %% %d == 0" % (sel.STREAM_N_ROWS * p["R"],
                                                    sel.STREAM_K_STEP * p["U"])
        elif kind == "shared":
            spw = p["SN"] // 2 if epi else p["SN"]
            fit = "N %% %d == 0 and K %% %d == 0" % (sel.STREAM_N_ROWS * p["R"] * spw,
                                                    sel.STREAM_K_STEP * p["U"])
        elif kind == "ilv":
            fit = "N %% %d == 0 and K %% %d == 0 and K <= %d" % (p["BN"], max(64, p["BK"]),
                                                                 sel.ilv_ld_max(p))
        elif kind == "ilv8":
            fit = "N %% %d == 0 and K %% 128 == 0 and K <= %d" % (p["BN"], sel.ilv_ld_max(p))
        elif kind == "phase":
            fit = ("N %% 256 == 0, N / 256 %% 4 == 0 and ceil(N / 256 / 16) == %d, K %% 1024 == 0, "
                   "LDS <= 160 KiB" % p["NS"])
            if p.get("KS", 1) > 1:
                fit = ("N %% (256 / %d) == 0 with N / (256 / %d) rows per workgroup (%% 4 == 0, "
                       "ceil(rows / 16) == %d), K %% %d == 0 with >= 8 steps per slice, LDS <= "
                       "160 KiB; %d k slices, fp32 partials added in order"
                       % (p["KS"], p["KS"], p["NS"], 128 * p["KS"], p["KS"]))
            if "KMIN" in p:
                fit += " and K >= %d" % p["KMIN"]
            if "NMAX" in p:
                fit += " and N < %d" % p["NMAX"]
            if "KMAX" in p:
                fit += " and K < %d" % p["KMAX"]
        elif kind == "line" and p.get("TL"):
            fit = ("N %% %d == 0 and K %% %d == 0 and K <= %d; tail grid: q = (N / %d) // %d >= 1 "
                   "whole rounds, at most %d slabs left, q + 1 workgroups resident per CU" % (
                       sel.STREAM_N_ROWS * p["R"], sel.LINE_K_STEP, sel.LINE_K_MAX,
                       sel.STREAM_N_ROWS * p["R"], sel.LINE_CUS * p["SN"], sel.LINE_CUS))
        elif kind == "line":
            fit = "N %% %d == 0 and K %% %d == 0 and K <= %d" % (
                sel.STREAM_N_ROWS * p["R"] * p.get("SN", 1), sel.LINE_K_STEP, sel.LINE_K_MAX)
            if "NMAX" in p:
                fit += " and N < %d" % p["NMAX"]
        else:
            fit = "N %% %d == 0 and K %% %d == 0" % (p["BN"], p["BK"])
            if "NMAX" in p:
                fit += " and N < %d" % p["NMAX"]
        if kind in ("ilv", "ilv8"):
            if "NMAX" in p:
                fit += " and N < %d" % p["NMAX"]
            if "KMIN" in p:
                fit += " and K >= %d" % p["KMIN"]
            if "KMAX" in p:
                fit += " and K < %d" % p["KMAX"]
            if p.get("SW"):
                fit += "; split-K: at most %d workgroups, >= %d k-tiles per split" % (
                    p["SW"], p.get("MINKT", 0))
        man["dispatch" if not epi else "dispatch_gate_up"].append(dict(
                                    M_max=m_max, N_min=n_min, tag=tag, kind=kind,
                                    params={k: v for k, v in p.items() if k != "fmts"},
                                    fmts=list(p.get("fmts", OPS[op]["fmts"])), fit=fit))
    if op == "gemm_w8a16":
        man["predicate"]["formats"] = {"1": "int8 weights, fp16 scale per output channel",
                                       "2": "uint8 weights, fp16 scale + uint8 zero per (row, 128 k)"}
    for rf in rows_files:
        with open(rf) as f:
            got = json.load(f)
        if got.get("op") != op:
            continue
        man["rows"] = got["rows"]
        man["card"] = card_passport(got.get("card_before"), got.get("card_after"))
        man["rows_source_md5"] = got.get("source_md5")  # the sources the rows were timed on
    fold_counters(man["rows"], counter_files, op, man.get("rows_source_md5"))
    with open(path, "w") as f:
        json.dump(man, f, indent=1)
        f.write("\n")
    return path


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--rows", nargs="*", default=[])
    ap.add_argument("--counters", nargs="*", default=[])
    ap.add_argument("--op", nargs="*", default=list(OPS))
    a = ap.parse_args()
    for op in a.op:
        print(make(op, a.rows, a.counters))


if __name__ == "__main__":
    main()
