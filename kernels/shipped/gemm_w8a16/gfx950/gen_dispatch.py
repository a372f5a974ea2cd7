#!/usr/bin/env python3
"""Generates dispatch.inc from select.py: one source of the ladder, two consumers.

    python3 gen_dispatch.py > dispatch.inc

The Python predicate is what a host tree calls once at load time; the instantiation table is
what the compiler needs.  The second is generated from the first so they cannot drift
(reference: kernels/shipped/gemm_fp16/sm_70/gen_dispatch.py:6-13).
"""
from __future__ import annotations

import importlib.util
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))


def _select():
    spec = importlib.util.spec_from_file_location("tempo_select_w8a16_gfx950",
                                                  os.path.join(HERE, "select.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


HEAD = """// GENERATED from select.py -- do not edit.  Regenerate with:
//   python3 kernels/shipped/gemm_w8a16/gfx950/gen_dispatch.py > dispatch.inc
//
// Ladder, one TEMPO_ROW(band, fit, launcher, tag) per row; launch.hip expands it twice (launch
// and route).  The first row whose band holds (M, N) and whose kernel fits the shape runs; if
// none does, the answer is hipErrorInvalidConfiguration: the caller's own path takes over
// (TEMPO_FALLBACK) -- a legal answer, not a failure.
"""


def instantiation(kind, p, epi=0):
    tail = ",%d" % epi if epi else ""
    if kind == "phase" and p.get("KS", 1) > 1:  # k slices across workgroups: a workspace row
        if epi:
            raise ValueError("k slices take the plain epilogue")
        return "launch_phase_ks<%d,%d,%d,%d>" % (p["MB"], p["NS"], p["D"], p["KS"])
    if kind == "phase":
        return "launch_phase%s<%d,%d,%d>" % ("_gu" if epi else "", p["MB"], p["NS"], p["D"])
    if kind == "line" and p.get("MT"):  # row tiles x slab groups
        if epi or p.get("TL") or p.get("KS", 1) > 1:
            raise ValueError("row tiles take the plain epilogue, whole k and no tail grid")
        return "launch_line_mt<%d,%d,%d,%d>" % (p["MB"], p["R"], p["D"], p["S"])
    if kind == "line" and p.get("KS", 1) > 1:  # k slices across workgroups: a workspace row
        if epi or p.get("TL"):
            raise ValueError("k slices take the plain epilogue and no tail grid")
        return "launch_line_ks<%d,%d,%d,%d,%d,%d>" % (p["MB"], p["R"], p["D"], p.get("SN", 1),
                                                      p["W"], p["KS"])
    if kind == "line":
        if p.get("TL"):
            tail = ",%d,1" % epi
        return "launch_line<%d,%d,%d,%d,%d%s>" % (p["MB"], p["R"], p["D"], p.get("SN", 1), p["W"],
                                                  tail)
    if kind == "shared":
        return "launch_shared<%d,%d,%d,%d,%d%s>" % (p["MB"], p["R"], p["U"], p["SN"],
                                                    p.get("TPB", 1024), tail)
    if kind == "stream":
        return "launch_stream<%d,%d,%d,%d%s>" % (p["MB"], p["R"], p["U"], p.get("A", 0), tail)
    if epi and kind == "ilv8" and p.get("TAIL"):  # output columns in two parts
        return "launch_ilv8_gu_tail<%d,%d,%d,%d,%d,%d,%d,%d,%d,%s>" % (
            p["BM"], p["BN"], p["BK"], p["WM"], p["WN"], p["STAGES"], p["GROUP"], p["XCD"],
            p["RSP"], ",".join(str(v) for v in _select().ILV8_TAIL[p["TAIL"]]))
    if epi and kind == "ilv8":
        return "launch_ilv8_gu<%d,%d,%d,%d,%d,%d,%d,%d,%d>" % (
            p["BM"], p["BN"], p["BK"], p["WM"], p["WN"], p["STAGES"], p["GROUP"], p["XCD"],
            p["RSP"])
    if epi:
        raise ValueError("the fused gate/up epilogue exists for the stream and interleaved kernels")
    if kind == "ilv8" and p.get("TAIL"):  # N in two parts: whole rounds, then the tail part
        return "launch_ilv8_tail<%d,%d,%d,%d,%d,%d,%d,%d,%d,%s>" % (
            p["BM"], p["BN"], p["BK"], p["WM"], p["WN"], p["STAGES"], p["GROUP"], p["XCD"],
            p["RSP"], ",".join(str(v) for v in _select().ILV8_TAIL[p["TAIL"]]))
    if kind == "ilv8":
        return "launch_ilv8<%d,%d,%d,%d,%d,%d,%d,%d,%d,%d,%d>" % (
            p["BM"], p["BN"], p["BK"], p["WM"], p["WN"], p["STAGES"], p["GROUP"], p["XCD"],
            p["RSP"], p.get("SW", 0), p.get("MINKT", 0))
    return "launch_mfma<%d,%d,%d,%d,%d,%d,%d,%d,%d>" % (
        p["BM"], p["BN"], p["BK"], p["WM"], p["WN"], p["MS"], p["SWZ"], p["GROUP"], p["XCD"])


def condition(sel, kind, p, m_max, n_min=0, gate_up=False):
    if kind == "phase":
        if p.get("KS", 1) > 1:
            fit = "(phase_ks_fits<%d,%d,%d,%d>(p))" % (p["MB"], p["NS"], p["D"], p["KS"])
        else:
            fit = "(phase%s_fits<%d,%d,%d>(p))" % ("_gu" if gate_up else "", p["MB"], p["NS"],
                                                    p["D"])
        if "KMIN" in p:
            fit += " && p.K >= %d" % p["KMIN"]
        if "NMAX" in p:
            fit += " && p.N < %d" % p["NMAX"]
        if "KMAX" in p:
            fit += " && p.K < %d" % p["KMAX"]
    elif kind == "line" and p.get("TL"):
        fit = "(p.N %% %d) == 0 && (p.K %% %d) == 0 && (line_tail_fits<%d,%d,%d,%d,%d>(p))" % (
            sel.STREAM_N_ROWS * p["R"], sel.LINE_K_STEP, p["MB"], p["R"], p["D"], p["SN"],
            1 if gate_up else 0)
    elif kind == "line" and p.get("MT"):
        fit = "(p.N %% %d) == 0 && (p.K %% %d) == 0 && p.K <= %d" % (
            sel.STREAM_N_ROWS * p["R"], sel.LINE_K_STEP, sel.LINE_K_MAX)
        if "NMAX" in p:
            fit += " && p.N < %d" % p["NMAX"]
        fit += " && (line_mt_fits<%d,%d,%d,%d>(p))" % (p["MB"], p["R"], p["D"], p["S"])
    elif kind == "line":
        sno = p.get("SN", 1) // 2 if gate_up and p.get("SN", 1) >= 2 else p.get("SN", 1)
        fit = "(p.N %% %d) == 0 && (p.K %% %d) == 0 && p.K <= %d" % (
            sel.STREAM_N_ROWS * p["R"] * sno, sel.LINE_K_STEP, sel.LINE_K_MAX)
        if "NMAX" in p:
            fit += " && p.N < %d" % p["NMAX"]
        if "KMIN" in p:
            fit += " && p.K >= %d" % p["KMIN"]
    elif kind == "stream":
        fit = "(p.N %% %d) == 0 && (p.K %% %d) == 0" % (sel.STREAM_N_ROWS * p["R"],
                                                          sel.STREAM_K_STEP * p["U"])
    elif kind == "shared":
        spw = p["SN"] // 2 if gate_up else p["SN"]  # gate/up: the slab waves pair up
        fit = "(p.N %% %d) == 0 && (p.K %% %d) == 0" % (sel.STREAM_N_ROWS * p["R"] * spw,
                                                          sel.STREAM_K_STEP * p["U"])
    elif kind == "ilv8":  # a scale group is two k-tiles; 31-bit panel byte offsets
        fit = "(p.N %% %d) == 0 && (p.K %% 128) == 0 && p.lda <= %d && p.ldw <= %d" % (
            p["BN"] // 2 if gate_up else p["BN"], sel.ilv_ld_max(p), sel.ilv_ld_max(p))
        if "NMAX" in p:
            fit += " && p.N < %d" % p["NMAX"]
        if "KMIN" in p:
            fit += " && p.K >= %d" % p["KMIN"]
        if "KMAX" in p:
            fit += " && p.K < %d" % p["KMAX"]
        if p.get("TAIL") == 2:  # fits only where N splits in two
            fit += " && (ilv8_tail_cols<%d,%d>(p) > 0)" % (p["BM"], p["BN"])
        if p.get("FILL"):  # one round of its tiles, more of them than 256-row tiles give
            fit += " && (ilv8_fill_fits<%d,%d>(p))" % (p["BM"], p["BN"])
    else:
        fit = "(p.N %% %d) == 0 && (p.K %% %d) == 0" % (p["BN"], p["BK"])
        if "NMAX" in p:
            fit += " && p.N < %d" % p["NMAX"]
    band = "p.M <= %d" % m_max
    if n_min:
        band += " && p.N >= %d" % n_min
    if "fmts" in p:
        band += " && (%s)" % " || ".join("p.fmt == %d" % f for f in p["fmts"])
    return band, fit


HEAD_GATE_UP = """// GENERATED from select.py (LADDER_GATE_UP) -- do not edit.  Regenerate with:
//   python3 kernels/shipped/gemm_w8a16/gfx950/gen_dispatch.py --gate-up > dispatch_gate_up.inc
//
// Fused gate/up ladder: p.N is the output width, the weights hold 2N rows (gate, then up).  Same
// row rule as dispatch.inc; none -> hipErrorInvalidConfiguration.
"""


def render(gate_up: bool = False) -> str:
    sel = _select()
    out = [HEAD_GATE_UP if gate_up else HEAD]
    for m_max, n_min, tag, kind, p in (sel.LADDER_GATE_UP if gate_up else sel.LADDER):
        band, fit = condition(sel, kind, p, m_max, n_min, gate_up)
        out.append("TEMPO_ROW(%s, %s,\n          (%s), \"%s\")"
                   % (band, fit, instantiation(kind, p, 1 if gate_up else 0), tag))
    out.append("TEMPO_FALLBACK_ROW")
    return "\n".join(out) + "\n"


HEAD_PREFILL = """// GENERATED from select.py -- do not edit.  Regenerate with:
//   python3 kernels/shipped/gemm_w8a16/gfx950/gen_dispatch.py --prefill > prefill.inc
//
// Explicit instantiations of the interleaved int8 prefill launchers the ladder names; included
// by launch_prefill.hip, the translation unit that builds k_gemm_ilv8.
"""


def render_prefill() -> str:
    sel = _select()
    out = [HEAD_PREFILL]
    seen = set()
    for _m, _n, _tag, kind, p, epi in ([r + (0,) for r in sel.LADDER]
                                       + [r + (1,) for r in sel.LADDER_GATE_UP]):
        if kind != "ilv8":
            continue
        inst = instantiation(kind, p, epi)
        if inst in seen:
            continue
        seen.add(inst)
        out.append("template hipError_t %s(const W8A16Params&, hipStream_t, const Workspace&);"
                   % inst)
    return "\n".join(out) + "\n"


def main():
    if "--prefill" in sys.argv[1:]:
        sys.stdout.write(render_prefill())
    else:
        sys.stdout.write(render(gate_up="--gate-up" in sys.argv[1:]))
    return 0


if __name__ == "__main__":
    sys.exit(main())
