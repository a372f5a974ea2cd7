"""Pipeline closure on gfx950 and the pruner's acceptance rule, executed against OUR measured
manifests (the pattern of reference tests/test_prune_acceptance.py:119-308).

Part 1 -- closure.  Every measured row of both shipped deliveries (kernels/shipped/*/gfx950/
manifest.json, written on an MI355X by measure_shipped) names the kernel that won that shape.
For each row the naive input of its operation is recognised from its TEMPO-OP block
(kernels/naive/gemm_fp16.hip, gemm_w8a16_sym.hip, gemm_w8a16.hip), the plugin enumerates the
space, and the core prunes it without building.  FAILS if the winner's exact hyperform is not in
the enumeration (a hole in the axes) or the pruner throws it away (a kernel that was built and
measured declared hopeless unbuilt).  PRINTS the winner's rank by the model bound and the
bound_slack it would need: quality of the model, not correctness.

Part 2 -- the register gate (reference test_prune_acceptance.py:186-308).  The pruner estimates
registers before a body exists; the fixture is the compiler's own numbers for bodies of our
skeletons (manifest "build" = the ladder rows, "gate" = a seeded sample plus bodies heavy enough
to spill).  The gate asks for the DIRECTION of the error, not its size:
  A1  a body the compiler spilled is never called FITS;
  A2  a body the compiler built without spilling is never cut;
  B0  the budget is the one declared to the compiler: no body exceeds it, and every spilled
      body sits at it;
  B   the pessimistic edge does not understate the compiler on clean bodies that stayed under
      the budget (a body AT the budget without spilling took what it was given: no claim);
  V   the falsifier: the optimistic edge in the pessimistic role must FAIL the gate.

    python3 tests/test_prune_acceptance.py        # prints the tables
"""
from __future__ import annotations

import json
import os
import statistics
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from tempo.core.op import recognize  # noqa: E402
from tempo.core.search.prune import HARD_CODES, prune  # noqa: E402
from tempo.plugins.base import Hyperform  # noqa: E402
from tempo.plugins.gfx950 import load, manifest  # noqa: E402

NAIVE = {0: "kernels/naive/gemm_fp16.hip", 1: "kernels/naive/gemm_w8a16_sym.hip",
         2: "kernels/naive/gemm_w8a16.hip"}
OPS = ("gemm_fp16", "gemm_w8a16")
# below this M the weight stream binds; the model's rank there is reported separately
M_RIDGE = 32


def _manifest(op):
    with open(os.path.join(ROOT, "kernels", "shipped", op, "gfx950", "manifest.json")) as f:
        return json.load(f)


def _same(h, want):
    return dict(h.params) == want


def closure(verbose=True):
    plug = load()
    lost, missing = [], []
    ranks = {"decode": [], "prefill": []}
    need_slack = 0.0
    n = 0
    for opname in OPS:
        man = _manifest(opname)
        ladder = {t: (k, p) for _, _, t, k, p in manifest._select(opname).LADDER}
        if verbose:
            print("%s: %d measured rows" % (opname, len(man["rows"])))
            print("  %-6s %-6s %-5s %-3s %-20s %6s %6s %6s" % ("M", "N", "K", "fmt", "winner",
                                                            "space", "kept", "rank"))
        for row in man["rows"]:
            n += 1
            M, N, K, fmt, win = row["M"], row["N"], row["K"], row["fmt"], row["winner"]
            if win not in ladder:
                missing.append("%s M%d N%d K%d: winner %s is not a ladder row" % (opname, M, N, K, win))
                continue
            kind, p = ladder[win]
            want = manifest.hyper_params(kind, p, fmt)
            op = recognize.from_file(os.path.join(ROOT, NAIVE[fmt]), {"M": M, "N": N, "K": K})
            hyper = list(plug.skeletons.variants(op))
            cands = prune(plug, op, hyper)
            mine = [c for c in cands if _same(c.hyper, want)]
            if not mine:
                missing.append("%s M%d N%d K%d fmt%d: %s is not in the enumeration"
                               % (opname, M, N, K, fmt, win))
                continue
            if not mine[0].kept:
                lost.append("%s M%d N%d K%d fmt%d: winner %s CUT: %s"
                            % (opname, M, N, K, fmt, win, mine[0].reason))
            ranked = sorted([c for c in cands if c.kept and c.bound is not None
                             and not c.bound.silent], key=lambda c: c.bound.T)
            pos = [i for i, c in enumerate(ranked) if _same(c.hyper, want)]
            rank = pos[0] + 1 if pos else None
            if rank:
                ranks["decode" if M <= M_RIDGE else "prefill"].append(rank)
            wide = [c for c in prune(plug, op, hyper, bound_slack=float("inf"))
                    if c.bound is not None and not c.bound.silent]
            w_mine = [c for c in wide if _same(c.hyper, want)]
            if wide and w_mine:
                need_slack = max(need_slack, min(c.bound.T for c in w_mine)
                                 / min(c.bound.T for c in wide))
            if verbose:
                print("  %-6d %-6d %-5d %-3d %-20s %6d %6d %6s%s"
                      % (M, N, K, fmt, win, len(cands), sum(c.kept for c in cands),
                         rank or "-", "   <-- CUT" if not mine[0].kept else ""))
    if verbose:
        for r in lost + missing:
            print("  FAIL: " + r)
        print("  measured winners cut: %d of %d" % (len(lost), n))
        for band, arr in ranks.items():
            if arr:
                print("  winner rank by bound, %s: %d..%d, median %.0f (%d rows)"
                      % (band, min(arr), max(arr), statistics.median(arr), len(arr)))
        print("  bound_slack the winners need: %.2f (pruner default 4.0)" % need_slack)
    return lost, missing, need_slack


def _gate_rows():
    """(tag, fmt, shape, params, compiler regs, spilled) for every body of both manifests."""
    out = []
    for opname in OPS:
        man = _manifest(opname)
        ladder = {t: (k, p, e) for _, _, t, k, p, e in manifest.ladder_rows(manifest._select(opname))}
        for key, b in man["build"].items():
            tag, _, f = key.partition("/fmt")
            fmt = int(f) if f else 0
            kind, p, epi = ladder[tag]
            out.append((key, fmt, tuple(manifest.GATE_SHAPES[fmt][0]),
                        manifest.hyper_params(kind, p, fmt, epi), int(b["regs"]),
                        bool(b["vgpr_spill"] or b["scratch_bytes_per_lane"])))
        for b in man["gate"]:
            out.append(("gate", b["fmt"], tuple(b["shape"]), b["params"], int(b["regs"]),
                        bool(b["vgpr_spill"] or b["scratch_bytes_per_lane"])))
    return out


def regs_gate(verbose=True, optimistic=False):
    """-> list of claims against the estimator (empty = the gate holds)."""
    plug = load()
    R = plug.resources
    claims = []
    band = {}
    gran = 8
    for tag, fmt, shape, params, cc, spilled in _gate_rows():
        op = manifest._spec(fmt, shape)
        h = Hyperform(plugin="gfx950", params=params, key=tag)
        regs, max_live, smem = plug.skeletons.resources_of(op, h)
        if optimistic:
            max_live = regs
        lau = plug.skeletons.launch_of(op, h)
        budget = R.declared_budget(lau.threads, lau.min_ctas_per_sm, lau.bound_threads)
        v = R.verdict(regs, max_live, min(smem, 160 * 1024), lau.threads, lau.min_ctas_per_sm,
                      bound_threads=lau.bound_threads)
        name = "%s %s" % (tag, {k: x for k, x in params.items()})
        if spilled and v.code == "FITS":
            claims.append("A1 spilled body called FITS: %s (compiler %d, budget %d)"
                          % (name, cc, budget))
        if not spilled and v.code in HARD_CODES:
            claims.append("A2 clean body cut (%s): %s" % (v.code, name))
        if cc > budget:
            claims.append("B0 compiler %d over the declared budget %d: %s" % (cc, budget, name))
        if spilled and cc < budget - gran:
            claims.append("B0 spilled at %d, below the declared budget %d: %s" % (cc, budget, name))
        if not spilled and cc < budget and max_live < cc:
            claims.append("B pessimistic edge %d under the compiler's %d: %s" % (max_live, cc, name))
        if not spilled and cc < budget:
            band.setdefault(params["kind"], []).append(max_live / cc)
    if verbose:
        print("register gate%s: %d bodies" % (" (optimistic edge)" if optimistic else "",
                                              len(_gate_rows())))
        for kind, arr in sorted(band.items()):
            print("  %-7s pessimistic edge / compiler on clean bodies: %.2f..%.2f (%d)"
                  % (kind, min(arr), max(arr), len(arr)))
        for c in claims:
            print("  " + c)
    return claims


# ---------------------------------------------------------------------------------------- tests


def test_no_measured_winner_is_cut_or_missing():
    lost, missing, need = closure(verbose=True)
    assert not missing, missing
    assert not lost, lost
    assert need <= 4.0


def test_every_measured_row_was_measured_on_the_shipped_sources():
    for opname in OPS:
        man = _manifest(opname)
        assert man["rows"], "%s has no measured rows" % opname
        assert man.get("rows_source_md5") == man["source_md5"] == manifest.md5_of(opname), opname


def test_naive_inputs_recognise_to_the_three_formats():
    ops = {f: recognize.from_file(os.path.join(ROOT, p), {"M": 8, "N": 64, "K": 128})
           for f, p in NAIVE.items()}
    assert [ops[f].dtype_b for f in (0, 1, 2)] == ["fp16", "int8", "uint8"]
    assert ops[2].scale and ops[1].scale and ops[0].scale is None
    from tempo.plugins.gfx950 import space

    assert [space.bfmt(ops[f]) for f in (0, 1, 2)] == [0, 1, 2]


def test_register_gate_holds():
    rows = _gate_rows()
    assert sum(1 for r in rows if r[5]) >= 5, "the fixture must hold real spills"
    assert sum(1 for r in rows if not r[5]) >= 50
    claims = regs_gate(verbose=True)
    assert not claims, "\n".join(claims)


def test_register_gate_falsifier():
    """The optimistic edge in the pessimistic role must fail: a gate that passes both ways
    checks nothing."""
    assert regs_gate(verbose=False, optimistic=True)


if __name__ == "__main__":
    closure(verbose=True)
    print()
    regs_gate(verbose=True)
    print()
    print("falsifier claims: %d" % len(regs_gate(verbose=False, optimistic=True)))
