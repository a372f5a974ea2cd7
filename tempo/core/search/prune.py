"""Pruning without building: the plugin's resource verdict first, then the model's time bound.

Rules (the reference's pruner semantics, tempo/core/search/prune.py:52-151):
  * a hyperform whose resource verdict is a LAUNCH refusal (a code in HARD_CODES: more LDS than
    a workgroup may hold, no register budget at all) is cut -- that launch cannot happen;
  * a register verdict that is only an estimate (suspected spill) is advice: the hyperform is
    kept and the note says so; the build decides;
  * a hyperform the verdict cannot be computed for is cut (nothing is known that would let it
    run);
  * a hyperform the model is silent about, or cannot bound, is kept (no cut on ignorance);
  * of the rest, a hyperform whose bound is more than `bound_slack` times the best bound is cut.
    The bound is a lower bound, not a prediction, so the slack is wide.

Design: every hyperform is first ASSESSED independently (verdict, then bound), which yields an
Assessment; the best bound is taken over the assessments; then each assessment is DECIDED into a
Candidate.  Output order is input order.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

from tempo.core.model.bound import bound

HARD_CODES = frozenset({"WALL_SMEM", "NO_BUDGET"})

# decisions (Candidate.decision)
CUT_NO_VERDICT = "cut:no-verdict"
CUT_LAUNCH = "cut:launch-refused"
CUT_SLACK = "cut:bound-slack"
KEPT_BOUNDED = "kept:bounded"
KEPT_SILENT = "kept:model-silent"
KEPT_UNBOUNDED = "kept:no-bound"


@dataclass
class Assessment:
    hyper: object
    verdict: Optional[object] = None
    bound: Optional[object] = None
    error: str = ""          # why the verdict or the bound could not be computed

    @property
    def bounded(self) -> bool:
        return self.bound is not None and not self.bound.silent


@dataclass
class Candidate:
    hyper: object
    verdict: object
    bound: object
    kept: bool
    reason: str
    decision: str = ""

    def render(self) -> str:
        return "%-5s %-42s %s" % ("KEEP" if self.kept else "CUT", getattr(self.hyper, "key", "?"),
                                  self.reason)


def assess(plugin, op, h, channels) -> Assessment:
    a = Assessment(h)
    try:
        regs, max_live, lds = plugin.skeletons.resources_of(op, h)
        launch = plugin.skeletons.launch_of(op, h)
        a.verdict = plugin.resources.verdict(
            regs, max_live, lds, launch.threads, launch.min_ctas_per_sm,
            bound_threads=getattr(launch, "bound_threads", 0))
    except Exception as e:  # the plugin could not judge it
        a.error = "no resource verdict: %s" % e
        return a
    if not a.verdict.ok and a.verdict.code in HARD_CODES:
        return a
    try:
        a.bound = bound(plugin.skeletons.estimate_atoms(op, h), channels,
                        warps_per_sm=a.verdict.occ.warps_per_sm)
    except Exception as e:
        a.error = "no bound (%s)" % e
    return a


def decide(a: Assessment, best: Optional[float], keep_silent: bool, bound_slack: float) -> Candidate:
    v, b = a.verdict, a.bound
    if v is None:
        return Candidate(a.hyper, None, None, False, a.error, CUT_NO_VERDICT)
    if not v.ok and v.code in HARD_CODES:
        return Candidate(a.hyper, v, None, False, "%s: %s" % (v.code, v.explain), CUT_LAUNCH)
    note = "" if v.ok else "suspected spill (an estimate: kept, the build decides); "
    if b is None:
        return Candidate(a.hyper, v, None, keep_silent,
                         note + a.error + " -- kept, not cut on ignorance", KEPT_UNBOUNDED)
    if b.silent:
        return Candidate(a.hyper, v, b, keep_silent, note + "model silent: " + b.silent_reason,
                         KEPT_SILENT)
    if best is not None and b.T > bound_slack * best:
        return Candidate(a.hyper, v, b, False, note + "bound %.1f exceeds %.1f x the best %.1f"
                         % (b.T, bound_slack, best), CUT_SLACK)
    return Candidate(a.hyper, v, b, True, note + "%s; T >= %.1f, bound by %s"
                     % (v.code, b.T, b.binding), KEPT_BOUNDED)


def prune(plugin, op, hyperforms, keep_silent: bool = True, bound_slack: float = 4.0):
    """One Candidate per hyperform, in input order.  Builds and runs nothing."""
    channels = plugin.machine.channels()
    assessed = [assess(plugin, op, h, channels) for h in hyperforms]
    bounds = [a.bound.T for a in assessed if a.bounded]
    best = min(bounds) if bounds else None
    return [decide(a, best, keep_silent, bound_slack) for a in assessed]


def kept(cands):
    return [c for c in cands if c.kept]


def summary(cands) -> str:
    by = {}
    for c in cands:
        by[c.decision] = by.get(c.decision, 0) + 1
    risky = sum(1 for c in cands if c.kept and c.verdict is not None and not c.verdict.ok)
    parts = ", ".join("%s %d" % (k, by[k]) for k in sorted(by))
    return "hyperforms %d, kept %d (suspected spill %d); %s" % (
        len(cands), sum(c.kept for c in cands), risky, parts)
