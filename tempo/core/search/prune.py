"""Pruning without building (reference tempo/core/search/prune.py:52-171).

Resource verdict first, then the model bound.  Only WALL_SMEM and NO_BUDGET cut (a launch that
cannot happen); a suspected spill is an estimate and is KEPT with a note -- the build decides.
Variants the model is silent about are kept.  The bound cuts only variants more than
`bound_slack` times worse than the best bound."""
from __future__ import annotations

from dataclasses import dataclass

from tempo.core.model.bound import bound

HARD_CODES = frozenset({"WALL_SMEM", "NO_BUDGET"})


@dataclass
class Candidate:
    hyper: object
    verdict: object
    bound: object
    kept: bool
    reason: str

    def render(self) -> str:
        return "%s %-42s %s" % ("KEPT   " if self.kept else "CUT    ",
                                getattr(self.hyper, "key", "?"), self.reason)


def prune(plugin, op, hyperforms, keep_silent: bool = True, bound_slack: float = 4.0):
    channels = plugin.machine.channels()
    out, rows, best = [], [], None
    for h in hyperforms:
        try:
            regs, max_live, smem = plugin.skeletons.resources_of(op, h)
            lau = plugin.skeletons.launch_of(op, h)
            v = plugin.resources.verdict(regs, max_live, smem, lau.threads, lau.min_ctas_per_sm,
                                         bound_threads=getattr(lau, "bound_threads", 0))
        except Exception as e:
            out.append(Candidate(h, None, None, False, "no resource verdict: %s" % e))
            continue
        if not v.ok and v.code in HARD_CODES:
            out.append(Candidate(h, v, None, False, "%s: %s" % (v.code, v.explain)))
            continue
        advice = "" if v.ok else "SUSPECTED SPILL (estimate, kept; the build decides); "
        try:
            atoms = plugin.skeletons.estimate_atoms(op, h)
            b = bound(atoms, channels, warps_per_sm=v.occ.warps_per_sm)
        except Exception as e:
            out.append(Candidate(h, v, None, keep_silent,
                                 advice + "no bound (%s) -- kept, not cut on ignorance" % e))
            continue
        rows.append((h, v, b, advice))
        if not b.silent and (best is None or b.T < best):
            best = b.T
    for h, v, b, advice in rows:
        if b.silent:
            out.append(Candidate(h, v, b, keep_silent, advice + "MODEL SILENT: " + b.silent_reason))
        elif best is not None and b.T > best * bound_slack:
            out.append(Candidate(h, v, b, False, advice + "bound %.1f is over %.1fx the best %.1f"
                                 % (b.T, bound_slack, best)))
        else:
            out.append(Candidate(h, v, b, True, advice + "%s; T >= %.1f, bound by %s"
                                 % (v.code, b.T, b.binding)))
    return out


def kept(cands):
    return [c for c in cands if c.kept]


def summary(cands) -> str:
    k = sum(1 for c in cands if c.kept)
    silent = sum(1 for c in cands if c.bound is not None and c.bound.silent)
    risky = sum(1 for c in cands if c.kept and c.verdict is not None and not c.verdict.ok)
    return ("hyperforms %d, kept %d (of which suspected spill %d), cut %d (silent model %d)"
            % (len(cands), k, risky, len(cands) - k, silent))
