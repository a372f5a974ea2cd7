"""Correctness gate arithmetic (reference tempo/core/op/oracle.py:28-151).

A small relL2 against the reference is NECESSARY but not SUFFICIENT: it only proves the
arithmetic on the data both sides saw.  The gate passes only with a named independent path
(differing in one node, e.g. fp64 on sampled cells) that also agrees."""
from __future__ import annotations

from dataclasses import dataclass, field


@dataclass
class OracleResult:
    rel_l2: float
    tol: float
    coverage: object = None
    independent_rel_l2: float = float("nan")
    independent_path: str = ""
    notes: list = field(default_factory=list)

    @property
    def necessary_ok(self) -> bool:
        if self.rel_l2 != self.rel_l2 or self.rel_l2 > self.tol:
            return False
        if self.coverage is not None and not self.coverage.ok:
            return False
        return True

    @property
    def sufficient_ok(self) -> bool:
        if not self.independent_path.strip():
            return False
        if self.independent_rel_l2 != self.independent_rel_l2:
            return False
        return self.independent_rel_l2 <= self.tol

    @property
    def ok(self) -> bool:
        return self.necessary_ok and self.sufficient_ok

    def render(self) -> str:
        head = "CORRECTNESS GATE: relL2 = %.3e at tolerance %.3e -- %s" % (
            self.rel_l2, self.tol, "PASSED" if self.ok else "FAILED")
        if self.coverage is not None:
            head += "\n  " + self.coverage.render()
        if self.independent_rel_l2 == self.independent_rel_l2:
            head += "\n  independent path: %.3e%s" % (
                self.independent_rel_l2,
                (" -- differs in: " + self.independent_path) if self.independent_path.strip()
                else " -- path NOT NAMED, check not counted")
        if not self.sufficient_ok:
            head += "\n  small relL2 is necessary, not sufficient: no agreeing named independent path"
        for n in self.notes:
            head += "\n  " + n
        return head


def rel_l2(got, ref) -> float:
    num = den = 0.0
    for a, b in zip(got, ref):
        d = float(a) - float(b)
        num += d * d
        den += float(b) * float(b)
    if den <= 0.0:
        return float("nan")
    return (num / den) ** 0.5


def gate(got, ref, tol: float, stamps=None, independent=None, independent_path: str = ""):
    from .coverage import check

    cov = check(stamps) if stamps is not None else None
    ind = rel_l2(got, independent) if independent is not None else float("nan")
    res = OracleResult(rel_l2=rel_l2(got, ref), tol=tol, coverage=cov, independent_rel_l2=ind,
                       independent_path=independent_path)
    if cov is not None and cov.zero:
        res.notes.append("unwritten cells under a passing value check: trust the coverage")
    return res


def speedup_vs_input(t_input_s: float, t_output_s: float) -> float:
    """Output-vs-input speedup; only ever printed next to a second bar."""
    if t_output_s <= 0:
        return float("nan")
    return t_input_s / t_output_s
