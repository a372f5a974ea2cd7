"""A comparison bar is an object with a kind (reference tempo/core/measure/baseline.py:69-81)."""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

KINDS = ("INPUT", "LIBRARY", "SHIPPED", "FORMAT")


@dataclass(frozen=True)
class Baseline:
    kind: str
    name: str
    what: str
    entry_proof: Optional[str] = None

    def __post_init__(self):
        if self.kind not in KINDS:
            raise ValueError("bar kind %r not in %r" % (self.kind, KINDS))

    def label(self) -> str:
        return "%s (%s)" % (self.name, self.kind)


@dataclass(frozen=True)
class Comparison:
    baseline: Baseline
    ratio: float
    ci: tuple = ()
    rounds: int = 0
    note: str = ""

    def render(self) -> str:
        ci = " [%.3f..%.3f]" % self.ci if self.ci and len(self.ci) == 2 else ""
        return "vs %-28s x%.3f%s  rounds %d%s" % (self.baseline.label(), self.ratio, ci,
                                                 self.rounds, ("  -- " + self.note) if self.note else "")


def two_bars_required(comps) -> None:
    kinds = {c.baseline.kind for c in comps}
    if "INPUT" not in kinds:
        raise ValueError("no INPUT bar: unknown whether the product made the result")
    if not kinds & {"LIBRARY", "SHIPPED", "FORMAT"}:
        raise ValueError("no SECOND bar: beating the naive input alone proves nothing")
