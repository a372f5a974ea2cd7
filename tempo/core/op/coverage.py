"""Coverage stamp: every output cell written exactly once (reference tempo/core/op/coverage.py).

Value checks only look at what was computed; a kernel that skips a quarter of the tile passes
them.  The stamp (or, on the shipped path, the 0x7f7f poison fill) catches cells written zero
times or more than once."""
from __future__ import annotations

from dataclasses import dataclass

STAMP_MACRO = "TEMPO_COVERAGE_STAMP"


@dataclass
class Coverage:
    total: int
    zero: int
    over: int
    max_hits: int

    @property
    def ok(self) -> bool:
        return self.zero == 0 and self.over == 0

    def render(self) -> str:
        if self.ok:
            return "coverage complete: %d cells, each written once" % self.total
        return ("coverage BROKEN: %d cells unwritten, %d written more than once (max %d) of %d"
                % (self.zero, self.over, self.max_hits, self.total))


def check(stamps) -> Coverage:
    total = zero = over = mx = 0
    for v in stamps:
        total += 1
        v = int(v)
        if v == 0:
            zero += 1
        elif v > 1:
            over += 1
        mx = max(mx, v)
    return Coverage(total=total, zero=zero, over=over, max_hits=mx)


def from_poison(cells_bits, poison: int = 0x7F7F) -> Coverage:
    """Shipped-path form: a cell still holding the poison pattern was never written."""
    total = zero = 0
    for v in cells_bits:
        total += 1
        zero += int(v) == poison
    return Coverage(total=total, zero=zero, over=0, max_hits=1 if total > zero else 0)
