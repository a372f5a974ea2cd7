"""Median of paired ratios (reference tempo/core/measure/ratio.py:63-73).  Arms are measured in
alternation within a round; the median of per-round ratios cancels clock drift that a ratio of
medians would keep."""
from __future__ import annotations

DISCIPLINE = (
    "correctness gate before the stopwatch",
    "paired ratios, arms alternating within a round",
    "median of ratios, not ratio of medians",
    "clock and foreign GPU processes recorded before and after",
    "entry proven (route tag or bitwise diff)",
)


def median_ratio(pairs):
    vals = sorted(float(a) / float(b) for a, b in pairs if b)
    if not vals:
        return float("nan")
    n = len(vals)
    return vals[n // 2] if n % 2 else 0.5 * (vals[n // 2 - 1] + vals[n // 2])
