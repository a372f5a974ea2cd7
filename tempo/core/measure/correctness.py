"""The gate comes before the stopwatch (reference tempo/core/measure/correctness.py:21-39)."""
from __future__ import annotations

from tempo.core.op.coverage import check as coverage_check  # noqa: F401
from tempo.core.op.oracle import OracleResult, gate, rel_l2  # noqa: F401

ORDER = (
    "1. build the variant",
    "2. check COVERAGE (poison / stamp): catches skipped cells a value check misses",
    "3. check VALUES against a reference of at least single precision",
    "4. break the symmetry: an independent path differing in one NAMED node",
    "5. only now: the stopwatch",
)


def must_pass_before_timing(res: OracleResult) -> None:
    if not res.ok:
        raise AssertionError("stopwatch FORBIDDEN: the correctness gate did not pass.\n" + res.render())
