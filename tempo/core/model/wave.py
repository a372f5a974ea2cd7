"""Wave and tail arithmetic (reference tempo/core/model/wave.py:22-44).  The plugin supplies the
quantum (compute units x resident workgroups per unit); useful grid sizes are multiples of it."""
from __future__ import annotations


def waves(ctas: int, quantum: int) -> float:
    return float("nan") if quantum <= 0 else ctas / float(quantum)


def efficiency(ctas: int, quantum: int) -> float:
    if quantum <= 0 or ctas <= 0:
        return 0.0
    full = -(-ctas // quantum)
    return ctas / float(quantum * full)


def tail_share(ctas: int, quantum: int) -> float:
    return 1.0 - efficiency(ctas, quantum)


def nearest_quantised(ctas: int, quantum: int) -> int:
    return ctas if quantum <= 0 else quantum * -(-ctas // quantum)
