"""gfx950: TENSOR UNIT -- section 3 of the contract (tempo/plugins/base.py TensorUnit, TensorOp,
FragmentMap; reference pattern tempo/plugins/sm70/tensor.py).

The matrix-core instructions the skeletons use, with their fragment maps written as data: lane ->
[(row, col, slot)] for the A operand, the B operand and the result.  The result map is what the
epilogues depend on; tests/test_gpu_gemm.py measures it on the GPU (tempo_probe_mfma_layout) and
compares it with result_map() below, and checks it is a bijection onto the tile.
"""
from __future__ import annotations

import numpy as np

WAVE = 64


def result_map(ms: int):
    """(rows, cols) int arrays [64][nacc]: where result register v of lane l sits in the tile.

    32x32x16: column l % 32, rows 8*(v//4) + 4*(l//32) + v%4 (16 registers)
    16x16x32: column l % 16, rows 4*(l//16) + v                (4 registers)
    """
    if ms == 32:
        nacc, gstride = 16, 8
    elif ms == 16:
        nacc, gstride = 4, 16
    else:
        raise ValueError("MFMA shape %r" % ms)
    lanes = np.arange(WAVE)[:, None]
    v = np.arange(nacc)[None, :]
    rows = (v // 4) * gstride + 4 * (lanes // ms) + (v % 4)
    cols = np.broadcast_to(lanes % ms, (WAVE, nacc))
    return rows.astype(int), cols.astype(int).copy()


def operand_map(ms: int):
    """lane -> (row, k-group): operand lane l carries row l % ms and the 8 k-values of group
    l // ms (the same map for both operands; the k order within a group is immaterial as long
    as both operands agree)."""
    lanes = np.arange(WAVE)
    return lanes % ms, lanes // ms
