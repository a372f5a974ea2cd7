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


# ---- the contract's TensorUnit over the MFMA shapes the skeletons use -----------------------
from ..base import FragmentMap, PluginCapabilityError, TensorOp, rate  # noqa: E402


def _frag(ms: int):
    rows, cols = result_map(ms)
    orow, ogrp = operand_map(ms)

    def a(lane):  # operand A: (row, k, slot) for its 8 k-values
        return [(int(orow[lane]), 8 * int(ogrp[lane]) + e, e) for e in range(8)]

    def b(lane):  # operand B: (k, col, slot)
        return [(8 * int(ogrp[lane]) + e, int(orow[lane]), e) for e in range(8)]

    def c(lane):  # result: (row, col, register)
        return [(int(rows[lane][v]), int(cols[lane][v]), v) for v in range(rows.shape[1])]

    return FragmentMap(a=a, b=b, c=c)


OPS = (
    TensorOp(id="v_mfma_f32_32x32x16_f16", m=32, n=32, k=16, in_dtypes=("fp16", "fp16"),
             acc_dtype="fp32", frag=_frag(32),
             cost=rate("MFMA32.CYCLES", 32, "clk/instr/SIMD", "UPPER_BOUND",
                       note="32768 flop at 1024 flop/clk per SIMD"),
             operand_source="registers", loader="ds_read_b128",
             exact_while="fp32 accumulation; products of fp16 exact in fp32"),
    TensorOp(id="v_mfma_f32_16x16x32_f16", m=16, n=16, k=32, in_dtypes=("fp16", "fp16"),
             acc_dtype="fp32", frag=_frag(16),
             cost=rate("MFMA16.CYCLES", 16, "clk/instr/SIMD", "UPPER_BOUND",
                       note="16384 flop at 1024 flop/clk per SIMD"),
             operand_source="registers", loader="ds_read_b128 | global_load_dwordx4",
             exact_while="fp32 accumulation; products of fp16 exact in fp32"),
)


class Gfx950TensorUnit:
    def ops(self) -> tuple:
        return OPS

    def select(self, in_dtypes: tuple, acc_dtype: str) -> TensorOp:
        if acc_dtype != "fp32":
            raise PluginCapabilityError("gfx950 MFMA f16 ops accumulate in fp32")
        ins = tuple(in_dtypes)
        if ins in (("fp16", "fp16"), ("fp16", "int8"), ("fp16", "uint8")):
            # int8/uint8 weights are dequantised to fp16 in registers before the f16 MFMA
            return OPS[0]
        raise PluginCapabilityError("no MFMA for %r -> %s" % (ins, acc_dtype))
