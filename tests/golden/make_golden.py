"""Writes tests/golden/ship_probe_cells.json -- known-answer vectors for gemm_fp16.

Inputs are the reference's ship-probe fill (kernels/shipped/gemm_fp16/sm_70/ship_probe.cu:54-55):
    A[i] = ((i % 7) - 3) / 8,   B[i] = ((i % 5) - 2) / 8     (flat row-major index i)
on its six serving shapes (ship_probe.cu:41-45), sampled at its 64 cells m = (t*37) % M,
n = (t*53) % N (ship_probe.cu:70-71).

Every product is a multiple of 1/64 and every partial sum stays below 2^24 / 64, so fp32
accumulation is exact in ANY order and the fp16 output is a closed form: the integer sum
S = sum_k ((m*K+k)%7-3)((n*K+k)%5-2), divided by 64, rounded once to fp16.  The sum is computed
here with exact integers (no floating point), so the expected bits do not depend on any code
under test.  Any correct kernel -- the CPU oracle, the naive HIP kernel, every MFMA tile --
must reproduce these bits exactly.

    python3 tests/golden/make_golden.py
"""
import json
import os

import numpy as np

SHAPES = [(1, 4096, 3840, "q"), (8, 4096, 3840, "q"), (32, 15360, 3840, "gate,up"),
          (128, 4096, 3840, "q"), (512, 15360, 3840, "gate,up"), (2048, 3840, 15360, "down")]
CELLS = 64


def exact_cell(m, n, K):
    k = np.arange(K, dtype=np.int64)
    a = ((m * K + k) % 7) - 3
    b = ((n * K + k) % 5) - 2
    return int(np.sum(a * b))  # exact integer; value = S / 64


def main():
    out = []
    for M, N, K, role in SHAPES:
        cells = []
        for t in range(CELLS):
            m, n = (t * 37) % M, (t * 53) % N
            S = exact_cell(m, n, K)
            assert abs(S) < (1 << 24)
            bits = int(np.array([S / 64.0], dtype=np.float64).astype(np.float16).view(np.uint16)[0])
            cells.append([m, n, S, bits])
        out.append({"M": M, "N": N, "K": K, "role": role, "cells": cells})
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ship_probe_cells.json")
    with open(path, "w") as f:
        json.dump({"source": "ship_probe.cu:41-79 inputs, exact integer sums",
                   "cell": "[m, n, S (value = S/64), expected fp16 bits]", "shapes": out}, f)
    print(path)


if __name__ == "__main__":
    main()
