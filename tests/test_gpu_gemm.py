"""GPU parity of the shipped gemm_fp16 (through the C ABI) against the CPU oracle.

Gates, in the reference's order (tempo/core/measure/correctness.py:21-27): coverage (0x7f7f
poison must be gone from every cell), values (relL2 against the naive kernel's arithmetic,
3e-3), an independent fp64 spot check on sampled cells, and -- where the arithmetic is exact --
bit equality with known answers.
"""
import json
import os

import numpy as np
import pytest

from oracle import oracle as O
from tests.gpu_util import dev, host, poisoned, say

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden", "ship_probe_cells.json")


def _run(A, B, device):
    import torch
    from cuda_tempiler_amd import capi

    M, K = A.shape
    N = B.shape[0]
    dA, dB = dev(A, device), dev(B, device)
    dC = poisoned((M, N), device)
    capi.gemm_fp16(dA, dB, dC)
    torch.cuda.synchronize()
    return host(dC)


@pytest.mark.parametrize("ms", [32, 16])
def test_mfma_result_layout_probe(gpu, ms):
    """The result map the epilogues assume (cdna4.h) is what the matrix core produces."""
    from cuda_tempiler_amd import capi
    from tempo.plugins.gfx950 import tensor

    rows, cols = capi.probe_mfma_layout(ms)
    nacc = rows.shape[1]
    exp_r, exp_c = tensor.result_map(ms)
    assert np.array_equal(rows, exp_r) and np.array_equal(cols, exp_c)
    cells = {(int(r), int(c)) for r, c in zip(rows.ravel(), cols.ravel())}
    assert len(cells) == 64 * nacc == ms * ms  # a bijection onto the ms x ms tile


def test_naive_hip_bit_exact_with_oracle(gpu):
    import torch
    from cuda_tempiler_amd import capi

    A = O.randn_f16((67, 320), 1, 320 ** -0.5)
    B = O.randn_f16((129, 320), 2, 320 ** -0.5)
    dC = poisoned((67, 129), gpu)
    capi.naive_gemm_fp16(dev(A, gpu), dev(B, gpu), dC)
    torch.cuda.synchronize()
    assert np.array_equal(host(dC).view(np.uint16), O.gemm_f16(A, B).view(np.uint16))


def test_shipped_known_answers_bit_exact(gpu):
    """ship_probe.cu's six shapes and 64 cells: exact arithmetic, so bits must match."""
    gold = json.load(open(GOLD))
    for sh in gold["shapes"]:
        M, N, K = sh["M"], sh["N"], sh["K"]
        say("known-answer", M, N, K)
        A, B = O.ship_probe_inputs(M, N, K)
        C = _run(A, B, gpu)
        assert O.count_poison(C) == 0, (M, N, K)
        for m, n, S, bits in sh["cells"]:
            assert int(C.view(np.uint16)[m, n]) == bits, (M, N, K, m, n)


# one shape per ladder row at least (route named in the test id), plus ragged M and a shape whose
# first matching row does not fit (N = 12304: N % 64 != 0, falls through to the next row)
SHAPES = [(1, 15360, 3840), (1, 3840, 15360), (8, 15360, 3840), (8, 12304, 3840),
          (16, 3840, 15360), (17, 4096, 3840), (24, 15360, 3840), (32, 3840, 15360),
          (64, 15360, 3840), (96, 15360, 3840), (128, 3840, 15360), (200, 4096, 3840),
          (256, 15360, 3840),
          (256, 3840, 15360), (256, 8192, 3840),
          (512, 4096, 3840), (300, 15360, 3840), (1000, 4096, 3840), (2049, 3840, 15360),
          # K > 65536: past the line rows, the stream rows run
          (1, 512, 66048), (16, 512, 66048), (32, 512, 66048)]


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_gemm_fp16_parity(gpu, M, N, K):
    say("parity", M, N, K)
    A = O.randn_f16((M, K), 11, K ** -0.5)
    B = O.randn_f16((N, K), 77, K ** -0.5)
    C = _run(A, B, gpu)
    assert O.count_poison(C) == 0
    ref = O.gemm_f16(A, B)
    rel = O.rel_l2(C, ref)
    worst, bad = O.spot_fp64(A, B, C, cells=256)
    say("  relL2 %.3e spot %.3e" % (rel, worst))
    assert rel <= 3e-3 and bad == 0


# BASELINE config 2, every point of the decode sweep: (N, K) in {(15360, 3840), (3840, 15360)} x
# M in {1, 8, 16, 32, 64, 128, 256}
C2_SWEEP = [(M, N, K) for (N, K) in ((15360, 3840), (3840, 15360))
            for M in (1, 8, 16, 32, 64, 128, 256)]


@pytest.mark.parametrize("M,N,K", C2_SWEEP)
def test_gemm_fp16_parity_config2_sweep(gpu, M, N, K):
    """Each C2 point in full: coverage of every cell, the whole output and its worst row against
    the oracle, and the fp64 spot rule on 512 cells; the test id carries the shape and the log the
    ladder row the compiled dispatcher took."""
    from cuda_tempiler_amd import capi

    say("config2", M, N, K, capi.route(0, M, N, K))
    A = O.randn_f16((M, K), 11, K ** -0.5)
    B = O.randn_f16((N, K), 77, K ** -0.5)
    C = _run(A, B, gpu)
    assert O.count_poison(C) == 0
    ref = O.gemm_f16(A, B)
    rel = O.rel_l2(C, ref)
    d = C.astype(np.float64) - ref.astype(np.float64)
    row_rel = np.sqrt((d * d).sum(1) / np.maximum((ref.astype(np.float64) ** 2).sum(1), 1e-30))
    worst, bad = O.spot_fp64(A, B, C, cells=512)
    say("  relL2 %.3e worst row %.3e spot %.3e" % (rel, row_rel.max(), worst))
    assert rel <= 3e-3 and row_rel.max() <= 3e-3 and bad == 0


def test_gemm_fp16_parity_config1(gpu):
    """BASELINE config 1 at full size: 4096 x 15360 x 3840.  Coverage over every cell; the WHOLE
    output against the oracle (relL2), fp64 on 2048 cells, and the worst row's relL2 so a
    localised error (one bad tile) cannot hide in the global norm."""
    M, N, K = 4096, 15360, 3840
    say("config1", M, N, K)
    A = O.randn_f16((M, K), 11, K ** -0.5)
    B = O.randn_f16((N, K), 77, K ** -0.5)
    C = _run(A, B, gpu)
    assert O.count_poison(C) == 0
    ref = O.gemm_f16(A, B)
    rel = O.rel_l2(C, ref)
    d = C.astype(np.float64) - ref.astype(np.float64)
    row_rel = np.sqrt((d * d).sum(1) / np.maximum((ref.astype(np.float64) ** 2).sum(1), 1e-30))
    worst, bad = O.spot_fp64(A, B, C, cells=2048)
    say("  relL2 %.3e worst row %.3e spot %.3e" % (rel, row_rel.max(), worst))
    assert rel <= 3e-3 and row_rel.max() <= 3e-3 and bad == 0


def test_not_covered_returns_fallback(gpu):
    import torch
    from cuda_tempiler_amd import capi

    A = torch.zeros((4, 100), dtype=torch.float16, device=gpu)   # K % 8 != 0
    B = torch.zeros((64, 100), dtype=torch.float16, device=gpu)
    with pytest.raises(capi.NotCovered):
        capi.gemm_fp16(A, B)
