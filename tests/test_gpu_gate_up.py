"""GPU parity of the fused gate/up epilogue (C = silu(A.B[:N]^T) * (A.B[N:]^T), B [2N, K]) of both
shipped deliveries against the CPU oracle.

fp16 output: relL2 <= 3e-3 against the oracle's fp64 silu on the fp16-rounded gate and up
results.  On inputs whose products are exact (small integers) the gate and up results are exact
too, so the fused output differs from the oracle only by the hardware exponential: at most one
fp16 unit in the last place.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.gpu_util import dev, host, poisoned, say

pytestmark = pytest.mark.gpu
TOL = 3e-3


def _route(op, M, N, K):
    from cuda_tempiler_amd import capi

    return capi.route(op, M, N, K)


@pytest.mark.parametrize("M", [1, 5, 16, 27, 32, 33, 128, 300])
@pytest.mark.parametrize("NK", [(17408, 5120), (1024, 3840)], ids=lambda nk: "n%d_k%d" % nk)
def test_fp16_gate_up_parity(gpu, M, NK):
    import torch
    from cuda_tempiler_amd import capi

    N, K = NK
    say("fp16 gate_up M=%d N=%d K=%d" % (M, N, K), _route(3, M, N, K))
    g = np.random.Generator(np.random.PCG64(M * 7 + N))
    A = O.f2h(g.standard_normal((M, K), dtype=np.float32))
    B = O.f2h(g.standard_normal((2 * N, K), dtype=np.float32) / np.float32(np.sqrt(K)) * 2)
    C = capi.gemm_fp16_gate_up(dev(A, gpu), dev(B, gpu), C=poisoned((M, N), gpu))
    torch.cuda.synchronize()
    got = host(C)
    assert O.count_poison(got) == 0
    ref = O.gemm_gate_up_f16(A, B)
    r = O.rel_l2(got, ref)
    say("  relL2 %.3e" % r)
    assert r <= TOL


@pytest.mark.parametrize("M", [1, 16, 32, 64, 257])
def test_fp16_gate_up_exact_regime(gpu, M):
    """Small-integer inputs: every gate and up sum is exact, so only the exponential differs."""
    import torch
    from cuda_tempiler_amd import capi

    N, K = 2048, 1024
    g = np.random.Generator(np.random.PCG64(M))
    A = (g.integers(-2, 3, (M, K)) / 4).astype(np.float16)
    B = (g.integers(-2, 3, (2 * N, K)) / 8).astype(np.float16)
    C = capi.gemm_fp16_gate_up(dev(A, gpu), dev(B, gpu))
    torch.cuda.synchronize()
    got = host(C)
    ref = O.gemm_gate_up_f16(A, B)
    d = np.abs(got.view(np.int16).astype(np.int32) - ref.view(np.int16).astype(np.int32))
    say("gate_up exact regime M=%d: max ulp %d, exact %.4f" % (M, d.max(), (d == 0).mean()))
    assert d.max() <= 1


@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("M", [1, 8, 16, 32, 64, 300])
def test_w8a16_gate_up_parity(gpu, fmt, M):
    """The production shape S1 (bench/shapes/qwen36_27b_int8.json): gate_up with 2N = 34816."""
    import torch
    from cuda_tempiler_amd import capi

    N, K = 17408, 5120
    say("w8a16 gate_up fmt=%d M=%d" % (fmt, M), _route(3 + fmt, M, N, K))
    g = np.random.Generator(np.random.PCG64(fmt * 100 + M))
    if fmt == 1:
        q = g.integers(-127, 128, (2 * N, K), dtype=np.int16).astype(np.int8)
        s = O.f2h(g.uniform(0.5, 1.5, 2 * N).astype(np.float32) / 127 * 2)
        z = None
    else:
        q = g.integers(0, 256, (2 * N, K), dtype=np.int16).astype(np.uint8)
        s = O.f2h(g.uniform(0.5, 1.5, (2 * N, K // 128)).astype(np.float32) / 255 * 2)
        z = g.integers(100, 157, (2 * N, K // 128), dtype=np.int16).astype(np.uint8)
    A = O.f2h((g.standard_normal((M, K), dtype=np.float32) / np.float32(np.sqrt(K) / 3)))
    C = capi.gemm_w8a16_gate_up(dev(A, gpu), dev(q, gpu), dev(s, gpu),
                                dev(z, gpu) if z is not None else None, fmt=fmt, group=128,
                                C=poisoned((M, N), gpu))
    torch.cuda.synchronize()
    got = host(C)
    assert O.count_poison(got) == 0
    ref = O.gemm_gate_up_w8a16(A, q, s, z, 128, fmt)
    r = O.rel_l2(got, ref)
    say("  relL2 %.3e" % r)
    assert r <= TOL


def test_gate_up_uncovered_shape_is_refused(gpu):
    """N % 128 != 0 past the decode band: no row fits, the caller's own path (TEMPO_FALLBACK)."""
    from cuda_tempiler_amd import capi

    A = dev(np.zeros((64, 512), np.float16), gpu)
    B = dev(np.zeros((2 * 1000, 512), np.float16), gpu)
    with pytest.raises(capi.NotCovered):
        capi.gemm_fp16_gate_up(A, B)
