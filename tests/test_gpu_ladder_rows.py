"""GPU parity of every row of the shipped ladders (cases in tests/ladder_cases.py, whose coverage
of the ladders tests/test_ladder_coverage.py checks on the CPU).

Each case: the compiled dispatcher must route it to the row the case names; every output cell
must be written (0x7f7f poison gone, reference harness.cu:50-57); the whole output must match the
oracle within relL2 3e-3 (the north star's bar for fp16 outputs), and fp16 GEMM cases also pass
the reference's fp64 spot rule on 256 sampled cells (ship_probe.cu:70-79).
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests import ladder_cases as LC
from tests.gpu_util import dev, host, poisoned, say

pytestmark = pytest.mark.gpu
TOL = 3e-3


def _weights(N, K, fmt, seed, G=128):
    g = np.random.Generator(np.random.PCG64(seed))
    if fmt == 1:
        q = g.integers(-127, 128, (N, K), dtype=np.int16).astype(np.int8)
        s = O.f2h(g.uniform(0.5, 1.5, N).astype(np.float32) / 127)
        return q, s, None
    q = g.integers(0, 256, (N, K), dtype=np.int16).astype(np.uint8)
    s = O.f2h(g.uniform(0.5, 1.5, (N, K // G)).astype(np.float32) / 255)
    z = g.integers(100, 157, (N, K // G), dtype=np.int16).astype(np.uint8)
    return q, s, z


def _check(got, ref, what):
    assert O.count_poison(got) == 0, what + ": unwritten cells"
    r = O.rel_l2(got, ref)
    say("  relL2 %.3e" % r)
    assert r <= TOL, what


@pytest.mark.parametrize("case", LC.FP16, ids=LC.case_id)
def test_fp16_row(gpu, case):
    import torch
    from cuda_tempiler_amd import capi

    tag, M, N, K = case
    route = capi.route(0, M, N, K)
    say("fp16 row", tag, "M", M, "N", N, "K", K, "route", route)
    assert route == tag
    A = O.randn_f16((M, K), 11 + M, K ** -0.5)
    B = O.randn_f16((N, K), 77 + N, K ** -0.5)
    C = poisoned((M, N), gpu)
    capi.gemm_fp16(dev(A, gpu), dev(B, gpu), C)
    torch.cuda.synchronize()
    got = host(C)
    _check(got, O.gemm_f16(A, B), tag)
    worst, bad = O.spot_fp64(A, B, got, cells=256)
    assert bad == 0, "fp64 spot %.3e" % worst


@pytest.mark.parametrize("case", LC.FP16_STRIDED, ids=LC.case_id)
def test_fp16_row_strided(gpu, case):
    """lda > K, ldb > K, ldc > N (views into wider buffers); ldc = N + 4 leaves every other C row
    8-byte but not 16-byte aligned.  The padding columns of C must stay untouched."""
    import torch
    from cuda_tempiler_amd import capi

    tag, M, N, K, pa, pb, pc = case
    say("fp16 strided row", tag, "M", M, "N", N, "K", K, "pads", pa, pb, pc)
    assert capi.route(0, M, N, K) == tag
    A = O.randn_f16((M, K), 5, K ** -0.5)
    B = O.randn_f16((N, K), 6, K ** -0.5)
    Aw = np.zeros((M, K + pa), np.float16)
    Aw[:, :K] = A
    Bw = np.zeros((N, K + pb), np.float16)
    Bw[:, :K] = B
    dA, dB = dev(Aw, gpu)[:, :K], dev(Bw, gpu)[:, :K]
    Cw = poisoned((M, N + pc), gpu)
    dC = Cw[:, :N]
    assert dA.stride(0) == K + pa and dB.stride(0) == K + pb and dC.stride(0) == N + pc
    capi.gemm_fp16(dA, dB, dC)
    torch.cuda.synchronize()
    full = host(Cw)
    assert O.count_poison(full[:, N:]) == full[:, N:].size, "padding columns written"
    _check(np.ascontiguousarray(full[:, :N]), O.gemm_f16(A, B), tag)


@pytest.mark.parametrize("case", LC.FP16_GATE_UP, ids=LC.case_id)
def test_fp16_gate_up_row(gpu, case):
    import torch
    from cuda_tempiler_amd import capi

    tag, M, N, K = case
    route = capi.route(3, M, N, K)
    say("fp16 gate_up row", tag, "M", M, "N", N, "K", K, "route", route)
    assert route == tag
    A = O.randn_f16((M, K), 3 + M, 1.0)
    B = O.randn_f16((2 * N, K), 4 + N, 2 * K ** -0.5)
    C = capi.gemm_fp16_gate_up(dev(A, gpu), dev(B, gpu), C=poisoned((M, N), gpu))
    torch.cuda.synchronize()
    _check(host(C), O.gemm_gate_up_f16(A, B), tag)


@pytest.mark.parametrize("fmt,case", [(f, c) for f in (1, 2) for c in LC.W8[f]],
                         ids=lambda v: v if isinstance(v, int) else LC.case_id(v))
def test_w8a16_row(gpu, fmt, case):
    import torch
    from cuda_tempiler_amd import capi

    tag, M, N, K = case
    route = capi.route(fmt, M, N, K)
    say("w8a16 fmt", fmt, "row", tag, "M", M, "N", N, "K", K, "route", route)
    assert route == tag
    A = O.randn_f16((M, K), 11 + M, K ** -0.5)
    q, s, z = _weights(N, K, fmt, 77 + N)
    C = poisoned((M, N), gpu)
    capi.gemm_w8a16(dev(A, gpu), dev(q, gpu), dev(s, gpu), dev(z, gpu) if z is not None else None,
                    fmt=fmt, group=128, C=C)
    torch.cuda.synchronize()
    _check(host(C), O.gemm_w8a16(A, q, s, z, 128, fmt), tag)


@pytest.mark.parametrize("fmt,case", [(f, c) for f in (1, 2) for c in LC.W8_GATE_UP[f]],
                         ids=lambda v: v if isinstance(v, int) else LC.case_id(v))
def test_w8a16_gate_up_row(gpu, fmt, case):
    import torch
    from cuda_tempiler_amd import capi

    tag, M, N, K = case
    route = capi.route(3 + fmt, M, N, K)
    say("w8a16 gate_up fmt", fmt, "row", tag, "M", M, "N", N, "K", K, "route", route)
    assert route == tag
    A = O.randn_f16((M, K), 3 + M, 3 * K ** -0.5)
    q, s, z = _weights(2 * N, K, fmt, 9 + N)
    s = O.f2h(O.h2f(s) * 2)
    C = capi.gemm_w8a16_gate_up(dev(A, gpu), dev(q, gpu), dev(s, gpu),
                                dev(z, gpu) if z is not None else None, fmt=fmt, group=128,
                                C=poisoned((M, N), gpu))
    torch.cuda.synchronize()
    _check(host(C), O.gemm_gate_up_w8a16(A, q, s, z, 128, fmt), tag)


def _strided_w8(gpu, A, q, s, z, M, N, K, pa, pb, pc):
    """A, q as views into buffers pa / pb wider, C a view pc columns narrower than its buffer."""
    Aw = np.zeros((M, K + pa), np.float16)
    Aw[:, :K] = A
    qw = np.zeros((q.shape[0], K + pb), q.dtype)
    qw[:, :K] = q
    dA, dq = dev(Aw, gpu)[:, :K], dev(qw, gpu)[:, :K]
    Cw = poisoned((M, N + pc), gpu)
    dC = Cw[:, :N]
    assert dA.stride(0) == K + pa and dq.stride(0) == K + pb and dC.stride(0) == N + pc
    return dA, dq, dev(s, gpu), (dev(z, gpu) if z is not None else None), Cw, dC


@pytest.mark.parametrize("fmt,case", [(f, c) for f in (1, 2) for c in LC.W8_STRIDED[f]],
                         ids=lambda v: v if isinstance(v, int) else LC.case_id(v))
def test_w8a16_row_strided(gpu, fmt, case):
    """lda > K, ldw > K, ldc > N; the padding columns of C must stay untouched."""
    import torch
    from cuda_tempiler_amd import capi

    tag, M, N, K, pa, pb, pc = case
    say("w8a16 fmt", fmt, "strided row", tag, "M", M, "N", N, "K", K, "pads", pa, pb, pc)
    assert capi.route(fmt, M, N, K) == tag
    A = O.randn_f16((M, K), 5 + M, K ** -0.5)
    q, s, z = _weights(N, K, fmt, 31 + N)
    dA, dq, ds, dz, Cw, dC = _strided_w8(gpu, A, q, s, z, M, N, K, pa, pb, pc)
    capi.gemm_w8a16(dA, dq, ds, dz, fmt=fmt, group=128, C=dC)
    torch.cuda.synchronize()
    full = host(Cw)
    assert O.count_poison(full[:, N:]) == full[:, N:].size, "padding columns written"
    _check(np.ascontiguousarray(full[:, :N]), O.gemm_w8a16(A, q, s, z, 128, fmt), tag)


@pytest.mark.parametrize("fmt,case", [(f, c) for f in (1, 2) for c in LC.W8_GATE_UP_STRIDED[f]],
                         ids=lambda v: v if isinstance(v, int) else LC.case_id(v))
def test_w8a16_gate_up_row_strided(gpu, fmt, case):
    """The fused gate/up on views into wider buffers (2N weight rows of ldw > K)."""
    import torch
    from cuda_tempiler_amd import capi

    tag, M, N, K, pa, pb, pc = case
    say("w8a16 gate_up fmt", fmt, "strided row", tag, "M", M, "N", N, "K", K, "pads", pa, pb, pc)
    assert capi.route(3 + fmt, M, N, K) == tag
    A = O.randn_f16((M, K), 7 + M, 3 * K ** -0.5)
    q, s, z = _weights(2 * N, K, fmt, 13 + N)
    s = O.f2h(O.h2f(s) * 2)
    dA, dq, ds, dz, Cw, dC = _strided_w8(gpu, A, q, s, z, M, N, K, pa, pb, pc)
    capi.gemm_w8a16_gate_up(dA, dq, ds, dz, fmt=fmt, group=128, C=dC)
    torch.cuda.synchronize()
    full = host(Cw)
    assert O.count_poison(full[:, N:]) == full[:, N:].size, "padding columns written"
    _check(np.ascontiguousarray(full[:, :N]), O.gemm_gate_up_w8a16(A, q, s, z, 128, fmt), tag)
