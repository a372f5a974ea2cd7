"""GPU parity of the shipped gemm_w8a16 (both weight formats) against the CPU oracle.

Dequantisation must be bit-exact (tempo_dequant_tile runs the GEMM feeds' own device functions);
the GEMM output must match the oracle (dequantise, then the naive fp16 GEMM) within relL2 3e-3,
and bit-exactly on inputs whose arithmetic is exact.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.gpu_util import dev, host, poisoned, say

pytestmark = pytest.mark.gpu

SHAPES_NK = [(7168, 5120), (5120, 6144), (34816, 5120), (5120, 17408), (1024, 5120), (5120, 5120)]


def make_weights(N, K, fmt, seed, G=128):
    g = np.random.Generator(np.random.PCG64(seed))
    if fmt == 1:
        q = g.integers(-127, 128, (N, K), dtype=np.int16).astype(np.int8)
        s = O.f2h(g.uniform(0.5, 1.5, N).astype(np.float32) / 127)
        return q, s, None
    q = g.integers(0, 256, (N, K), dtype=np.int16).astype(np.uint8)
    s = O.f2h(g.uniform(0.5, 1.5, (N, K // G)).astype(np.float32) / 255)
    z = g.integers(100, 157, (N, K // G), dtype=np.int16).astype(np.uint8)
    return q, s, z


def _route(fmt, M, N, K):
    from cuda_tempiler_amd import capi

    return capi.route(fmt, M, N, K)


def _run(A, q, s, z, fmt, device, G=128):
    import torch
    from cuda_tempiler_amd import capi

    M, K = A.shape
    N = q.shape[0]
    dC = poisoned((M, N), device)
    capi.gemm_w8a16(dev(A, device), dev(q, device), dev(s, device),
                    dev(z, device) if z is not None else None, fmt=fmt, group=G, C=dC)
    torch.cuda.synchronize()
    return host(dC)


@pytest.mark.parametrize("fmt", [1, 2])
def test_dequant_tile_bit_exact(gpu, fmt):
    import torch
    from cuda_tempiler_amd import capi

    N, K = 512, 1024
    q, s, z = make_weights(N, K, fmt, 5)
    ref = O.dequant_sym(q, s) if fmt == 1 else O.dequant_asym(q, s, z, 128)
    dq, ds = dev(q, gpu), dev(s, gpu)
    dz = dev(z, gpu) if z is not None else None
    full = capi.dequant_tile(dq, ds, dz, fmt, 0, 0, N, K)
    torch.cuda.synchronize()
    assert np.array_equal(host(full).view(np.uint16), ref.view(np.uint16))
    part = capi.dequant_tile(dq, ds, dz, fmt, 100, 264, 37, 136)
    torch.cuda.synchronize()
    assert np.array_equal(host(part).view(np.uint16), ref[100:137, 264:400].view(np.uint16))


@pytest.mark.parametrize("fmt", [1, 2])
def test_dequant_covers_every_byte_and_zero_point(gpu, fmt):
    """All 256 weight bytes against every zero-point (fmt 2) / many scales (fmt 1)."""
    import torch
    from cuda_tempiler_amd import capi

    N, K = 256, 256
    q = np.tile(np.arange(256, dtype=np.uint8), (N, 1))
    if fmt == 1:
        q = q.view(np.int8)
        s = O.f2h(np.linspace(1e-4, 60.0, N).astype(np.float32))
        z = None
        ref = O.dequant_sym(q, s)
    else:
        s = O.f2h(np.linspace(1e-3, 3.0, N * 2).astype(np.float32).reshape(N, 2))
        z = np.repeat(np.arange(256, dtype=np.uint8)[:, None], 2, axis=1)
        ref = O.dequant_asym(q, s, z, 128)
    out = capi.dequant_tile(dev(q, gpu), dev(s, gpu), dev(z, gpu) if z is not None else None,
                            fmt, 0, 0, N, K)
    torch.cuda.synchronize()
    assert np.array_equal(host(out).view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("M", [1, 5, 8, 16, 27, 32, 128])
def test_w8a16_parity_small_m(gpu, fmt, M):
    for N, K in SHAPES_NK:
        say("w8a16 fmt", fmt, "M", M, "N", N, "K", K, "route", _route(fmt, M, N, K))
        A = O.randn_f16((M, K), 11, K ** -0.5)
        q, s, z = make_weights(N, K, fmt, 77)
        C = _run(A, q, s, z, fmt, gpu)
        assert O.count_poison(C) == 0
        ref = O.gemm_w8a16(A, q, s, z, 128, fmt)
        rel = O.rel_l2(C, ref)
        say("  relL2 %.3e" % rel)
        assert rel <= 3e-3


@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("M", [1, 16, 32])
def test_w8a16_parity_past_the_line_rows(gpu, fmt, M):
    """K > 65536 is past the line kernel's rows: the register-pipelined stream / shared rows
    (its fallbacks) run, and must hold the same bar."""
    N, K = 512, 65536 + 512
    say("w8a16 fmt", fmt, "M", M, "N", N, "K", K, "route", _route(fmt, M, N, K))
    assert not _route(fmt, M, N, K).startswith("l")
    A = O.randn_f16((M, K), 11, K ** -0.5)
    q, s, z = make_weights(N, K, fmt, 77)
    C = _run(A, q, s, z, fmt, gpu)
    assert O.count_poison(C) == 0
    rel = O.rel_l2(C, O.gemm_w8a16(A, q, s, z, 128, fmt))
    say("  relL2 %.3e" % rel)
    assert rel <= 3e-3


@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("NK", SHAPES_NK, ids=lambda nk: "n%d_k%d" % nk)
def test_w8a16_parity_prefill(gpu, fmt, NK):
    """M = 2048 (configs 3 and 4) on all six dense shapes; the whole output against the oracle."""
    N, K = NK
    M = 2048
    say("w8a16 prefill fmt", fmt, M, N, K, "route", _route(fmt, M, N, K))
    A = O.randn_f16((M, K), 11, K ** -0.5)
    q, s, z = make_weights(N, K, fmt, 77)
    C = _run(A, q, s, z, fmt, gpu)
    assert O.count_poison(C) == 0
    rel = O.rel_l2(C, O.gemm_w8a16(A, q, s, z, 128, fmt))
    say("  relL2 %.3e" % rel)
    assert rel <= 3e-3


@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("M, N, K", [(2049, 2048, 5120), (512, 5120, 17408), (2048, 2048, 5184),
                                     (2049, 1024, 5120), (300, 1792, 5120), (2049, 7168, 1024)])
def test_w8a16_parity_interleaved_prefill_rows(gpu, fmt, M, N, K):
    """The interleaved int8 prefill kernel: a ragged last tile row (M = 2049), a long k loop
    (K = 17408), and K % 128 != 0, which it does not take (fmt 1: the register-staged row runs;
    fmt 2 needs whole 128-k groups, so the shape is not covered at all).  Narrow N (< 2048)
    takes the 128 x 128 split-K row of the same kernel on 128-k tiles instead, ragged M
    included.  Wider N takes 192 x 256 tiles where one round of them holds the grid with more
    tiles than 256 x 256 ones (the FILL row: (2049, 2048), (512, 5120)), else 256 x 256 tiles
    ((2049, 7168): 308 tiles of 192 rows would need a second round)."""
    import importlib.util
    import os

    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "kernels",
                        "shipped", "gemm_w8a16", "gfx950", "select.py")
    spec = importlib.util.spec_from_file_location("select_w8_prefill_rows", path)
    sel = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(sel)
    route = _route(fmt, M, N, K)
    say("w8a16 fmt", fmt, "M", M, "N", N, "K", K, "route", route)
    if K % 128:
        assert route == ("m256x256k64" if fmt == 1 else "")
        if fmt == 2:
            return
    elif N < 2048:
        assert route == "i8x128x128w1x4k128s2w256"
    else:
        assert route == ("i8x192x256w1x4k64s3f" if sel.fill_fits(M, N, 192, 256)
                         else "i8x256w1x4k64s3t")
    A = O.randn_f16((M, K), 13, K ** -0.5)
    q, s, z = make_weights(N, K, fmt, 79)
    C = _run(A, q, s, z, fmt, gpu)
    assert O.count_poison(C) == 0
    rows = np.r_[0:32, M // 2:M // 2 + 32, M - 32:M]
    rel = O.rel_l2(np.ascontiguousarray(C[rows]), O.gemm_w8a16(A[rows], q, s, z, 128, fmt))
    say("  relL2 %.3e" % rel)
    assert rel <= 3e-3


@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("M", [1, 8, 16, 32, 300])
@pytest.mark.parametrize("N", [1024, 17408])
def test_w8a16_exact_regime_bit_exact(gpu, fmt, M, N):
    """Scales that are powers of two and activations on a 1/8 grid make every product and
    partial sum exact in fp32, so the result is order-independent: bits must equal the oracle.
    N = 17408 reaches the wide-N ladder rows (shared activations, k-chunk reduction)."""
    K = 2048
    say("exact regime fmt", fmt, "M", M, "N", N, "route", _route(fmt, M, N, K))
    g = np.random.Generator(np.random.PCG64(31))
    A = (g.integers(-4, 5, (M, K)).astype(np.float32) / 8).astype(np.float16)
    if fmt == 1:
        q = g.integers(-127, 128, (N, K), dtype=np.int16).astype(np.int8)
        s = np.full(N, np.float16(2.0 ** -7))
        z = None
    else:
        q = g.integers(0, 256, (N, K), dtype=np.int16).astype(np.uint8)
        s = np.full((N, K // 128), np.float16(2.0 ** -8))
        z = g.integers(100, 157, (N, K // 128), dtype=np.int16).astype(np.uint8)
    C = _run(A, q, s, z, fmt, gpu)
    ref = O.gemm_w8a16(A, q, s, z, 128, fmt)
    assert np.array_equal(C.view(np.uint16), ref.view(np.uint16))


def _gptq_checkpoint(K, N, G, seed):
    """GPTQ int8 tensors over the full int32 range (bench/gemm_baseline.py:219-223)."""
    g = np.random.Generator(np.random.PCG64(seed))
    qw = g.integers(-(2**31), 2**31 - 1, (K // 4, N), dtype=np.int64).astype(np.int32)
    qz = g.integers(-(2**31), 2**31 - 1, (K // G, N // 4), dtype=np.int64).astype(np.int32)
    sc = O.f2h(g.uniform(0.001, 0.021, (K // G, N)).astype(np.float32))
    return qw, qz, sc


@pytest.mark.parametrize("KN", [(128, 64), (256, 192), (5120, 6144), (5120, 34816), (17408, 5120)],
                         ids=lambda kn: "k%d_n%d" % kn)
def test_gptq_repack_bit_exact(gpu, KN):
    """The device repack of a GPTQ checkpoint equals the oracle's byte for byte (weights, scales
    and zero-points), at the model's full layer shapes included."""
    import torch
    from cuda_tempiler_amd import capi

    K, N = KN
    say("gptq repack", KN)
    qw, qz, sc = _gptq_checkpoint(K, N, 128, K + N)
    wq, s, z = capi.gptq_repack(dev(qw, gpu), dev(qz, gpu), dev(sc, gpu))
    torch.cuda.synchronize()
    rw, rs, rz = O.gptq_to_nk(qw, qz, sc)
    assert np.array_equal(host(wq), rw)
    assert np.array_equal(host(s).view(np.uint16), rs.view(np.uint16))
    assert np.array_equal(host(z), rz)


@pytest.mark.parametrize("M", [1, 16, 200])
def test_gptq_checkpoint_to_gemm(gpu, M):
    """GPTQ checkpoint -> device repack -> fmt 2 GEMM: matches the oracle built on the reference's
    dense formula (gemm_baseline.py:229) within relL2 3e-3, and bit-for-bit the same GEMM fed
    with the oracle's repack."""
    import torch
    from cuda_tempiler_amd import capi

    K, N = 5120, 6144
    say("gptq gemm M=%d" % M, _route(2, M, N, K))
    qw, qz, sc = _gptq_checkpoint(K, N, 128, 77)
    wq, s, z = capi.gptq_repack(dev(qw, gpu), dev(qz, gpu), dev(sc, gpu))
    g = np.random.Generator(np.random.PCG64(M))
    A = O.f2h(g.standard_normal((M, K), dtype=np.float32))
    dA = dev(A, gpu)
    C = capi.gemm_w8a16(dA, wq, s, z, fmt=2, group=128, C=poisoned((M, N), gpu))
    rw, rs, rz = O.gptq_to_nk(qw, qz, sc)
    C2 = capi.gemm_w8a16(dA, dev(rw, gpu), dev(rs, gpu), dev(rz, gpu), fmt=2, group=128,
                         C=poisoned((M, N), gpu))
    torch.cuda.synchronize()
    got = host(C)
    assert O.count_poison(got) == 0
    assert np.array_equal(got.view(np.uint16), host(C2).view(np.uint16))
    W = O.gptq_dense(qw, qz, sc)
    ref = O.gemm_f16(A, np.ascontiguousarray(W.T))
    r = O.rel_l2(got, ref)
    say("  relL2 %.3e" % r)
    assert r <= 3e-3


@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("shape", [(1, 64, 128), (7, 200, 384), (33, 1024, 1280)],
                         ids=lambda s: "m%d_n%d_k%d" % s)
def test_naive_w8a16_input_is_the_oracle(gpu, fmt, shape):
    """The naive W8A16 input kernel (kernels/naive/gemm_w8a16.hip, the "vs input" bar of the
    pipeline) is bit-exact against the oracle: same dequantisation, same sequential fp32 FMA."""
    import torch
    from cuda_tempiler_amd import capi

    M, N, K = shape
    say("naive w8a16", fmt, shape)
    q, s, z = make_weights(N, K, fmt, seed=M + N + fmt)
    g = np.random.Generator(np.random.PCG64(M))
    A = O.f2h(g.standard_normal((M, K), dtype=np.float32))
    C = capi.naive_gemm_w8a16(dev(A, gpu), dev(q, gpu), dev(s, gpu),
                              dev(z, gpu) if z is not None else None, fmt=fmt, group=128,
                              C=poisoned((M, N), gpu))
    torch.cuda.synchronize()
    ref = O.gemm_w8a16(A, q, s, z, 128, fmt)
    assert np.array_equal(host(C).view(np.uint16), ref.view(np.uint16))
