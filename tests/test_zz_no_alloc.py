"""The allocation-free W8A16 entry point (tempo_gemm_w8a16_launch_noalloc) against the allocating
one (tempo_gemm_w8a16_launch), through the C ABI.

Both run the same ladder rows and kernels; only where a split-K row's workspace comes from
differs (a static per-GPU scratch array instead of the per-stream pool), and the split-K sum is
taken in a fixed order, so the outputs must agree bit for bit -- and match the oracle within the
north star's relL2 3e-3.  Two calls in a row on the same scratch, the second with a smaller
shape, show that what the first call left in the scratch does not leak into the second.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.gpu_util import dev, host, poisoned, say

pytestmark = pytest.mark.gpu


def _weights(N, K, fmt, seed):
    g = np.random.Generator(np.random.PCG64(seed))
    if fmt == 1:
        return (g.integers(-127, 128, (N, K), dtype=np.int16).astype(np.int8),
                O.f2h(g.uniform(0.5, 1.5, N).astype(np.float32) / 127), None)
    return (g.integers(0, 256, (N, K), dtype=np.int16).astype(np.uint8),
            O.f2h(g.uniform(0.5, 1.5, (N, K // 128)).astype(np.float32) / 255),
            g.integers(100, 157, (N, K // 128), dtype=np.int16).astype(np.uint8))


@pytest.mark.parametrize("fmt", [1, 2])
def test_noalloc_matches_the_allocating_entry_point(gpu, fmt):
    import torch
    from cuda_tempiler_amd import capi

    # first a split-K shape with a large workspace, then a smaller split-K shape, then a shape
    # whose row uses no workspace at all
    for i, (M, N, K) in enumerate([(128, 5120, 17408), (100, 2048, 5120), (16, 7168, 5120)]):
        need = capi.workspace_bytes(fmt, M, N, K)
        say("noalloc fmt", fmt, "M", M, "N", N, "K", K, "route", capi.route(fmt, M, N, K),
            "workspace", need)
        assert need <= capi.NOALLOC_SCRATCH_BYTES
        # the first two shapes must exercise the scratch (a ladder change that stopped routing
        # them to split-K rows would otherwise leave it untested), the third must not
        assert (need > 0) == (i < 2), (M, N, K, need)
        A = O.randn_f16((M, K), 3 + M, K ** -0.5)
        q, s, z = _weights(N, K, fmt, 5 + N)
        dA, dq, ds = dev(A, gpu), dev(q, gpu), dev(s, gpu)
        dz = dev(z, gpu) if z is not None else None
        C_pool = poisoned((M, N), gpu)
        C_none = poisoned((M, N), gpu)
        capi.gemm_w8a16(dA, dq, ds, dz, fmt=fmt, group=128, C=C_pool)
        capi.gemm_w8a16_noalloc(dA, dq, ds, dz, fmt=fmt, group=128, C=C_none)
        torch.cuda.synchronize()
        a, b = host(C_pool), host(C_none)
        assert O.count_poison(b) == 0
        assert np.array_equal(a.view(np.uint16), b.view(np.uint16)), "entry points disagree"
        rel = O.rel_l2(b, O.gemm_w8a16(A, q, s, z, 128, fmt))
        say("  bit-equal to the allocating entry point; relL2 vs oracle %.3e" % rel)
        assert rel <= 3e-3
