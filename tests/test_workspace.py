"""Split-K workspace bounds and the host-side checks of the C-ABI binding (CPU only: every call
here is host-only -- route and workspace sizing -- or is refused before any launch).

The allocation-free entry point serves split-K rows from a static TEMPO_NOALLOC_SCRATCH_BYTES
(32 MiB) array per GPU, so no W8A16 ladder row may ever need more.  Two row kinds take a
workspace: interleaved tile rows (tiles x splits <= 256 workgroups of at most 128 x 256 fp32
partials: 256 x 128 x 256 x 4 = 32 MiB) and line rows with k slices (ks <= 8 slices of M x N
fp32 over each row's band).  The sweep below runs every W8A16 row's sizing over the shape grid
of the ladder coverage test and both formats.
"""
import pytest

from tests import test_ladder_coverage as LCov


@pytest.fixture(scope="module")
def capi():
    from cuda_tempiler_amd import capi as c

    c.lib()
    return c


@pytest.mark.parametrize("fmt", [1, 2])
def test_every_w8a16_row_fits_the_noalloc_scratch(capi, fmt):
    worst, where, seen = 0, None, 0
    for M in LCov._M:
        for N in LCov._N:
            for K in LCov._K:
                need = capi.workspace_bytes(fmt, M, N, K)
                seen += need > 0
                if need > worst:
                    worst, where = need, (M, N, K, capi.route(fmt, M, N, K))
    assert seen > 0, "no shape of the grid takes a split-K row: the sweep checks nothing"
    assert worst <= capi.NOALLOC_SCRATCH_BYTES, "%d bytes at %s" % (worst, where)


def test_output_is_validated_before_any_launch(capi):
    """A wrong C (dtype, shape, inner stride) is refused on the host: the kernels would write it
    as raw fp16 [M, N] memory."""
    import torch

    M, N, K = 4, 64, 256
    A = torch.zeros(M, K, dtype=torch.float16)
    wq = torch.zeros(N, K, dtype=torch.int8)
    s = torch.ones(N, dtype=torch.float16)
    for C in (torch.zeros(M, N, dtype=torch.float32),          # fp32
              torch.zeros(M - 1, N, dtype=torch.float16),      # too few rows
              torch.zeros(N, M, dtype=torch.float16).t()):     # no unit inner stride
        for fn in (capi.gemm_w8a16, capi.gemm_w8a16_noalloc):
            with pytest.raises(ValueError):
                fn(A, wq, s, None, fmt=1, C=C)
        with pytest.raises(ValueError):
            capi.gemm_w8a16_gate_up(A, torch.zeros(2 * N, K, dtype=torch.int8),
                                    torch.ones(2 * N, dtype=torch.float16), None, fmt=1, C=C)


def test_workspace_argument_is_checked(capi):
    import torch

    A = torch.zeros(4, 256, dtype=torch.float16)
    B = torch.zeros(64, 256, dtype=torch.float16)
    with pytest.raises(ValueError):
        capi.gemm_fp16(A, B, workspace="pool")  # only None, "torch" or a tensor
