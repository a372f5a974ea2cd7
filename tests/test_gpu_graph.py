"""Split-K rows under HIP graph capture (torch.cuda.graph).

The torch ops take a split-K row's workspace from torch's caching allocator (graph-aware: under
capture it hands out memory of the graph's own pool, valid for every replay) through the C ABI's
tempo_gemm_*_launch_ws.  The library's own pool cannot grow under capture (hipMalloc is not
capturable): there tempo_gemm_*_launch returns hipErrorStreamCaptureUnsupported and records
nothing.  No memset is recorded: the workspace is written in full before it is read.

Each graph is replayed several times with eager work and synchronisations between the replays,
and every replay is compared bit for bit with the eager result on the same inputs.
"""
import pytest

from tests.gpu_util import say

pytestmark = pytest.mark.gpu


def _capture_and_replay(fn, inputs, fresh):
    """Warm fn up on a side stream, capture it, then replay it three times; between replays,
    eager calls on other inputs and a synchronisation.  fresh() refills the inputs in place."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn(*inputs)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn(*inputs)
    results = []
    for r in range(3):
        fresh(r)
        torch.cuda.synchronize()
        eager = fn(*inputs).clone()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        results.append((r, torch.equal(out.view(torch.int16), eager.view(torch.int16))))
        other = fn(*[x.clone() for x in inputs])  # eager work between replays
        del other
    return results


@pytest.mark.parametrize("shape", [(128, 3840, 15360), (64, 3840, 15360)],
                         ids=lambda s: "m%d_n%d_k%d" % s)
def test_linear_fp16_split_k_under_capture(gpu, monkeypatch, shape):
    import torch
    from cuda_tempiler_amd import capi
    import cuda_tempiler_amd.torch_ops  # noqa: F401  (registers the ops)

    M, N, K = shape
    assert capi.workspace_bytes(0, M, N, K) > 0, "the shape must take a split-K row"
    say("capture fp16", shape, capi.route(0, M, N, K))
    monkeypatch.setenv("TEMPO_KERNELS", "1")
    gen = torch.Generator(device=gpu)
    x = torch.empty((M, K), dtype=torch.float16, device=gpu)
    w = (torch.randn((N, K), generator=gen.manual_seed(1), device=gpu) / K ** 0.5).half()

    def fresh(r):
        x.copy_(torch.randn((M, K), generator=gen.manual_seed(10 + r), device=gpu).half())

    fresh(-1)
    res = _capture_and_replay(lambda a, b: torch.ops.tempo.linear_fp16(a, b), (x, w), fresh)
    say("  replays bit-equal to eager:", res)
    assert all(ok for _, ok in res)


@pytest.mark.parametrize("fmt", [1, 2])
def test_linear_w8a16_split_k_under_capture(gpu, monkeypatch, fmt):
    import torch
    from cuda_tempiler_amd import capi
    import cuda_tempiler_amd.torch_ops  # noqa: F401

    M, N, K, G = 128, 5120, 17408, 128
    assert capi.workspace_bytes(fmt, M, N, K) > 0
    say("capture w8a16 fmt", fmt, (M, N, K), capi.route(fmt, M, N, K))
    monkeypatch.setenv("TEMPO_KERNELS", "1")
    gen = torch.Generator(device=gpu)
    x = torch.empty((M, K), dtype=torch.float16, device=gpu)
    if fmt == 1:
        wq = torch.randint(-127, 128, (N, K), generator=gen.manual_seed(2), device=gpu,
                           dtype=torch.int8)
        s = (torch.rand(N, generator=gen, device=gpu) + 0.5).div(127).half()
        z = None
    else:
        wq = torch.randint(0, 256, (N, K), generator=gen.manual_seed(2), device=gpu,
                           dtype=torch.uint8)
        s = (torch.rand((N, K // G), generator=gen, device=gpu) + 0.5).div(255).half()
        z = torch.randint(100, 157, (N, K // G), generator=gen, device=gpu, dtype=torch.uint8)

    def fresh(r):
        x.copy_((torch.randn((M, K), generator=gen.manual_seed(20 + r), device=gpu)
                 / K ** 0.5).half())

    fresh(-1)
    res = _capture_and_replay(
        lambda a: torch.ops.tempo.linear_w8a16(a, wq, s, z, fmt, G), (x,), fresh)
    say("  replays bit-equal to eager:", res)
    assert all(ok for _, ok in res)


def test_pool_refuses_to_grow_under_capture(gpu):
    """On a stream whose pool buffer has never been allocated, a split-K launch under capture
    returns hipErrorStreamCaptureUnsupported (900) instead of calling hipMalloc; nothing is
    recorded or launched."""
    import torch
    from cuda_tempiler_amd import capi

    M, N, K = 128, 3840, 15360
    A = torch.zeros((M, K), dtype=torch.float16, device=gpu)
    B = torch.zeros((N, K), dtype=torch.float16, device=gpu)
    C = torch.empty((M, N), dtype=torch.float16, device=gpu)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    code = None
    with torch.cuda.graph(g, stream=s):
        C.zero_()  # a fill kernel, so the graph is not empty
        try:
            capi.gemm_fp16(A, B, C)  # the pool path (workspace=None)
        except capi.TempoError as e:
            code = e.code
    torch.cuda.synchronize()
    say("pool under capture ->", code)
    assert code == capi.HIP_ERROR_CAPTURE_UNSUPPORTED
    # the same call eagerly on that stream grows the pool and runs
    with torch.cuda.stream(s):
        capi.gemm_fp16(A, B, C)
    torch.cuda.synchronize()
    assert not torch.any(C.float()).item()
