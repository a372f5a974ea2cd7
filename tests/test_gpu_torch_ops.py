"""Entry proof of the torch.library integration on the GPU (reference INTEGRATION.md:107-116):
with TEMPO_KERNELS=1 the custom ops run the shipped ladder (the row counter names the row and
the output is bit-for-bit the direct C-ABI call's); with the gate off they run F.linear."""
import numpy as np
import pytest

from oracle import oracle as O
from tests.gpu_util import dev, host, say

pytestmark = pytest.mark.gpu


@pytest.fixture
def tops(monkeypatch):
    import cuda_tempiler_amd.torch_ops as t

    t.reset_counters()
    return t


@pytest.mark.parametrize("shape", [(1, 15360, 3840), (16, 3840, 15360), (300, 4096, 3840)],
                         ids=lambda s: "m%d_n%d_k%d" % s)
def test_linear_fp16_entry_proof(gpu, tops, monkeypatch, shape):
    import torch
    from cuda_tempiler_amd import capi

    M, N, K = shape
    x = torch.randn((M, K), dtype=torch.float16, device=gpu) / K ** 0.5
    w = torch.randn((N, K), dtype=torch.float16, device=gpu)
    monkeypatch.setenv("TEMPO_KERNELS", "1")
    y = torch.ops.tempo.linear_fp16(x, w)
    direct = capi.gemm_fp16(x, w)
    torch.cuda.synchronize()
    tag = capi.route(0, M, N, K)
    say("entry", shape, tops.counters())
    assert tops.counters() == {tag: 1}
    assert torch.equal(y.view(torch.int16), direct.view(torch.int16))
    monkeypatch.setenv("TEMPO_KERNELS", "0")
    off = torch.ops.tempo.linear_fp16(x, w)
    assert tops.counters() == {tag: 1, "off": 1}
    r = O.rel_l2(host(y), host(off))
    say("  relL2 vs F.linear %.2e" % r)
    assert r <= 3e-3


def test_linear_fp16_batched_leading_dims(gpu, tops, monkeypatch):
    import torch

    monkeypatch.setenv("TEMPO_KERNELS", "1")
    x = torch.randn((2, 3, 512), dtype=torch.float16, device=gpu) / 512 ** 0.5
    w = torch.randn((1024, 512), dtype=torch.float16, device=gpu)
    y = torch.ops.tempo.linear_fp16(x, w)
    torch.cuda.synchronize()
    assert y.shape == (2, 3, 1024)
    assert "fallback" not in tops.counters() and "off" not in tops.counters()
    ref = O.gemm_f16(host(x).reshape(6, 512), host(w)).reshape(2, 3, 1024)
    assert O.rel_l2(host(y), ref) <= 3e-3


def test_linear_fp16_refusal_takes_own_path(gpu, tops, monkeypatch):
    """K = 100 is not covered by any row: TEMPO_FALLBACK, F.linear, counted as fallback."""
    import torch

    monkeypatch.setenv("TEMPO_KERNELS", "1")
    x = torch.randn((8, 100), dtype=torch.float16, device=gpu)
    w = torch.randn((256, 100), dtype=torch.float16, device=gpu)
    y = torch.ops.tempo.linear_fp16(x, w)
    torch.cuda.synchronize()
    assert tops.counters() == {"fallback": 1}
    assert torch.equal(y, torch.nn.functional.linear(x, w))


@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("M", [1, 32, 256])
def test_linear_w8a16_entry_proof(gpu, tops, monkeypatch, fmt, M):
    import torch
    from cuda_tempiler_amd import capi

    N, K = 5120, 6144
    g = torch.Generator(device="cpu").manual_seed(M + fmt)
    if fmt == 1:
        q = torch.randint(-127, 128, (N, K), dtype=torch.int8, generator=g).to(gpu)
        s = (torch.rand(N, generator=g) / 127 + 1e-3).half().to(gpu)
        z = None
    else:
        q = torch.randint(0, 256, (N, K), dtype=torch.uint8, generator=g).to(gpu)
        s = (torch.rand((N, K // 128), generator=g) / 255 + 1e-4).half().to(gpu)
        z = torch.randint(100, 157, (N, K // 128), dtype=torch.uint8, generator=g).to(gpu)
    x = (torch.randn((M, K), generator=g) / K ** 0.5).half().to(gpu)
    monkeypatch.setenv("TEMPO_KERNELS", "1")
    y = torch.ops.tempo.linear_w8a16(x, q, s, z, fmt, 128)
    direct = capi.gemm_w8a16(x, q, s, z, fmt=fmt, group=128)
    torch.cuda.synchronize()
    tag = capi.route(fmt, M, N, K)
    say("entry w8a16", fmt, M, tops.counters())
    assert tops.counters() == {tag: 1}
    assert torch.equal(y.view(torch.int16), direct.view(torch.int16))
    monkeypatch.delenv("TEMPO_KERNELS")
    off = torch.ops.tempo.linear_w8a16(x, q, s, z, fmt, 128)
    assert tops.counters() == {tag: 1, "off": 1}
    assert O.rel_l2(host(y), host(off)) <= 3e-3


def test_gptq_linear_module(gpu, tops, monkeypatch):
    """GPTQ checkpoint -> GPTQLinear (device repack at construction) -> tempo::linear_w8a16,
    against the oracle's dense weights (gemm_baseline.py:229) plus bias."""
    import torch

    K, N, G = 5120, 6144, 128
    rg = np.random.Generator(np.random.PCG64(4))
    qw = rg.integers(-(2**31), 2**31 - 1, (K // 4, N), dtype=np.int64).astype(np.int32)
    qz = rg.integers(-(2**31), 2**31 - 1, (K // G, N // 4), dtype=np.int64).astype(np.int32)
    sc = O.f2h(rg.uniform(0.001, 0.021, (K // G, N)).astype(np.float32))
    b = O.f2h(rg.standard_normal(N).astype(np.float32))
    layer = tops.GPTQLinear(dev(qw, gpu), dev(qz, gpu), dev(sc, gpu), bias=dev(b, gpu))
    A = O.f2h(rg.standard_normal((4, K), dtype=np.float32))
    monkeypatch.setenv("TEMPO_KERNELS", "1")
    y = layer(dev(A, gpu))
    torch.cuda.synchronize()
    assert list(tops.counters()) == [tops.capi.route(2, 4, N, K)]
    W = O.gptq_dense(qw, qz, sc)
    ref = O.gemm_f16(A, np.ascontiguousarray(W.T)).astype(np.float32) + b.astype(np.float32)
    r = O.rel_l2(host(y), ref)
    say("GPTQLinear relL2 %.2e" % r)
    assert r <= 3e-3


@pytest.mark.parametrize("M", [1, 16, 64])
def test_gate_up_entry_proof(gpu, tops, monkeypatch, M):
    """Decode M: the fused kernel runs (counter = its ladder row, bit-for-bit the C-ABI call);
    M = 64 is not covered: the fallback (F.linear, silu, product) runs and is counted."""
    import torch
    from cuda_tempiler_amd import capi

    N, K = 4096, 2048
    x = torch.randn((M, K), dtype=torch.float16, device=gpu) / K ** 0.5
    w = torch.randn((2 * N, K), dtype=torch.float16, device=gpu)
    monkeypatch.setenv("TEMPO_KERNELS", "1")
    y = torch.ops.tempo.linear_gate_up_fp16(x, w)
    torch.cuda.synchronize()
    tag = capi.route(3, M, N, K)
    say("gate_up entry M=%d" % M, tops.counters())
    g, u = torch.nn.functional.linear(x, w).chunk(2, dim=-1)
    own = torch.nn.functional.silu(g) * u
    if tag:
        assert tops.counters() == {tag: 1}
        assert torch.equal(y.view(torch.int16), capi.gemm_fp16_gate_up(x, w).view(torch.int16))
        assert O.rel_l2(host(y), host(own)) <= 3e-3
    else:
        assert tops.counters() == {"fallback": 1}
        assert torch.equal(y, own)
