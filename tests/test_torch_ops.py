"""CPU checks of the torch.library integration (reference INTEGRATION.md:81-116): the gate is
off by default, refusals take the caller's own path, every call is counted, and the 8-bit
fallback dequantises exactly as the oracle does."""
import numpy as np
import pytest
import torch

from oracle import oracle as O


@pytest.fixture
def tops(monkeypatch):
    import cuda_tempiler_amd.torch_ops as t

    monkeypatch.delenv("TEMPO_KERNELS", raising=False)
    t.reset_counters()
    return t


def test_gate_defaults_off(tops):
    assert not tops.enabled()
    x = torch.randn(4, 64, dtype=torch.float16)
    w = torch.randn(32, 64, dtype=torch.float16)
    y = torch.ops.tempo.linear_fp16(x, w)
    assert torch.equal(y, torch.nn.functional.linear(x, w))
    assert tops.counters() == {"off": 1}


@pytest.mark.parametrize("val", ["0", "", "true", "yes"])
def test_gate_only_opens_on_one(tops, monkeypatch, val):
    monkeypatch.setenv("TEMPO_KERNELS", val)
    assert not tops.enabled()


def test_gate_on_host_tensors_fall_back(tops, monkeypatch):
    monkeypatch.setenv("TEMPO_KERNELS", "1")
    x = torch.randn(2, 3, 64, dtype=torch.float16)
    w = torch.randn(32, 64, dtype=torch.float16)
    y = torch.ops.tempo.linear_fp16(x, w)
    assert y.shape == (2, 3, 32)
    assert torch.equal(y, torch.nn.functional.linear(x, w))
    assert tops.counters() == {"fallback": 1}


def test_fake_kernels_and_schema(tops):
    x = torch.randn(2, 5, 64, dtype=torch.float16)
    w = torch.randn(48, 64, dtype=torch.float16)
    torch.library.opcheck(torch.ops.tempo.linear_fp16, (x, w))
    q = torch.randint(0, 256, (48, 128), dtype=torch.uint8)
    s = torch.rand(48, 1, dtype=torch.float16) / 255
    z = torch.randint(100, 157, (48, 1), dtype=torch.uint8)
    torch.library.opcheck(torch.ops.tempo.linear_w8a16, (x[..., :64].new_zeros(2, 5, 128), q, s,
                                                         z, 2, 128))
    with torch.device("meta"):
        y = torch.ops.tempo.linear_fp16(torch.empty(7, 3, 64, dtype=torch.float16),
                                        torch.empty(96, 64, dtype=torch.float16))
    assert y.shape == (7, 3, 96)


@pytest.mark.parametrize("fmt", [1, 2])
def test_fallback_dequant_is_the_oracles(tops, fmt):
    g = np.random.Generator(np.random.PCG64(fmt))
    N, K = 64, 384
    if fmt == 1:
        q = g.integers(-128, 128, (N, K), dtype=np.int16).astype(np.int8)
        s = O.f2h(g.uniform(1e-4, 3.0, N).astype(np.float32))
        ref = O.dequant_sym(q, s)
        got = tops.dequantize(torch.from_numpy(q), torch.from_numpy(s), None, 1)
    else:
        q = g.integers(0, 256, (N, K), dtype=np.int16).astype(np.uint8)
        s = O.f2h(g.uniform(1e-4, 3.0, (N, K // 128)).astype(np.float32))
        z = g.integers(0, 256, (N, K // 128), dtype=np.int16).astype(np.uint8)
        ref = O.dequant_asym(q, s, z, 128)
        got = tops.dequantize(torch.from_numpy(q), torch.from_numpy(s), torch.from_numpy(z), 2)
    assert np.array_equal(got.numpy().view(np.uint16), ref.view(np.uint16))


def test_swap_linears_counts_fp16_layers_only(tops):
    m = torch.nn.Sequential(torch.nn.Linear(64, 32, bias=False).half(), torch.nn.ReLU(),
                            torch.nn.Sequential(torch.nn.Linear(32, 16, bias=False).half()),
                            torch.nn.Linear(16, 8))
    x = torch.randn(4, 64, dtype=torch.float16)
    ref = m[2](m[1](m[0](x)))
    assert tops.swap_linears(m) == 2
    assert isinstance(m[0], tops.Linear) and isinstance(m[2][0], tops.Linear)
    assert isinstance(m[3], torch.nn.Linear)
    assert torch.equal(m[2](m[1](m[0](x))), ref)
    assert tops.counters() == {"off": 2}


def test_linear_bias_is_added_after_the_product(tops):
    lin = torch.nn.Linear(64, 32).half()
    x = torch.randn(4, 64, dtype=torch.float16)
    got = tops.Linear.from_linear(lin)(x)
    want = torch.nn.functional.linear(x, lin.weight) + lin.bias
    assert torch.equal(got, want)
    assert torch.allclose(got.float(), lin(x).float(), atol=2e-3, rtol=2e-3)


def test_gate_up_fallback_is_silu_times_up(tops, monkeypatch):
    x = torch.randn(2, 3, 64, dtype=torch.float16)
    w = torch.randn(2 * 40, 64, dtype=torch.float16)
    y = torch.ops.tempo.linear_gate_up_fp16(x, w)
    g, u = torch.nn.functional.linear(x, w).chunk(2, dim=-1)
    assert y.shape == (2, 3, 40)
    assert torch.equal(y, torch.nn.functional.silu(g) * u)
    assert tops.counters() == {"off": 1}
    monkeypatch.setenv("TEMPO_KERNELS", "1")
    assert torch.equal(torch.ops.tempo.linear_gate_up_fp16(x, w), y)  # host tensors: fallback
    assert tops.counters() == {"off": 1, "fallback": 1}
    torch.library.opcheck(torch.ops.tempo.linear_gate_up_fp16, (x, w))
    q = torch.randint(-127, 128, (80, 64), dtype=torch.int8)
    s = torch.rand(80, dtype=torch.float16) / 127
    y8 = torch.ops.tempo.linear_gate_up_w8a16(x, q, s, None, 1, 128)
    g8, u8 = torch.nn.functional.linear(x, tops.dequantize(q, s, None, 1)).chunk(2, dim=-1)
    assert torch.equal(y8, torch.nn.functional.silu(g8) * u8)
