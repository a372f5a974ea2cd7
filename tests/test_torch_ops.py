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


# ---- operand validation: malformed 8-bit operands never reach the kernels ---------------------
def _w8(fmt, N=64, K=256, G=128):
    A = torch.zeros(3, K, dtype=torch.float16)
    if fmt == 1:
        return A, torch.zeros(N, K, dtype=torch.int8), torch.ones(N, dtype=torch.float16), None
    return (A, torch.zeros(N, K, dtype=torch.uint8), torch.ones(N, K // G, dtype=torch.float16),
            torch.zeros(N, K // G, dtype=torch.uint8))


@pytest.mark.parametrize("fmt", [1, 2])
def test_w8_operands_well_formed(fmt):
    from cuda_tempiler_amd import capi

    assert capi.w8a16_operand_error(*_w8(fmt), fmt, 128) is None


@pytest.mark.parametrize("case", [
    "u8_with_fmt1", "i8_with_fmt2", "fp32_scale", "gptq_layout_scale", "short_scale",
    "short_zero", "zero_wrong_dtype", "zero_with_fmt1", "no_zero_fmt2", "strided_scale",
    "bad_fmt", "ragged_group", "k_mismatch"])
def test_w8_operands_malformed_are_refused(case):
    from cuda_tempiler_amd import capi

    fmt = 2 if case in ("i8_with_fmt2", "gptq_layout_scale", "short_zero", "zero_wrong_dtype",
                        "no_zero_fmt2", "ragged_group") else 1
    A, wq, s, z = _w8(fmt)
    N, K = wq.shape
    group = 128
    if case == "u8_with_fmt1":
        wq = wq.to(torch.uint8)
    elif case == "i8_with_fmt2":
        wq = wq.to(torch.int8)
    elif case == "fp32_scale":
        s = s.float()
    elif case == "gptq_layout_scale":          # [K/G, N] has the element count of [N, K/G]
        s = torch.ones(K // 128, N, dtype=torch.float16)
    elif case == "short_scale":
        s = s[: N // 2]
    elif case == "short_zero":
        z = z[: N // 2]
    elif case == "zero_wrong_dtype":
        z = z.to(torch.int8)
    elif case == "zero_with_fmt1":
        z = torch.zeros(N, 2, dtype=torch.uint8)
    elif case == "no_zero_fmt2":
        z = None
    elif case == "strided_scale":
        s = torch.ones(N, 2, dtype=torch.float16)[:, 0]
    elif case == "bad_fmt":
        fmt = 3
    elif case == "ragged_group":
        group = 96
    elif case == "k_mismatch":
        A = torch.zeros(3, K + 8, dtype=torch.float16)
    assert capi.w8a16_operand_error(A, wq, s, z, fmt, group) is not None
    with pytest.raises(ValueError):
        capi._require_w8(A, wq, s, z, fmt, group)


def test_w8_gate_on_malformed_takes_own_path(tops, monkeypatch):
    """With the gate on, a malformed operand set is the caller's path (counted 'fallback'), and
    that path computes the same thing it computes with the gate off."""
    monkeypatch.setenv("TEMPO_KERNELS", "1")
    x = torch.randn(2, 256, dtype=torch.float16)
    wq = torch.randint(-127, 128, (64, 256), dtype=torch.int8)
    s = (torch.rand(64) / 127).float()   # fp32 scale: not the kernels' layout
    y_on = torch.ops.tempo.linear_w8a16(x, wq, s, None, 1, 128)
    monkeypatch.setenv("TEMPO_KERNELS", "0")
    y_off = torch.ops.tempo.linear_w8a16(x, wq, s, None, 1, 128)
    assert torch.equal(y_on, y_off)
    assert tops.counters() == {"fallback": 1, "off": 1}


@pytest.mark.parametrize("case", ["ok", "qweight_dtype", "qzeros_shape", "scales_layout",
                                  "scales_dtype", "ragged_k"])
def test_gptq_operand_checks(case):
    from cuda_tempiler_amd import capi

    K, N, G = 256, 64, 128
    qw = torch.zeros(K // 4, N, dtype=torch.int32)
    qz = torch.zeros(K // G, N // 4, dtype=torch.int32)
    sc = torch.ones(K // G, N, dtype=torch.float16)
    if case == "qweight_dtype":
        qw = qw.to(torch.int64)
    elif case == "qzeros_shape":
        qz = torch.zeros(K // G, N, dtype=torch.int32)
    elif case == "scales_layout":               # kernel layout [N, K/G] instead of [K/G, N]
        sc = torch.ones(N, K // G, dtype=torch.float16)
    elif case == "scales_dtype":
        sc = sc.float()
    elif case == "ragged_k":
        qw = torch.zeros(K // 4 - 8, N, dtype=torch.int32)
    why = capi.gptq_operand_error(qw, qz, sc, G)
    assert (why is None) == (case == "ok"), why
