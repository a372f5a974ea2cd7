"""GPU parity of the causal FMHA forward (skeletons/fmha_fwd) against the CPU oracle.

Semantics follow the reference's attention path: bottom-right causal mask with off = Sk - Sq
(attn_fwd_cutlass.cu:137, volta_fwd_ws.cuh:863), GQA head map h -> h / (H / Hkv)
(volta_fwd_ws.cuh:432), LSE in natural-log units (volta_fwd_ws.cuh:1063).  Outputs are fp16:
relL2 <= 3e-3 against the oracle's fp32-softmax result; LSE within 2e-3 absolute.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.gpu_util import dev, host, poisoned, say

pytestmark = pytest.mark.gpu

TOL = 3e-3
LSE_TOL = 2e-3


def _inputs(B, Sq, Sk, H, Hkv, D, seed):
    g = np.random.Generator(np.random.PCG64(seed))
    Q = O.f2h(g.standard_normal((B, Sq, H, D), dtype=np.float32))
    K = O.f2h(g.standard_normal((B, Sk, Hkv, D), dtype=np.float32))
    V = O.f2h(g.standard_normal((B, Sk, Hkv, D), dtype=np.float32))
    return Q, K, V


def _run(Q, K, V, scale, causal, device):
    import torch
    from cuda_tempiler_amd import capi

    dQ = dev(Q, device)
    dO = poisoned(Q.shape, device)
    O_, L_ = capi.fmha_fwd(dQ, dev(K, device), dev(V, device), scale, causal, O=dO)
    torch.cuda.synchronize()
    return host(O_), host(L_)


CASES = [
    # B, Sq, Sk, H, Hkv, D, causal
    (1, 64, 64, 4, 2, 128, True),
    (1, 128, 128, 2, 2, 256, True),
    (2, 200, 200, 4, 4, 256, True),
    (1, 130, 130, 2, 1, 128, False),
    (1, 77, 300, 4, 2, 256, True),     # Sq < Sk: off = 223, rows see a prefix plus their own
    (1, 1, 517, 8, 2, 128, True),      # one decode row over a ragged key tail
    (1, 300, 300, 2, 1, 256, False),   # ragged query and key tails
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "b%d_q%d_k%d_h%d_kv%d_d%d_%s" % (
    c[0], c[1], c[2], c[3], c[4], c[5], "causal" if c[6] else "full"))
def test_fmha_parity_small(gpu, case):
    B, Sq, Sk, H, Hkv, D, causal = case
    say("fmha case", case)
    Q, K, V = _inputs(B, Sq, Sk, H, Hkv, D, seed=1000 + Sq + Sk + D)
    scale = 1.0 / np.sqrt(D)
    got, lse = _run(Q, K, V, scale, causal, gpu)
    ref, lref = O.fmha_fwd(Q, K, V, scale, causal)
    assert O.count_poison(got) == 0
    r = O.rel_l2(got, ref)
    say("  relL2 %.3e" % r)
    assert r <= TOL
    assert _lse_close(lse, lref)


def _lse_close(lse, lref):
    inf = np.isneginf(lref)
    assert np.array_equal(np.isneginf(lse), inf)
    return np.max(np.abs(lse[~inf] - lref[~inf]), initial=0.0) <= LSE_TOL


def test_fmha_rows_without_keys(gpu):
    """Causal with Sq > Sk: off = Sk - Sq < 0, the first Sq - Sk rows see no key at all; their
    output is 0 and their LSE -inf, as in the oracle."""
    B, Sq, Sk, H, Hkv, D = 1, 300, 130, 2, 1, 128
    Q, K, V = _inputs(B, Sq, Sk, H, Hkv, D, seed=21)
    got, lse = _run(Q, K, V, 1.0 / np.sqrt(D), True, gpu)
    ref, lref = O.fmha_fwd(Q, K, V, 1.0 / np.sqrt(D), True)
    assert O.count_poison(got) == 0
    assert not np.any(got[:, : Sq - Sk].astype(np.float32))
    assert O.rel_l2(got, ref) <= TOL
    assert _lse_close(lse, lref)


@pytest.mark.parametrize("causal", [True, False])
def test_fmha_growing_scores_rescale(gpu, causal):
    """Key rows scaled up along the sequence: every block's max overtakes the running one by a
    wide margin, so the running-max rescale of the output is taken again and again."""
    B, S, H, Hkv, D = 1, 512, 2, 2, 128
    Q, K, V = _inputs(B, S, S, H, Hkv, D, seed=33)
    grow = (1.0 + np.arange(S, dtype=np.float32) / 24.0)[None, :, None, None]
    K = O.f2h(K.astype(np.float32) * grow)
    got, lse = _run(Q, K, V, 1.0 / np.sqrt(D), causal, gpu)
    ref, lref = O.fmha_fwd(Q, K, V, 1.0 / np.sqrt(D), causal)
    r = O.rel_l2(got, ref)
    say("growing scores relL2 %.3e" % r)
    assert r <= TOL
    assert _lse_close(lse, lref)


def test_fmha_strided_bhsd(gpu):
    """Q/K/V handed over as BSHD views of BHSD storage: the kernel honours every stride."""
    import torch
    from cuda_tempiler_amd import capi

    B, S, H, Hkv, D = 1, 192, 4, 2, 128
    Q, K, V = _inputs(B, S, S, H, Hkv, D, seed=7)
    tQ = dev(np.ascontiguousarray(Q.transpose(0, 2, 1, 3)), gpu).permute(0, 2, 1, 3)
    tK = dev(np.ascontiguousarray(K.transpose(0, 2, 1, 3)), gpu).permute(0, 2, 1, 3)
    tV = dev(np.ascontiguousarray(V.transpose(0, 2, 1, 3)), gpu).permute(0, 2, 1, 3)
    assert not tQ.is_contiguous()
    O_, _ = capi.fmha_fwd(tQ, tK, tV, 1.0 / np.sqrt(D), True)
    torch.cuda.synchronize()
    ref, _ = O.fmha_fwd(Q, K, V, 1.0 / np.sqrt(D), True)
    assert O.rel_l2(host(O_), ref) <= TOL


def test_fmha_c5_sampled_rows(gpu):
    """Config C5 at full size (B=1, H=16, Hkv=8, S=4096, D=256, causal); the oracle computes 512
    query rows of all 16 heads: the first and last of the sequence, the edges of query blocks and
    a seeded random set."""
    B, S, H, Hkv, D = 1, 4096, 16, 8, 256
    Q, K, V = _inputs(B, S, S, H, Hkv, D, seed=5)
    scale = 1.0 / 16
    got, lse = _run(Q, K, V, scale, True, gpu)
    assert O.count_poison(got) == 0
    g = np.random.Generator(np.random.PCG64(99))
    edges = [0, 1, 31, 32, 63, 64, 127, 128, 255, 256, 2047, 2048, S - 129, S - 128, S - 2, S - 1]
    rest = g.permutation(np.setdiff1d(np.arange(S), edges))[:512 - len(edges)]
    rows = np.unique(np.concatenate([edges, rest])).astype(np.int32)
    assert rows.size == 512
    ref, lref = O.fmha_fwd(Q, K, V, scale, True, rows=rows)
    r = O.rel_l2(got[:, rows], ref[:, rows])
    say("C5 sampled relL2 %.3e over %d rows x %d heads" % (r, rows.size, H))
    assert r <= TOL
    assert np.max(np.abs(lse[:, :, rows] - lref[:, :, rows])) <= LSE_TOL


def test_fmha_refuses_uncovered_head_dim(gpu):
    from cuda_tempiler_amd import capi

    Q, K, V = _inputs(1, 64, 64, 2, 2, 64, seed=3)
    with pytest.raises(capi.NotCovered):
        _run(Q, K, V, 0.125, True, gpu)


NAIVE_CASES = [c for c in CASES if c[1] * c[3] <= 1200]  # the naive kernel is one thread per row


@pytest.mark.parametrize("case", NAIVE_CASES, ids=lambda c: "b%d_q%d_k%d_h%d_kv%d_d%d_%s" % (
    c[0], c[1], c[2], c[3], c[4], c[5], "causal" if c[6] else "full"))
def test_naive_attention_input_against_oracle_and_shipped(gpu, case):
    """The naive attention input (kernels/naive/fmha_fwd.hip, the operation's declaration and
    "vs input" bar) against the oracle, and the shipped kernel against it."""
    import torch
    from cuda_tempiler_amd import capi

    B, Sq, Sk, H, Hkv, D, causal = case
    say("naive fmha case", case)
    Q, K, V = _inputs(B, Sq, Sk, H, Hkv, D, seed=2000 + Sq + Sk + D)
    scale = 1.0 / np.sqrt(D)
    On, Ln = capi.naive_fmha_fwd(dev(Q, gpu), dev(K, gpu), dev(V, gpu), scale, causal)
    torch.cuda.synchronize()
    naive, lnaive = host(On), host(Ln)
    ref, lref = O.fmha_fwd(Q, K, V, scale, causal)
    r = O.rel_l2(naive, ref)
    say("  naive relL2 vs oracle %.3e" % r)
    assert r <= TOL
    inf = ~np.isfinite(lref)
    assert np.array_equal(inf, ~np.isfinite(lnaive))
    assert np.max(np.abs(lnaive[~inf] - lref[~inf]), initial=0.0) <= LSE_TOL
    got, _ = _run(Q, K, V, scale, causal, gpu)
    r2 = O.rel_l2(got, naive)
    say("  shipped relL2 vs naive %.3e" % r2)
    assert r2 <= TOL
