"""Pins the CPU oracle (oracle/tempo_oracle.c) before anything is checked against it.

Each check is independent of the code under test: exact integer arithmetic, the F16C hardware
converter, numpy's IEEE casts, fp64 brute force, or a closed form.  A plausible slip in the
oracle -- a transposed operand, a dropped term, a wrong rounding, a swapped index -- fails at
least one of them.
"""
import json
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden", "ship_probe_cells.json")


def test_f2h_exhaustive_against_f16c():
    # every one of the 2^32 float bit patterns, against the hardware converter
    assert O.check_f2h_exhaustive(0) == 0


def test_h2f_all_halves_against_numpy():
    h = np.arange(65536, dtype=np.uint16)
    got = O.h2f(h)
    ref = h.view(np.float16).astype(np.float32)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all()


def test_f2h_against_numpy_cast():
    g = np.random.Generator(np.random.PCG64(3))
    x = np.concatenate([
        g.standard_normal(200000).astype(np.float32) * 1000,
        g.standard_normal(200000).astype(np.float32) * 1e-5,          # subnormal fp16 range
        np.array([65504, 65519.99, 65520, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 0.0, -0.0],
                 dtype=np.float32),
    ])
    got = O.f2h(x).view(np.uint16)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_gemm_known_answers_bit_exact():
    """ship_probe.cu inputs: every fp32 partial sum is exact, so the fp16 result is the closed
    form S/64 rounded once; expected bits come from exact integer sums (tests/golden)."""
    gold = json.load(open(GOLD))
    for sh in gold["shapes"]:
        M, N, K = sh["M"], sh["N"], sh["K"]
        A, B = O.ship_probe_inputs(M, N, K)
        rows = sorted({c[0] for c in sh["cells"]})
        Cs = O.gemm_f16(A[rows], B)
        ri = {m: i for i, m in enumerate(rows)}
        for m, n, S, bits in sh["cells"]:
            assert int(Cs.view(np.uint16)[ri[m], n]) == bits, (M, N, K, m, n, S)


def test_gemm_bit_exact_against_numpy_sequential_emulation():
    # fp16*fp16 is exact in fp32, so fp32(acc + a*b) == fmaf(a, b, acc): numpy's float32 ops
    # restate the naive kernel's arithmetic independently of the C code.
    A = O.randn_f16((37, 203), 1, 203 ** -0.5)
    B = O.randn_f16((45, 203), 2, 203 ** -0.5)
    got = O.gemm_f16(A, B)
    Af, Bf = A.astype(np.float32), B.astype(np.float32)
    acc = np.zeros((37, 45), np.float32)
    for k in range(203):
        acc = acc + np.outer(Af[:, k], Bf[:, k]).astype(np.float32)
    assert np.array_equal(got.view(np.uint16), acc.astype(np.float16).view(np.uint16))


def test_gemm_against_fp64_and_operand_order():
    A = O.randn_f16((64, 512), 5, 512 ** -0.5)
    B = O.randn_f16((96, 512), 6, 512 ** -0.5)
    got = O.gemm_f16(A, B)
    ref = A.astype(np.float64) @ B.astype(np.float64).T
    assert O.rel_l2(got, ref.astype(np.float32)) < 1e-3
    # the known operand order: C[m][n] pairs row m of A with row n of B
    assert abs(float(got[3, 7]) - float(ref[3, 7])) < 2e-3
    assert O.rel_l2(O.gemm_f16(B, A).T.copy(), got) == 0.0


def test_dequant_sym_exhaustive_over_q_and_all_scales():
    q = np.arange(-128, 128, dtype=np.int8)
    s_bits = np.arange(0, 0x7c00, dtype=np.uint16)  # every finite non-negative fp16 scale
    s = s_bits.view(np.float16)
    Q = np.broadcast_to(q, (s.size, q.size)).copy()
    got = O.dequant_sym(Q, s)
    ref = (q.astype(np.float32)[None, :] * s.astype(np.float32)[:, None]).astype(np.float16)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))


def test_dequant_asym_exhaustive_over_q_and_z():
    G = 128
    q = np.tile(np.arange(256, dtype=np.uint8), 256).reshape(256, 256)  # row r: all q
    z = np.arange(256, dtype=np.uint8)                                   # row r: z = r
    g = np.random.Generator(np.random.PCG64(9))
    for s_val in list(g.uniform(0.5, 1.5, 6) / 255) + [1.0, 2.0 ** -10, 65504.0 / 512]:
        s16 = np.float16(s_val)
        S = np.full((256, 2), s16, dtype=np.float16)
        Z = np.stack([z, z], axis=1)
        Q = np.concatenate([q, q], axis=1)  # K = 512 -> two groups per row
        got = O.dequant_asym(Q[:, :256], S[:, :2], Z, G=G)
        d = q.astype(np.int32) - z.astype(np.int32)[:, None]
        ref = (d.astype(np.float32) * np.float32(s16)).astype(np.float16)
        assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))


def test_dequant_asym_distinct_scales_per_row_and_group():
    """Every (row, group) gets its own scale and zero-point, so a swapped or shifted metadata
    index changes the result.  Reference: the GPTQ formula of bench/gemm_baseline.py:229,
    W[k, n] = half((q[k, n] - z[k // G, n]) * s[k // G, n]), evaluated here in numpy on the
    reference's k-major storage and transposed to the oracle's [N, K] layout."""
    G, N, K = 128, 48, 1024
    ng = K // G
    g = np.random.Generator(np.random.PCG64(21))
    q_kn = g.integers(0, 256, (K, N), dtype=np.uint8)
    z_gn = g.integers(100, 157, (ng, N), dtype=np.uint8)
    # N * ng distinct fp16 scales in [0.5, 1.5] / 255 (a random draw of distinct bit patterns)
    lo = np.float16(0.5 / 255).view(np.uint16)
    hi = np.float16(1.5 / 255).view(np.uint16)
    bits = g.choice(np.arange(lo, hi + 1, dtype=np.uint16), N * ng, replace=False)
    s_gn = bits.reshape(ng, N).view(np.float16)
    gidx = np.arange(K) // G
    W_kn = ((q_kn.astype(np.float32) - z_gn.astype(np.float32)[gidx])
            * s_gn.astype(np.float32)[gidx]).astype(np.float16)
    got = O.dequant_asym(q_kn.T.copy(), s_gn.T.copy(), z_gn.T.copy(), G=G)
    assert np.array_equal(got.view(np.uint16), W_kn.T.view(np.uint16))
    # sensitivity: the same formula with the metadata of the next group (a shifted index) or of
    # the row's mirror (a transposed index) disagrees almost everywhere
    for perm in (np.roll(np.arange(ng), 1), None):
        if perm is None:
            s_bad, z_bad = s_gn[:, ::-1], z_gn[:, ::-1]
        else:
            s_bad, z_bad = s_gn[perm], z_gn[perm]
        W_bad = ((q_kn.astype(np.float32) - z_bad.astype(np.float32)[gidx])
                 * s_bad.astype(np.float32)[gidx]).astype(np.float16)
        assert np.mean(got.view(np.uint16) != W_bad.T.view(np.uint16)) > 0.9


def test_dequant_invariants():
    g = np.random.Generator(np.random.PCG64(4))
    q = g.integers(0, 256, (8, 256), dtype=np.uint8)
    z = g.integers(0, 256, (8, 2), dtype=np.uint8)
    one = np.ones((8, 2), np.float16)
    W = O.dequant_asym(q, one, z, 128)
    zz = np.repeat(z, 128, axis=1).astype(np.int32)
    assert np.array_equal(W.astype(np.int32), q.astype(np.int32) - zz)   # s = 1 -> q - z
    W0 = O.dequant_asym(np.repeat(z, 128, axis=1), one * np.float16(0.37), z, 128)
    assert not np.any(W0.astype(np.float32))                             # q = z -> 0


def _fmha_fp64(Q, K, V, scale, causal):
    Qd, Kd, Vd = (x.astype(np.float64) for x in (Q, K, V))
    B, Sq, H, D = Q.shape
    Sk, Hkv = K.shape[1], K.shape[2]
    O64 = np.zeros((B, Sq, H, D))
    L64 = np.zeros((B, H, Sq))
    for b in range(B):
        for h in range(H):
            hk = h // (H // Hkv)
            s = scale * Qd[b, :, h, :] @ Kd[b, :, hk, :].T
            if causal:
                i = np.arange(Sq)[:, None]
                j = np.arange(Sk)[None, :]
                s = np.where(j <= i + (Sk - Sq), s, -np.inf)
            mx = s.max(axis=1, keepdims=True)
            p = np.exp(s - mx)
            l = p.sum(axis=1, keepdims=True)
            O64[b, :, h, :] = (p / l) @ Vd[b, :, hk, :]
            L64[b, h, :] = (mx + np.log(l))[:, 0]
    return O64, L64


@pytest.mark.parametrize("Sq,Sk,causal", [(37, 37, True), (24, 40, True), (33, 33, False)])
def test_fmha_against_fp64_brute_force(Sq, Sk, causal):
    B, H, Hkv, D = 2, 4, 2, 32
    Q = O.randn_f16((B, Sq, H, D), 11)
    K = O.randn_f16((B, Sk, Hkv, D), 12)
    V = O.randn_f16((B, Sk, Hkv, D), 13)
    scale = D ** -0.5
    got, lse = O.fmha_fwd(Q, K, V, scale, causal)
    ref, lref = _fmha_fp64(Q, K, V, scale, causal)
    assert O.rel_l2(got, ref.astype(np.float32)) < 1e-3
    assert np.max(np.abs(lse - lref)) < 1e-4


def test_fmha_invariants():
    B, S, H, Hkv, D = 1, 16, 2, 1, 8
    Q = O.randn_f16((B, S, H, D), 21)
    K = O.randn_f16((B, S, Hkv, D), 22)
    V = O.randn_f16((B, S, Hkv, D), 23)
    got, lse = O.fmha_fwd(Q, K, V, 0.5, True)
    # causal row 0 sees only key 0: softmax of one element is 1, output is V[0] exactly
    for h in range(H):
        assert np.array_equal(got[0, 0, h].view(np.uint16), V[0, 0, 0].view(np.uint16))
    # constant keys -> uniform weights over the visible prefix -> running mean of V
    Kc = np.ones_like(K)
    got2, _ = O.fmha_fwd(Q, Kc, V, 0.5, True)
    Vd = V[0, :, 0, :].astype(np.float64)
    mean = np.cumsum(Vd, axis=0) / np.arange(1, S + 1)[:, None]
    assert np.max(np.abs(got2[0, :, 0, :].astype(np.float64) - mean)) < 2e-3
    # every query head of a GQA group reads the same KV head: heads 0 and 1 share KV head 0
    Qs = np.repeat(Q[:, :, :1, :], 2, axis=2)
    got3, _ = O.fmha_fwd(Qs, K, V, 0.5, True)
    assert np.array_equal(got3[:, :, 0].view(np.uint16), got3[:, :, 1].view(np.uint16))


def test_rel_l2_closed_forms():
    x = O.randn_f16((1000,), 1)
    assert O.rel_l2(x, x) == 0.0
    assert O.rel_l2(np.zeros_like(x), x) == pytest.approx(1.0)
    assert O.rel_l2((x.astype(np.float32) * 2).astype(np.float16), x) == pytest.approx(1.0)


def test_poison_and_spot():
    C = np.full((4, 4), 0x7f7f, np.uint16)
    assert O.count_poison(C) == 16
    A, B = O.ship_probe_inputs(8, 16, 64)
    Cm = O.gemm_f16(A, B)
    worst, bad = O.spot_fp64(A, B, Cm, cells=64)
    assert bad == 0 and worst < 1e-3
    Cm2 = Cm.copy()
    Cm2[0, 0] = np.float16(float(Cm2[0, 0]) + 1.0)  # one wrong cell is seen by the spot check
    worst2, bad2 = O.spot_fp64(A, B, Cm2, cells=64)
    assert bad2 >= 1


def _gptq_checkpoint(K, N, G, seed):
    """Random GPTQ int8 tensors over the full int32 range, as bench/gemm_baseline.py:219-223."""
    g = np.random.Generator(np.random.PCG64(seed))
    qw = g.integers(-(2**31), 2**31 - 1, (K // 4, N), dtype=np.int64).astype(np.int32)
    qz = g.integers(-(2**31), 2**31 - 1, (K // G, N // 4), dtype=np.int64).astype(np.int32)
    sc = O.f2h(g.uniform(0.001, 0.021, (K // G, N)).astype(np.float32))
    return qw, qz, sc


def test_gptq_unpack_against_python_brute_force():
    """Byte k%4 of qweight[k/4][n] and byte n%4 of qzeros[g][n/4], read with Python's arbitrary
    precision ints (arithmetic shift of the signed word, then & 0xFF, as the reference's torch
    expression does on int32)."""
    K, N, G = 256, 12, 128
    qw, qz, sc = _gptq_checkpoint(K, N, G, 3)
    q, z, s = O.gptq_unpack(qw, qz, sc, G)
    for k in range(K):
        for n in range(N):
            assert q[k, n] == (int(qw[k // 4, n]) >> (8 * (k % 4))) & 0xFF
    for gi in range(K // G):
        for n in range(N):
            assert z[gi, n] == (int(qz[gi, n // 4]) >> (8 * (n % 4))) & 0xFF
    assert np.array_equal(s.view(np.uint16), sc.view(np.uint16))


def test_gptq_pack_unpack_round_trip():
    """An independent packer (little-endian bytes via numpy views) inverts the unpack."""
    K, N, G = 512, 64, 128
    g = np.random.Generator(np.random.PCG64(8))
    q = g.integers(0, 256, (K, N), dtype=np.int16).astype(np.uint8)
    z = g.integers(0, 256, (K // G, N), dtype=np.int16).astype(np.uint8)
    qw = np.ascontiguousarray(q.reshape(K // 4, 4, N).transpose(0, 2, 1)).view("<i4")[..., 0]
    qz = np.ascontiguousarray(z.reshape(K // G, N // 4, 4)).view("<i4")[..., 0]
    sc = O.f2h(np.full((K // G, N), 0.01, np.float32))
    q2, z2, _ = O.gptq_unpack(qw, qz, sc, G)
    assert np.array_equal(q2, q) and np.array_equal(z2, z)
    wq, s_nk, z_nk = O.gptq_to_nk(qw, qz, sc, G)
    assert wq.shape == (N, K) and np.array_equal(wq, q.T)
    assert s_nk.shape == (N, K // G) and np.array_equal(z_nk, z.T)


def test_gptq_dense_against_reference_formula():
    """W[k][n] = half((q - z[k/G]) * s[k/G]) (gemm_baseline.py:229); (q - z) * s has at most
    9 + 11 significant bits, so the fp64 product is exact and one rounding to fp16 is the whole
    answer."""
    K, N, G = 384, 16, 128
    qw, qz, sc = _gptq_checkpoint(K, N, G, 11)
    W = O.gptq_dense(qw, qz, sc, G)
    assert W.shape == (K, N)
    ref = np.empty((K, N), np.float16)
    for k in range(K):
        for n in range(N):
            q = (int(qw[k // 4, n]) >> (8 * (k % 4))) & 0xFF
            z = (int(qz[k // G, n // 4]) >> (8 * (n % 4))) & 0xFF
            ref[k, n] = np.float16(float(q - z) * float(sc[k // G, n]))
    assert np.array_equal(W.view(np.uint16), ref.view(np.uint16))


def test_silu_mul_against_scipy_expit():
    """silu(g) = g * expit(g) with scipy's logistic function, independent of the oracle's
    formula; both rounded once to fp16: at most one unit in the last place apart (ties)."""
    from scipy.special import expit

    g = np.random.Generator(np.random.PCG64(4))
    G = O.f2h((g.standard_normal(20000) * 4).astype(np.float32))
    U = O.f2h(g.standard_normal(20000).astype(np.float32))
    got = O.silu_mul(G, U)
    ref = (G.astype(np.float64) * expit(G.astype(np.float64)) * U.astype(np.float64)).astype(np.float16)
    d = np.abs(got.view(np.int16).astype(np.int32) - ref.view(np.int16).astype(np.int32))
    assert d.max() <= 1 and (d == 0).mean() > 0.999


def test_silu_mul_closed_forms():
    one = np.ones(5, np.float16)
    assert not np.any(O.silu_mul(np.zeros(5, np.float16), one).astype(np.float32))
    big = np.array([12.0, 20.0, 100.0, 1000.0, 60000.0], np.float16)
    assert np.array_equal(O.silu_mul(big, one), big)            # sigmoid -> 1
    neg = -big
    assert np.all(np.abs(O.silu_mul(neg, one).astype(np.float32)) < 1e-3)   # -> 0
    x = O.f2h(np.linspace(-6, 6, 97).astype(np.float32))
    odd = O.silu_mul(x, np.ones_like(x)).astype(np.float64) - O.silu_mul(-x, np.ones_like(x)).astype(np.float64)
    assert np.max(np.abs(odd - x.astype(np.float64))) <= 8e-3   # silu(x) - silu(-x) = x
    # u scales the result: u = 2 doubles it exactly (a power of two)
    assert np.array_equal(O.silu_mul(x, np.full_like(x, 2)).astype(np.float32),
                          2 * O.silu_mul(x, np.ones_like(x)).astype(np.float32))


def test_gate_up_oracle_splits_rows_gate_then_up():
    """Rows [0, N) are the gate, [N, 2N) the up: swapping the halves changes the result, and a
    B whose up half is the identity's rows gives silu(gate) * A."""
    g = np.random.Generator(np.random.PCG64(9))
    M, N, K = 3, 8, 8
    A = O.f2h(g.standard_normal((M, K)).astype(np.float32))
    Bg = O.f2h(g.standard_normal((N, K)).astype(np.float32))
    Bu = np.eye(N, K, dtype=np.float16)
    C = O.gemm_gate_up_f16(A, np.concatenate([Bg, Bu]))
    Gm = O.gemm_f16(A, Bg)
    assert np.array_equal(C, O.silu_mul(Gm, A[:, :N]))
    C2 = O.gemm_gate_up_f16(A, np.concatenate([Bu, Bg]))
    assert not np.array_equal(C, C2)
