"""numpy front end of the C oracle (tempo_oracle.c) -- TEST INFRASTRUCTURE ONLY.

Every array crossing into C is made contiguous first; fp16 data travels as uint16 bit patterns,
so no numpy rounding sits between the caller and the C restatement.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

_p = C.c_void_p
_i = C.c_int
_l = C.c_long
_f = C.c_float
_d = C.c_double


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            from . import build as _b

            _b.build()
        L = C.CDLL(path)
        L.oracle_h2f.argtypes = [C.c_uint16]
        L.oracle_h2f.restype = _f
        L.oracle_f2h.argtypes = [_f]
        L.oracle_f2h.restype = C.c_uint16
        L.oracle_h2f_array.argtypes = [_p, _p, _l]
        L.oracle_f2h_array.argtypes = [_p, _p, _l]
        L.oracle_check_f2h_exhaustive.argtypes = [_i]
        L.oracle_check_f2h_exhaustive.restype = _l
        L.oracle_gemm_f16.argtypes = [_p, _p, _p, _i, _i, _i, _l, _l, _l, _i]
        L.oracle_dequant_sym.argtypes = [_p, _p, _p, _i, _i, _l, _l]
        L.oracle_dequant_asym.argtypes = [_p, _p, _p, _p, _i, _i, _i, _l, _l]
        L.oracle_gemm_w8a16.argtypes = [_p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i]
        L.oracle_fmha_fwd.argtypes = [_p, _p, _p, _p, _p] + [_i] * 6 + [_f, _i] + [_l] * 12 + [_p, _i, _i]
        L.oracle_rel_l2_f16.argtypes = [_p, _p, _l]
        L.oracle_rel_l2_f16.restype = _d
        L.oracle_rel_l2_f16_f32.argtypes = [_p, _p, _l]
        L.oracle_rel_l2_f16_f32.restype = _d
        L.oracle_count_poison.argtypes = [_p, _l]
        L.oracle_count_poison.restype = _l
        L.oracle_spot_fp64.argtypes = [_p, _p, _p, _i, _i, _i, _i, _d, C.POINTER(_i)]
        L.oracle_spot_fp64.restype = _d
        _LIB = L
    return _LIB


def _bits(a) -> np.ndarray:
    """fp16 array (float16 or uint16 bit patterns) -> contiguous uint16 view."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16:
        return a.view(np.uint16)
    if a.dtype != np.uint16:
        raise TypeError("expected float16 or uint16 bit patterns, got %s" % a.dtype)
    return a


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(_p)


def h2f(h) -> np.ndarray:
    h = _bits(h)
    out = np.empty(h.shape, np.float32)
    lib().oracle_h2f_array(_ptr(h), _ptr(out), h.size)
    return out


def f2h(f) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().oracle_f2h_array(_ptr(f), _ptr(out), f.size)
    return out.view(np.float16)


def check_f2h_exhaustive(threads: int = 0) -> int:
    return int(lib().oracle_check_f2h_exhaustive(threads))


def gemm_f16(A, B, threads: int = 0) -> np.ndarray:
    """C = fp16_rn(A . B^T), A [M,K], B [N,K] fp16; the naive kernel's exact arithmetic."""
    A = _bits(A)
    B = _bits(B)
    M, K = A.shape
    N, K2 = B.shape
    if K != K2:
        raise ValueError("K mismatch %d vs %d" % (K, K2))
    Cm = np.empty((M, N), np.uint16)
    lib().oracle_gemm_f16(_ptr(A), _ptr(B), _ptr(Cm), M, N, K, K, K, N, threads)
    return Cm.view(np.float16)


def dequant_sym(q, s) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.int8)
    s = _bits(s)
    N, K = q.shape
    W = np.empty((N, K), np.uint16)
    lib().oracle_dequant_sym(_ptr(q), _ptr(s), _ptr(W), N, K, K, K)
    return W.view(np.float16)


def dequant_asym(q, s, z, G: int = 128) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    s = _bits(s)
    z = np.ascontiguousarray(z, dtype=np.uint8)
    N, K = q.shape
    if K % G or s.shape != (N, K // G) or z.shape != (N, K // G):
        raise ValueError("bad group shapes")
    W = np.empty((N, K), np.uint16)
    lib().oracle_dequant_asym(_ptr(q), _ptr(s), _ptr(z), _ptr(W), N, K, G, K, K)
    return W.view(np.float16)


def gemm_w8a16(A, q, s, z=None, G: int = 0, fmt: int = 1, threads: int = 0) -> np.ndarray:
    A = _bits(A)
    M, K = A.shape
    if fmt == 1:
        q = np.ascontiguousarray(q, dtype=np.int8)
        zp = None
    else:
        q = np.ascontiguousarray(q, dtype=np.uint8)
        z = np.ascontiguousarray(z, dtype=np.uint8)
        zp = _ptr(z)
    s = _bits(s)
    N = q.shape[0]
    Cm = np.empty((M, N), np.uint16)
    lib().oracle_gemm_w8a16(_ptr(A), _ptr(q), _ptr(s), zp, _ptr(Cm), M, N, K, G, fmt, threads)
    return Cm.view(np.float16)


def fmha_fwd(Q, K, V, scale: float, causal: bool = True, rows=None, threads: int = 0):
    """Q [B,Sq,H,D], K/V [B,Sk,Hkv,D] (BSHD, contiguous) -> (O [B,Sq,H,D] fp16, LSE [B,H,Sq]).

    With `rows`, only those query rows are computed (others stay zero / NaN)."""
    Q, K, V = _bits(Q), _bits(K), _bits(V)
    B, Sq, H, D = Q.shape
    _, Sk, Hkv, _ = K.shape
    O = np.zeros(Q.shape, np.uint16)
    L = np.full((B, H, Sq), np.nan, np.float32)
    r = None
    nr = 0
    if rows is not None:
        r = np.ascontiguousarray(rows, dtype=np.int32)
        nr = r.size
    lib().oracle_fmha_fwd(
        _ptr(Q), _ptr(K), _ptr(V), _ptr(O), _ptr(L), B, H, Hkv, Sq, Sk, D, float(scale),
        int(bool(causal)),
        Sq * H * D, H * D, D, Sk * Hkv * D, Hkv * D, D, Sk * Hkv * D, Hkv * D, D,
        Sq * H * D, H * D, D,
        _ptr(r) if r is not None else None, nr, threads,
    )
    return O.view(np.float16), L


def rel_l2(got, ref) -> float:
    """tempo/core/op/oracle.py:114-124 with double accumulation; ref may be fp16 or fp32."""
    got = _bits(got)
    ref = np.ascontiguousarray(ref)
    if ref.dtype == np.float32:
        return float(lib().oracle_rel_l2_f16_f32(_ptr(got), _ptr(ref), got.size))
    ref = _bits(ref)
    return float(lib().oracle_rel_l2_f16(_ptr(got), _ptr(ref), got.size))


def count_poison(Cm) -> int:
    Cm = _bits(Cm)
    return int(lib().oracle_count_poison(_ptr(Cm), Cm.size))


def spot_fp64(A, B, Cm, cells: int = 64, tol: float = 3e-3):
    """ship_probe.cu:70-79: returns (max rel, number of cells above tol)."""
    A, B, Cm = _bits(A), _bits(B), _bits(Cm)
    M, K = A.shape
    N = B.shape[0]
    nb = C.c_int(0)
    worst = lib().oracle_spot_fp64(_ptr(A), _ptr(B), _ptr(Cm), M, N, K, cells, tol, C.byref(nb))
    return float(worst), int(nb.value)


# -- seeded synthetic inputs (numpy PCG64, generated in fp32, RNE to fp16) --
def randn_f16(shape, seed: int, scale: float = 1.0) -> np.ndarray:
    g = np.random.Generator(np.random.PCG64(seed))
    x = g.standard_normal(size=shape, dtype=np.float32) * np.float32(scale)
    return f2h(x)


def ship_probe_inputs(M: int, N: int, K: int):
    """ship_probe.cu:54-55 known-answer inputs: A[i] = ((i%7)-3)/8, B[i] = ((i%5)-2)/8."""
    ia = np.arange(M * K, dtype=np.int64)
    ib = np.arange(N * K, dtype=np.int64)
    A = (((ia % 7) - 3).astype(np.float32) * np.float32(0.125)).astype(np.float16).reshape(M, K)
    B = (((ib % 5) - 2).astype(np.float32) * np.float32(0.125)).astype(np.float16).reshape(N, K)
    return A, B


def gptq_unpack(qweight, qzeros, scales, G: int = 128):
    """GPTQ int8 checkpoint (bench/gemm_baseline.py:214-232): qweight int32 [K/4,N], qzeros int32
    [K/G,N/4], scales fp16 [K/G,N] -> q uint8 [K,N], z uint8 [K/G,N], s fp16 [K/G,N]."""
    qw = np.ascontiguousarray(qweight).view(np.uint32)
    qz = np.ascontiguousarray(qzeros).view(np.uint32)
    K4, N = qw.shape
    q = np.stack([(qw >> (8 * b)) & 0xFF for b in range(4)], axis=1).reshape(K4 * 4, N)
    z = np.stack([(qz >> (8 * b)) & 0xFF for b in range(4)], axis=2).reshape(qz.shape[0], N)
    return q.astype(np.uint8), z.astype(np.uint8), np.ascontiguousarray(scales).view(np.float16)


def gptq_to_nk(qweight, qzeros, scales, G: int = 128):
    """The fmt 2 operands of gemm_w8a16 for a GPTQ checkpoint: (wq [N,K], s [N,K/G], z [N,K/G])."""
    q, z, s = gptq_unpack(qweight, qzeros, scales, G)
    return (np.ascontiguousarray(q.T), np.ascontiguousarray(s.T), np.ascontiguousarray(z.T))


def gptq_dense(qweight, qzeros, scales, G: int = 128):
    """W [K,N] fp16 = fp16_rn((q - z[k/G]) * s[k/G]) -- gemm_baseline.py:229."""
    wq, s, z = gptq_to_nk(qweight, qzeros, scales, G)
    return np.ascontiguousarray(dequant_asym(wq, s, z, G).T)


def silu_mul(g, u) -> np.ndarray:
    """The fused gate/up epilogue on fp16 GEMM results: fp16_rn(silu(g) * u), silu(x) =
    x / (1 + e^-x), evaluated in fp64 (one rounding).  The reference names this fusion without
    shipping it (docs/NOT_YET.md:141-146); its unfused form is F.silu(g) * u on the two fp16
    outputs."""
    g = np.asarray(g, np.float16).astype(np.float64)
    u = np.asarray(u, np.float16).astype(np.float64)
    with np.errstate(over="ignore"):
        return (g / (1.0 + np.exp(-g)) * u).astype(np.float16)


def gemm_gate_up_f16(A, B, threads: int = 0) -> np.ndarray:
    """C [M,N] = silu_mul(A.B[:N]^T, A.B[N:]^T) for B [2N,K] (gate rows, then up rows)."""
    N = B.shape[0] // 2
    return silu_mul(gemm_f16(A, B[:N], threads), gemm_f16(A, B[N:], threads))


def gemm_gate_up_w8a16(A, q, s, z=None, G: int = 0, fmt: int = 1, threads: int = 0) -> np.ndarray:
    """The fused gate/up GEMM on 8-bit weights [2N,K] (scale / zero rows follow the weights)."""
    N = q.shape[0] // 2
    sg, su = (s[:N], s[N:])
    zg, zu = (z[:N], z[N:]) if z is not None else (None, None)
    return silu_mul(gemm_w8a16(A, q[:N], sg, zg, G, fmt, threads),
                    gemm_w8a16(A, q[N:], su, zu, G, fmt, threads))
