"""ctypes binding of libtempo_gfx950.so (C ABI: include/tempo_gfx950.h).

This is the binding a Python host tree would add (the reference's hot path crosses into native
code through a POD launcher, kernels/shipped/gemm_fp16/sm_70/launch.cuh:20-75; its host binding
is a template in INTEGRATION.md:83-97).  Device memory and streams come from PyTorch-ROCm
tensors; only raw pointers cross the boundary.

There is no CPU fallback anywhere in this module: if the library is missing, lib() raises.
"""
from __future__ import annotations

import ctypes as ct
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtempo_gfx950.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "tempo_gfx950.h")

TEMPO_OK = 0
TEMPO_FALLBACK = 9  # hipErrorInvalidConfiguration: "not covered, take your own path"
W8_SYM_I8 = 1
W8_ASYM_U8 = 2

_p = ct.c_void_p
_i = ct.c_int
_l = ct.c_long


class TempoGemmParams(ct.Structure):
    _fields_ = [("A", _p), ("B", _p), ("C", _p), ("M", _i), ("N", _i), ("K", _i),
                ("lda", _i), ("ldb", _i), ("ldc", _i)]


class TempoW8A16Params(ct.Structure):
    _fields_ = [("A", _p), ("Wq", _p), ("scale", _p), ("zero", _p), ("C", _p),
                ("M", _i), ("N", _i), ("K", _i), ("lda", _i), ("ldw", _i), ("ldc", _i),
                ("group", _i), ("fmt", _i)]


class TempoFmhaParams(ct.Structure):
    _fields_ = [("Q", _p), ("K", _p), ("V", _p), ("O", _p), ("LSE", _p),
                ("B", _i), ("H", _i), ("Hkv", _i), ("Sq", _i), ("Sk", _i), ("D", _i),
                ("scale", ct.c_float), ("causal", _i)] + [
                   (n, _l) for n in ("q_sb", "q_ss", "q_sh", "k_sb", "k_ss", "k_sh",
                                     "v_sb", "v_ss", "v_sh", "o_sb", "o_ss", "o_sh")]


class TempoError(RuntimeError):
    def __init__(self, code: int, what: str):
        super().__init__("%s failed with hipError %d" % (what, code))
        self.code = code


class NotCovered(TempoError):
    """The shipped ladder does not cover this shape: the caller takes its own path."""


_LIB = None

EXPORTS = {
    "tempo_abi_version": ([], _i),
    "tempo_gemm_fp16_applicable": ([ct.POINTER(TempoGemmParams)], _i),
    "tempo_gemm_fp16_launch": ([ct.POINTER(TempoGemmParams), _p], _i),
    "tempo_gemm_w8a16_applicable": ([ct.POINTER(TempoW8A16Params)], _i),
    "tempo_gemm_w8a16_launch": ([ct.POINTER(TempoW8A16Params), _p], _i),
    "tempo_dequant_tile": ([ct.POINTER(TempoW8A16Params), _i, _i, _i, _i, _p, _p], _i),
    "tempo_fmha_fwd_applicable": ([ct.POINTER(TempoFmhaParams)], _i),
    "tempo_fmha_fwd_launch": ([ct.POINTER(TempoFmhaParams), _p], _i),
    "tempo_naive_gemm_fp16_launch": ([_p, _p, _p, _i, _i, _i, _p], _i),
    "tempo_probe_mfma_layout": ([_i, _p, _p], _i),
    "tempo_route": ([_i, _i, _i, _i, ct.c_char_p, _i], _i),
    "tempo_gemm_fp16_gate_up_launch": ([ct.POINTER(TempoGemmParams), _p], _i),
    "tempo_gemm_w8a16_gate_up_launch": ([ct.POINTER(TempoW8A16Params), _p], _i),
    "tempo_naive_gemm_w8a16_launch": ([ct.POINTER(TempoW8A16Params), _p], _i),
    "tempo_naive_fmha_fwd_launch": ([_p, _p, _p, _p, _p] + [_i] * 6 + [ct.c_float, _i, _p], _i),
    "tempo_gptq_repack_u8": ([_p, _p, _p, _i, _i, _i, _p, _p, _p, _p], _i),
    "tempo_gemm_fp16_workspace_bytes": ([ct.POINTER(TempoGemmParams)], ct.c_size_t),
    "tempo_gemm_w8a16_workspace_bytes": ([ct.POINTER(TempoW8A16Params)], ct.c_size_t),
    "tempo_gemm_w8a16_launch_noalloc": ([ct.POINTER(TempoW8A16Params), _p], _i),
    "tempo_gemm_fp16_launch_ws": ([ct.POINTER(TempoGemmParams), _p, ct.c_size_t, _p], _i),
    "tempo_gemm_w8a16_launch_ws": ([ct.POINTER(TempoW8A16Params), _p, ct.c_size_t, _p], _i),
}
HIP_ERROR_CAPTURE_UNSUPPORTED = 900  # hipErrorStreamCaptureUnsupported: the pool cannot grow
NOALLOC_SCRATCH_BYTES = 32 << 20


def lib():
    """Load the library; raises if it was not built (the product path has no fallback)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                "libtempo_gfx950.so is not built (%s); run `python3 -m cuda_tempiler_amd.build`"
                % LIB_PATH)
        L = ct.CDLL(LIB_PATH)
        for name, (args, res) in EXPORTS.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = res
        _LIB = L
    return _LIB


def _check(rc: int, what: str) -> None:
    if rc == TEMPO_FALLBACK:
        raise NotCovered(rc, what)
    if rc != TEMPO_OK:
        raise TempoError(rc, what)


def _stream(stream):
    if stream is None:
        import torch

        return _p(torch.cuda.current_stream().cuda_stream)
    if isinstance(stream, int):
        return _p(stream)
    return _p(stream.cuda_stream)


def workspace_bytes(op: int, M: int, N: int, K: int) -> int:
    """Host-only: workspace bytes the shipped row for this shape needs (0 = none / not covered).
    op 0 = gemm_fp16, 1 / 2 = gemm_w8a16 fmt 1 / 2 (dense strides)."""
    fake = _p(0x1000)
    if op == 0:
        return int(lib().tempo_gemm_fp16_workspace_bytes(
            TempoGemmParams(fake, fake, fake, M, N, K, K, K, N)))
    return int(lib().tempo_gemm_w8a16_workspace_bytes(
        TempoW8A16Params(fake, fake, fake, fake if op == 2 else None, fake, M, N, K, K, K, N,
                         128 if op == 2 else 0, op)))


def route(op: int, M: int, N: int, K: int) -> str:
    """Host-only: ladder row the shipped dispatcher picks ('' = not covered)."""
    buf = ct.create_string_buffer(64)
    lib().tempo_route(op, M, N, K, buf, 64)
    return buf.value.decode()


# ---- torch-facing helpers (torch is plumbing: device memory and streams) ------------------
def _ptr(t):
    return _p(t.data_ptr()) if t is not None else None


def _require_out(C, M, N, A, what):
    """C must be fp16 [M, N] with unit inner stride on A's device: the kernels write it as raw
    memory of that layout."""
    import torch

    if C.dtype != torch.float16 or C.dim() != 2 or tuple(C.shape) != (M, N) \
            or C.stride(1) != 1 or C.device != A.device:
        raise ValueError("%s: C must be fp16 [%d, %d] with unit inner stride on %s, got %s %s "
                         "strides %s on %s" % (what, M, N, A.device, C.dtype, tuple(C.shape),
                                               tuple(C.stride()), C.device))


def _launch(name, name_ws, p, need_fn, workspace, device, stream):
    """Run a GEMM entry point.  workspace=None: the library's pool (tempo_*_launch); "torch": a
    workspace from torch's caching allocator when the row needs one (graph-capture safe: under
    capture torch hands out memory of the graph's pool); a tensor: that device memory."""
    L = lib()
    if workspace is None:
        _check(getattr(L, name)(p, _stream(stream)), name)
        return
    if isinstance(workspace, str):
        if workspace != "torch":
            raise ValueError("workspace must be None, 'torch' or a device tensor")
        import torch

        need = int(need_fn(p))
        buf = torch.empty(need, dtype=torch.uint8, device=device) if need else None
    else:
        buf = workspace
    nbytes = 0 if buf is None else buf.numel() * buf.element_size()
    _check(getattr(L, name_ws)(p, _ptr(buf), nbytes, _stream(stream)), name_ws)


def gemm_fp16(A, B, C=None, stream=None, workspace=None):
    """C[M,N] = A[M,K] . B[N,K]^T on the shipped gfx950 ladder.  Raises NotCovered.  `workspace`
    as for _launch (None = the library's pool)."""
    import torch

    M, K = A.shape
    N = B.shape[0]
    if C is None:
        C = torch.empty((M, N), dtype=torch.float16, device=A.device)
    p = TempoGemmParams(_ptr(A), _ptr(B), _ptr(C), M, N, K, A.stride(0), B.stride(0), C.stride(0))
    _launch("tempo_gemm_fp16_launch", "tempo_gemm_fp16_launch_ws", p,
            lib().tempo_gemm_fp16_workspace_bytes, workspace, A.device, stream)
    return C


def gemm_fp16_gate_up(A, B, C=None, stream=None):
    """C[M,N] = silu(A.B[:N]^T) * (A.B[N:]^T) for B [2N, K] (gate rows, then up rows)."""
    import torch

    M, K = A.shape
    N = B.shape[0] // 2
    if C is None:
        C = torch.empty((M, N), dtype=torch.float16, device=A.device)
    p = TempoGemmParams(_ptr(A), _ptr(B), _ptr(C), M, N, K, A.stride(0), B.stride(0), C.stride(0))
    _check(lib().tempo_gemm_fp16_gate_up_launch(p, _stream(stream)),
           "tempo_gemm_fp16_gate_up_launch")
    return C


def gemm_w8a16_gate_up(A, Wq, scale, zero=None, fmt: int = W8_SYM_I8, group: int = 128, C=None,
                       stream=None):
    """The fused gate/up GEMM on 8-bit weights: Wq [2N, K] (and its scale / zero rows)."""
    import torch

    M = A.shape[0]
    N = Wq.shape[0] // 2
    _require_w8(A, Wq, scale, zero, fmt, group)
    if C is None:
        C = torch.empty((M, N), dtype=torch.float16, device=A.device)
    _require_out(C, M, N, A, "gemm_w8a16_gate_up")
    p = w8a16_params(A, Wq, scale, zero, C, fmt, group)
    p.N = N
    _check(lib().tempo_gemm_w8a16_gate_up_launch(p, _stream(stream)),
           "tempo_gemm_w8a16_gate_up_launch")
    return C


def w8a16_operand_error(A, Wq, scale, zero, fmt: int, group: int = 128, rows=None):
    """Why these tensors are not a well-formed W8A16 operand set (None if they are).

    The kernels read the weight bytes, scales and zero-points as raw memory of the declared
    layout, so a wrong dtype or shape would be read as something else (or past its end):
      A     fp16 [M, K], unit inner stride
      Wq    [rows, K], unit inner stride: int8 for fmt 1, uint8 for fmt 2
      scale fp16, contiguous: [rows] for fmt 1, [rows, K/group] for fmt 2
      zero  None for fmt 1; uint8 [rows, K/group], contiguous, for fmt 2
    `rows` defaults to Wq.shape[0] (the gate/up weight has 2N rows and so does its metadata).
    """
    import torch

    if fmt not in (W8_SYM_I8, W8_ASYM_U8):
        return "fmt %r is neither 1 (int8 symmetric) nor 2 (uint8 asymmetric)" % (fmt,)
    if A.dtype != torch.float16 or A.dim() != 2 or A.stride(1) != 1:
        return "A must be fp16 [M, K] with unit inner stride"
    if Wq.dim() != 2 or Wq.stride(1) != 1 or Wq.shape[1] != A.shape[1]:
        return "Wq must be [N, K] with unit inner stride and the K of A"
    want = torch.int8 if fmt == W8_SYM_I8 else torch.uint8
    if Wq.dtype != want:
        return "fmt %d takes %s weights, got %s" % (fmt, want, Wq.dtype)
    rows = Wq.shape[0] if rows is None else rows
    K = A.shape[1]
    if scale is None or scale.dtype != torch.float16 or not scale.is_contiguous():
        return "scale must be a contiguous fp16 tensor"
    if fmt == W8_SYM_I8:
        if tuple(scale.shape) != (rows,):
            return "fmt 1 scale must be [%d], got %s" % (rows, tuple(scale.shape))
        if zero is not None:
            return "fmt 1 takes no zero-points"
        return None
    if group <= 0 or K % group:
        return "K = %d is not a whole number of groups of %d" % (K, group)
    meta = (rows, K // group)
    if tuple(scale.shape) != meta:
        return "fmt 2 scale must be %s, got %s" % (meta, tuple(scale.shape))
    if zero is None or zero.dtype != torch.uint8 or not zero.is_contiguous() \
            or tuple(zero.shape) != meta:
        return "fmt 2 zero must be a contiguous uint8 tensor of shape %s" % (meta,)
    return None


def _require_w8(A, Wq, scale, zero, fmt, group, rows=None):
    why = w8a16_operand_error(A, Wq, scale, zero, fmt, group, rows)
    if why:
        raise ValueError("W8A16 operands: " + why)


def w8a16_params(A, Wq, scale, zero, C, fmt: int, group: int = 128) -> TempoW8A16Params:
    M, K = A.shape
    N = Wq.shape[0]
    return TempoW8A16Params(_ptr(A), _ptr(Wq), _ptr(scale), _ptr(zero), _ptr(C), M, N, K,
                            A.stride(0), Wq.stride(0), C.stride(0) if C is not None else N,
                            group if fmt == W8_ASYM_U8 else 0, fmt)


def gemm_w8a16(A, Wq, scale, zero=None, fmt: int = W8_SYM_I8, group: int = 128, C=None,
               stream=None, workspace=None):
    """C[M,N] = A . deq(Wq)^T on the shipped ladder; `workspace` as for gemm_fp16."""
    import torch

    M = A.shape[0]
    N = Wq.shape[0]
    _require_w8(A, Wq, scale, zero, fmt, group)
    if C is None:
        C = torch.empty((M, N), dtype=torch.float16, device=A.device)
    _require_out(C, M, N, A, "gemm_w8a16")
    p = w8a16_params(A, Wq, scale, zero, C, fmt, group)
    _launch("tempo_gemm_w8a16_launch", "tempo_gemm_w8a16_launch_ws", p,
            lib().tempo_gemm_w8a16_workspace_bytes, workspace, A.device, stream)
    return C


def gemm_w8a16_noalloc(A, Wq, scale, zero=None, fmt: int = W8_SYM_I8, group: int = 128, C=None,
                       stream=None):
    """gemm_w8a16 through the allocation-free entry point (the library's static per-GPU scratch
    serves split-K rows); C must be given (this helper allocates nothing either)."""
    if C is None:
        raise ValueError("gemm_w8a16_noalloc writes into a caller-provided C")
    _require_w8(A, Wq, scale, zero, fmt, group)
    _require_out(C, A.shape[0], Wq.shape[0], A, "gemm_w8a16_noalloc")
    p = w8a16_params(A, Wq, scale, zero, C, fmt, group)
    _check(lib().tempo_gemm_w8a16_launch_noalloc(p, _stream(stream)),
           "tempo_gemm_w8a16_launch_noalloc")
    return C


def dequant_tile(Wq, scale, zero, fmt, n0, k0, rows, cols, group=128, stream=None):
    import torch

    N, K = Wq.shape
    dummyA = torch.empty((1, K), dtype=torch.float16, device=Wq.device)
    out = torch.empty((rows, cols), dtype=torch.float16, device=Wq.device)
    p = w8a16_params(dummyA, Wq, scale, zero, out, fmt, group)
    p.C = _ptr(out)
    p.ldc = max(N, 8)
    _check(lib().tempo_dequant_tile(p, n0, k0, rows, cols, _ptr(out), _stream(stream)),
           "tempo_dequant_tile")
    return out


def fmha_params(Q, K, V, O, LSE, scale: float, causal: bool = True) -> TempoFmhaParams:
    """Q/O [B,Sq,H,D], K/V [B,Sk,Hkv,D] tensors (any strides with d contiguous)."""
    B, Sq, H, D = Q.shape
    _, Sk, Hkv, _ = K.shape
    return TempoFmhaParams(
        _ptr(Q), _ptr(K), _ptr(V), _ptr(O), _ptr(LSE), B, H, Hkv, Sq, Sk, D, float(scale),
        int(bool(causal)),
        Q.stride(0), Q.stride(1), Q.stride(2), K.stride(0), K.stride(1), K.stride(2),
        V.stride(0), V.stride(1), V.stride(2), O.stride(0), O.stride(1), O.stride(2))


def fmha_fwd(Q, K, V, scale: float, causal: bool = True, O=None, LSE=None, stream=None):
    import torch

    B, Sq, H, D = Q.shape
    if O is None:
        O = torch.empty_like(Q)
    if LSE is None:
        LSE = torch.empty((B, H, Sq), dtype=torch.float32, device=Q.device)
    p = fmha_params(Q, K, V, O, LSE, scale, causal)
    _check(lib().tempo_fmha_fwd_launch(p, _stream(stream)), "tempo_fmha_fwd_launch")
    return O, LSE


def naive_gemm_fp16(A, B, C=None, stream=None):
    import torch

    M, K = A.shape
    N = B.shape[0]
    if C is None:
        C = torch.empty((M, N), dtype=torch.float16, device=A.device)
    _check(lib().tempo_naive_gemm_fp16_launch(_ptr(A), _ptr(B), _ptr(C), M, N, K,
                                               _stream(stream)), "tempo_naive_gemm_fp16_launch")
    return C


def naive_fmha_fwd(Q, K, V, scale: float, causal: bool = True, stream=None):
    """The naive attention input kernel on dense BSHD tensors: Q [B,Sq,H,D], K/V [B,Sk,Hkv,D]
    -> (O [B,Sq,H,D] fp16, LSE [B,H,Sq] fp32)."""
    import torch

    for t in (Q, K, V):
        if t.dtype != torch.float16 or not t.is_contiguous() or t.dim() != 4:
            raise ValueError("naive_fmha_fwd takes contiguous fp16 [B, S, heads, D] tensors")
    B, Sq, H, D = Q.shape
    Sk, Hkv = K.shape[1], K.shape[2]
    if tuple(K.shape) != (B, Sk, Hkv, D) or tuple(V.shape) != tuple(K.shape):
        raise ValueError("K and V must be [B, Sk, Hkv, D] with Q's B and D")
    O = torch.empty_like(Q)
    LSE = torch.empty((B, H, Sq), dtype=torch.float32, device=Q.device)
    _check(lib().tempo_naive_fmha_fwd_launch(_ptr(Q), _ptr(K), _ptr(V), _ptr(O), _ptr(LSE), B, H,
                                             Hkv, Sq, Sk, D, float(scale), int(bool(causal)),
                                             _stream(stream)), "tempo_naive_fmha_fwd_launch")
    return O, LSE


def naive_gemm_w8a16(A, Wq, scale, zero=None, fmt: int = W8_SYM_I8, group: int = 128, C=None,
                     stream=None):
    """The naive W8A16 input kernel (one thread per output): the "vs input" bar."""
    import torch

    M = A.shape[0]
    N = Wq.shape[0]
    if C is None:
        C = torch.empty((M, N), dtype=torch.float16, device=A.device)
    p = w8a16_params(A, Wq, scale, zero, C, fmt, group)
    _check(lib().tempo_naive_gemm_w8a16_launch(p, _stream(stream)), "tempo_naive_gemm_w8a16_launch")
    return C


def gptq_operand_error(qweight, qzeros, scales, group: int = 128):
    """Why these are not GPTQ int8 checkpoint tensors of one layer (None if they are):
    qweight int32 [K/4, N], qzeros int32 [K/group, N/4], scales fp16 [K/group, N], all
    contiguous (the layout of bench/gemm_baseline.py:214-232 in the reference)."""
    import torch

    if qweight.dtype != torch.int32 or qweight.dim() != 2 or not qweight.is_contiguous():
        return "qweight must be a contiguous int32 [K/4, N] tensor"
    K, N = qweight.shape[0] * 4, qweight.shape[1]
    if group <= 0 or K % group or N % 4:
        return "K = %d must be a multiple of group %d and N = %d of 4" % (K, group, N)
    if qzeros.dtype != torch.int32 or not qzeros.is_contiguous() or \
            tuple(qzeros.shape) != (K // group, N // 4):
        return "qzeros must be a contiguous int32 tensor of shape %s" % ((K // group, N // 4),)
    if scales.dtype != torch.float16 or not scales.is_contiguous() or \
            tuple(scales.shape) != (K // group, N):
        return "scales must be a contiguous fp16 tensor of shape %s" % ((K // group, N),)
    return None


def gptq_repack(qweight, qzeros, scales, group: int = 128, stream=None):
    """GPTQ int8 checkpoint tensors (qweight int32 [K/4,N], qzeros int32 [K/G,N/4], scales fp16
    [K/G,N]) -> (wq uint8 [N,K], scale fp16 [N,K/G], zero uint8 [N,K/G]) for gemm_w8a16 fmt 2."""
    import torch

    why = gptq_operand_error(qweight, qzeros, scales, group)
    if why:
        raise ValueError("GPTQ tensors: " + why)
    K = qweight.shape[0] * 4
    N = qweight.shape[1]
    dev = qweight.device
    wq = torch.empty((N, K), dtype=torch.uint8, device=dev)
    sc = torch.empty((N, K // group), dtype=torch.float16, device=dev)
    zr = torch.empty((N, K // group), dtype=torch.uint8, device=dev)
    _check(lib().tempo_gptq_repack_u8(_ptr(qweight), _ptr(qzeros), _ptr(scales), K, N, group,
                                      _ptr(wq), _ptr(sc), _ptr(zr), _stream(stream)),
           "tempo_gptq_repack_u8")
    return wq, sc, zr


def probe_mfma_layout(ms: int, device="cuda"):
    """Returns (rows, cols) int arrays [64][nacc] of the MFMA result map, measured on the GPU."""
    import torch

    nacc = 16 if ms == 32 else 4
    out = torch.zeros((2, 64, nacc), dtype=torch.float32, device=device)
    _check(lib().tempo_probe_mfma_layout(ms, _ptr(out), _stream(None)), "tempo_probe_mfma_layout")
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    return o[0].astype(int) - 1, o[1].astype(int) - 1
