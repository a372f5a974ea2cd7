"""PyTorch-ROCm integration of the shipped gfx950 GEMMs: torch.library custom ops that replace
F.linear for the shapes the ladder covers.

The binding follows the reference's integration contract for a shipped kernel
(kernels/shipped/gemm_fp16/sm_70/INTEGRATION.md:81-116):

* a default-OFF environment gate, TEMPO_KERNELS=1 to enable (INTEGRATION.md:99-106), read at
  every call so a server can flip it between requests;
* the shape predicate decides, and a refusal (TEMPO_FALLBACK) takes the caller's own path
  (F.linear, or dequantise + F.linear for 8-bit weights);
* an entry proof: every call is counted under the ladder row that ran it ("off" when gated,
  "fallback" when refused), so a benchmark can show the kernels were entered before it reports
  a speed-up (MEASURE_DISCIPLINE.md:79-83).

With the gate on and a CUDA tensor in hand, a missing native library raises: there is no silent
route around libtempo_gfx950.so.

    import cuda_tempiler_amd.torch_ops as tops
    y = torch.ops.tempo.linear_fp16(x, w)              # x [..., K] fp16, w [N, K] fp16
    y = torch.ops.tempo.linear_w8a16(x, wq, s, z, 2, 128)
    h = torch.ops.tempo.linear_gate_up_fp16(x, w_gate_up)   # silu(x.Wg^T) * (x.Wu^T), fused
    tops.counters()                                     # {"i256x256k64w4r8": 3, "off": 1, ...}
"""
from __future__ import annotations

import collections
import os
import threading
from typing import Optional

import torch
import torch.nn.functional as F

from . import capi

GATE_ENV = "TEMPO_KERNELS"

_lock = threading.Lock()
_counts: collections.Counter = collections.Counter()


def enabled() -> bool:
    """TEMPO_KERNELS=1 turns the kernels on; anything else (or unset) leaves them off."""
    return os.environ.get(GATE_ENV, "0") == "1"


def counters() -> dict:
    with _lock:
        return dict(_counts)


def reset_counters() -> None:
    with _lock:
        _counts.clear()


def _count(key: str) -> None:
    with _lock:
        _counts[key] += 1


def _rows(x: torch.Tensor):
    """x [..., K] -> a 2-D [M, K] view with unit inner stride (a copy only when unavoidable)."""
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    return x2


def _covered_device(*ts) -> bool:
    return all(t is None or (t.is_cuda and t.device == ts[0].device) for t in ts)


# ------------------------------------------------------------------------------ fp16 linear


def _linear_fp16_impl(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    if not enabled():
        _count("off")
        return F.linear(x, w)
    if (x.dtype != torch.float16 or w.dtype != torch.float16 or w.dim() != 2
            or w.stride(1) != 1 or not _covered_device(x, w) or x.shape[-1] != w.shape[1]):
        _count("fallback")
        return F.linear(x, w)
    x2 = _rows(x)
    M, K = x2.shape
    N = w.shape[0]
    tag = capi.route(0, M, N, K)
    y = torch.empty((M, N), dtype=torch.float16, device=x.device)
    try:
        # the split-K workspace comes from torch's caching allocator (graph-capture safe), not
        # from the library's pool
        capi.gemm_fp16(x2, w, y, workspace="torch")
    except capi.NotCovered:
        _count("fallback")
        return F.linear(x, w)
    _count(tag)
    return y.view(*x.shape[:-1], N)


@torch.library.custom_op("tempo::linear_fp16", mutates_args=())
def linear_fp16(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """y = x . w^T for x [..., K], w [N, K] (F.linear without bias), fp16 in and out."""
    return _linear_fp16_impl(x, w)


@linear_fp16.register_fake
def _(x, w):
    return x.new_empty((*x.shape[:-1], w.shape[0]))


# ------------------------------------------------------------------------------ 8-bit weights


def dequantize(wq: torch.Tensor, scale: torch.Tensor, zero: Optional[torch.Tensor], fmt: int,
               group: int = 128) -> torch.Tensor:
    """The caller's own path for 8-bit weights: W [N, K] fp16 = fp16_rn((q - z) * s).  The
    product of a 9-bit integer and an fp16 scale is exact in fp32, so this is the same single
    rounding the fused kernels perform."""
    if fmt == capi.W8_SYM_I8:
        return (wq.float() * scale.float()[:, None]).half()
    N, K = wq.shape
    s = scale.float().repeat_interleave(group, dim=1)[:, :K]
    z = zero.float().repeat_interleave(group, dim=1)[:, :K]
    return ((wq.float() - z) * s).half()


def _w8_covered(x, wq, scale, zero, fmt, group) -> bool:
    """The kernels take these operands as they are: right dtypes and shapes (the library reads
    them as raw memory of the declared layout), one device, x fp16 [..., K].  Anything else is
    the caller's own path, which gives the answer its own semantics give (or raises)."""
    if x.dtype != torch.float16 or x.dim() < 1 or not _covered_device(x, wq, scale, zero):
        return False
    x2 = x.reshape(-1, x.shape[-1])
    return capi.w8a16_operand_error(x2 if x2.stride(-1) == 1 else x2.contiguous(), wq, scale,
                                    zero, fmt, group) is None


def _packed_meta(scale, zero):
    """Scale and zero-points as the kernels read them: packed rows.  A strided view (a column
    slice of a larger table, say) is copied once here rather than sent to the caller's path."""
    if scale is not None and not scale.is_contiguous():
        scale = scale.contiguous()
    if zero is not None and not zero.is_contiguous():
        zero = zero.contiguous()
    return scale, zero


def _linear_w8a16_impl(x, wq, scale, zero, fmt, group):
    scale, zero = _packed_meta(scale, zero)

    def own_path():
        return F.linear(x, dequantize(wq, scale, zero, fmt, group).to(x.device))

    if not enabled():
        _count("off")
        return own_path()
    if not _w8_covered(x, wq, scale, zero, fmt, group):
        _count("fallback")
        return own_path()
    x2 = _rows(x)
    M, K = x2.shape
    N = wq.shape[0]
    tag = capi.route(fmt, M, N, K)
    y = torch.empty((M, N), dtype=torch.float16, device=x.device)
    try:
        capi.gemm_w8a16(x2, wq, scale, zero, fmt=fmt, group=group, C=y, workspace="torch")
    except capi.NotCovered:
        _count("fallback")
        return own_path()
    _count(tag)
    return y.view(*x.shape[:-1], N)


@torch.library.custom_op("tempo::linear_w8a16", mutates_args=())
def linear_w8a16(x: torch.Tensor, wq: torch.Tensor, scale: torch.Tensor,
                 zero: Optional[torch.Tensor], fmt: int, group: int) -> torch.Tensor:
    """y = x . dequant(wq)^T; fmt 1: int8 wq [N, K], scale [N]; fmt 2: uint8 wq [N, K], scale
    fp16 and zero uint8 [N, K/group]."""
    return _linear_w8a16_impl(x, wq, scale, zero, fmt, group)


@linear_w8a16.register_fake
def _(x, wq, scale, zero, fmt, group):
    return x.new_empty((*x.shape[:-1], wq.shape[0]))


# ------------------------------------------------------------------------------ fused gate/up


def _silu_mul_own(y: torch.Tensor) -> torch.Tensor:
    g, u = y.chunk(2, dim=-1)
    return F.silu(g) * u


def _gate_up_impl(x, run_kernel, own_path, op_code, N, K):
    if not enabled():
        _count("off")
        return own_path()
    x2 = _rows(x)
    M = x2.shape[0]
    tag = capi.route(op_code, M, N, K)
    y = torch.empty((M, N), dtype=torch.float16, device=x.device)
    try:
        run_kernel(x2, y)
    except capi.NotCovered:
        _count("fallback")
        return own_path()
    _count(tag)
    return y.view(*x.shape[:-1], N)


@torch.library.custom_op("tempo::linear_gate_up_fp16", mutates_args=())
def linear_gate_up_fp16(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """silu(x . w[:N]^T) * (x . w[N:]^T) for the merged gate_up weight w [2N, K] (gate rows, then
    up rows): the MLP's first projection with its activation fused into the GEMM epilogue."""
    N, K = w.shape[0] // 2, w.shape[1]

    def own_path():
        return _silu_mul_own(F.linear(x, w))

    if (x.dtype != torch.float16 or w.dtype != torch.float16 or w.dim() != 2 or w.shape[0] % 2
            or w.stride(1) != 1 or not _covered_device(x, w) or x.shape[-1] != K):
        if enabled():
            _count("fallback")
            return own_path()
    return _gate_up_impl(x, lambda x2, y: capi.gemm_fp16_gate_up(x2, w, y), own_path, 3, N, K)


@linear_gate_up_fp16.register_fake
def _(x, w):
    return x.new_empty((*x.shape[:-1], w.shape[0] // 2))


@torch.library.custom_op("tempo::linear_gate_up_w8a16", mutates_args=())
def linear_gate_up_w8a16(x: torch.Tensor, wq: torch.Tensor, scale: torch.Tensor,
                         zero: Optional[torch.Tensor], fmt: int, group: int) -> torch.Tensor:
    """The fused gate/up projection on 8-bit weights wq [2N, K] (scale / zero rows follow)."""
    N, K = wq.shape[0] // 2, wq.shape[1]
    scale, zero = _packed_meta(scale, zero)

    def own_path():
        return _silu_mul_own(F.linear(x, dequantize(wq, scale, zero, fmt, group).to(x.device)))

    if wq.dim() != 2 or wq.shape[0] % 2 or not _w8_covered(x, wq, scale, zero, fmt, group):
        if enabled():
            _count("fallback")
            return own_path()
    return _gate_up_impl(
        x, lambda x2, y: capi.gemm_w8a16_gate_up(x2, wq, scale, zero, fmt=fmt, group=group, C=y),
        own_path, 3 + fmt, N, K)


@linear_gate_up_w8a16.register_fake
def _(x, wq, scale, zero, fmt, group):
    return x.new_empty((*x.shape[:-1], wq.shape[0] // 2))


# ------------------------------------------------------------------------------ modules


class Linear(torch.nn.Module):
    """Drop-in for an fp16 nn.Linear: the GEMM goes through tempo::linear_fp16, the bias (if
    any) is added afterwards."""

    def __init__(self, weight: torch.Tensor, bias: Optional[torch.Tensor] = None):
        super().__init__()
        self.weight = torch.nn.Parameter(weight.contiguous(), requires_grad=False)
        self.bias = None if bias is None else torch.nn.Parameter(bias, requires_grad=False)

    @classmethod
    def from_linear(cls, lin: torch.nn.Linear) -> "Linear":
        return cls(lin.weight.detach(), None if lin.bias is None else lin.bias.detach())

    def forward(self, x):
        y = torch.ops.tempo.linear_fp16(x, self.weight)
        return y if self.bias is None else y + self.bias


class GPTQLinear(torch.nn.Module):
    """A GPTQ int8 layer (qweight [K/4, N] int32, qzeros [K/G, N/4] int32, scales [K/G, N] fp16;
    the reference's format, bench/gemm_baseline.py:214-232), repacked ONCE on the device into the
    [N, K] layout of the fused W8A16 kernels and served through tempo::linear_w8a16 (fmt 2)."""

    def __init__(self, qweight, qzeros, scales, bias=None, group: int = 128):
        super().__init__()
        if not qweight.is_cuda:
            raise ValueError("GPTQLinear repacks on the GPU: hand it device tensors")
        wq, s, z = capi.gptq_repack(qweight, qzeros, scales, group)
        self.register_buffer("wq", wq)
        self.register_buffer("scale", s)
        self.register_buffer("zero", z)
        self.group = group
        self.bias = None if bias is None else torch.nn.Parameter(bias, requires_grad=False)

    def forward(self, x):
        y = torch.ops.tempo.linear_w8a16(x, self.wq, self.scale, self.zero, capi.W8_ASYM_U8,
                                         self.group)
        return y if self.bias is None else y + self.bias


def swap_linears(module: torch.nn.Module) -> int:
    """Replace every fp16 nn.Linear under `module` by Linear (same weights); returns how many.
    Whether the kernels run is still decided per call by the gate and the shape predicate."""
    n = 0
    for name, child in list(module.named_children()):
        if isinstance(child, torch.nn.Linear) and child.weight.dtype == torch.float16:
            setattr(module, name, Linear.from_linear(child))
            n += 1
        else:
            n += swap_linears(child)
    return n
