"""Operation spec: validation and work count (reference tempo/core/op/spec.py:23-46).

The product recognises a DECLARED operation; an unknown kernel is refused, not guessed at."""
from __future__ import annotations

from tempo.plugins.base import OpSpec  # noqa: F401  (defined once, in the contract)

__all__ = ["OpSpec", "validate", "describe", "flops"]

KNOWN_KINDS = ("gemm",)
KNOWN_DTYPES = ("fp16", "fp32", "int8", "uint8", "q7", "bf16")


def validate(op: OpSpec) -> None:
    if op.kind not in KNOWN_KINDS:
        raise ValueError("operation %r is not declared; known: %s" % (op.kind, ", ".join(KNOWN_KINDS)))
    for name in ("dtype_a", "dtype_b", "dtype_c", "dtype_acc"):
        v = getattr(op, name)
        if v not in KNOWN_DTYPES:
            raise ValueError("type %s=%r is not declared" % (name, v))
    if op.kind == "gemm":
        for k in ("M", "N", "K"):
            if k not in op.shapes:
                raise ValueError("gemm needs shape %r" % k)
            if int(op.shapes[k]) <= 0:
                raise ValueError("shape %s = %r" % (k, op.shapes[k]))
    if op.tol_rel_l2 < 0:
        raise ValueError("negative tolerance")


def flops(op: OpSpec) -> float:
    if op.kind != "gemm":
        raise ValueError("work count is declared for 'gemm' only")
    s = op.shapes
    return 2.0 * s["M"] * s["N"] * s["K"]


def describe(op: OpSpec) -> str:
    """One line for logs and reports, e.g.
    "gemm[M=4096 N=15360 K=3840] A:fp16/k B:fp16/k -> C:fp16/n, fp32 accumulation"."""
    dims = " ".join("%s=%s" % (k, op.shapes[k]) for k in ("M", "N", "K") if k in op.shapes)
    return "%s[%s] A:%s/%s B:%s/%s -> C:%s/%s, %s accumulation" % (
        op.kind, dims, op.dtype_a, op.layout_a, op.dtype_b, op.layout_b, op.dtype_c, op.layout_c,
        op.dtype_acc)
