"""Operation spec: validation and work count (reference tempo/core/op/spec.py:23-46).

The product recognises a DECLARED operation; an unknown kernel is refused, not guessed at."""
from __future__ import annotations

from tempo.plugins.base import OpSpec  # noqa: F401  (defined once, in the contract)

__all__ = ["OpSpec", "validate", "describe", "flops"]

KNOWN_KINDS = ("gemm", "attention")
KNOWN_DTYPES = ("fp16", "fp32", "int8", "uint8", "q7", "bf16")
# the dimensions each kind declares (attention: batch, query heads, key/value heads, query and
# key lengths, head dimension, and CAUSAL = 1 for the bottom-right causal mask, 0 for none)
DIMS = {"gemm": ("M", "N", "K"), "attention": ("B", "H", "HKV", "SQ", "SK", "D", "CAUSAL")}


def validate(op: OpSpec) -> None:
    if op.kind not in KNOWN_KINDS:
        raise ValueError("operation %r is not declared; known: %s" % (op.kind, ", ".join(KNOWN_KINDS)))
    for name in ("dtype_a", "dtype_b", "dtype_c", "dtype_acc"):
        v = getattr(op, name)
        if v not in KNOWN_DTYPES:
            raise ValueError("type %s=%r is not declared" % (name, v))
    for k in DIMS[op.kind]:
        if k not in op.shapes:
            raise ValueError("%s needs shape %r" % (op.kind, k))
        if int(op.shapes[k]) <= 0 and k != "CAUSAL":
            raise ValueError("shape %s = %r" % (k, op.shapes[k]))
    if op.kind == "attention":
        if op.shapes["H"] % op.shapes["HKV"]:
            raise ValueError("attention: H = %r is not a multiple of HKV = %r"
                             % (op.shapes["H"], op.shapes["HKV"]))
        if op.shapes["CAUSAL"] not in (0, 1):
            raise ValueError("attention: CAUSAL = %r (0 or 1)" % (op.shapes["CAUSAL"],))
    if op.tol_rel_l2 < 0:
        raise ValueError("negative tolerance")


def visible_pairs(sq: int, sk: int, causal: int) -> int:
    """(query, key) pairs the mask leaves visible: all of them, or with the bottom-right causal
    mask (key j visible to query i iff j <= i + sk - sq) sum_i clamp(i + sk - sq + 1, 0, sk)."""
    if not causal:
        return sq * sk
    off = sk - sq
    lo = max(0, -off)  # the first query row that sees a key; row i sees i + off + 1 <= sk keys
    first, last = lo + off + 1, sq + off  # keys seen by rows lo and sq - 1
    return (first + last) * (sq - lo) // 2 if sq > lo else 0


def flops(op: OpSpec) -> float:
    s = op.shapes
    if op.kind == "gemm":
        return 2.0 * s["M"] * s["N"] * s["K"]
    if op.kind == "attention":  # scores and P.V: 2 D flops each per visible (query, key) pair
        return 4.0 * s["B"] * s["H"] * s["D"] * visible_pairs(s["SQ"], s["SK"], s["CAUSAL"])
    raise ValueError("no work count for %r" % op.kind)


def describe(op: OpSpec) -> str:
    """One line for logs and reports, e.g.
    "gemm[M=4096 N=15360 K=3840] A:fp16/k B:fp16/k -> C:fp16/n, fp32 accumulation"."""
    dims = " ".join("%s=%s" % (k, op.shapes[k]) for k in DIMS.get(op.kind, ()) if k in op.shapes)
    return "%s[%s] A:%s/%s B:%s/%s -> C:%s/%s, %s accumulation" % (
        op.kind, dims, op.dtype_a, op.layout_a, op.dtype_b, op.layout_b, op.dtype_c, op.layout_c,
        op.dtype_acc)
