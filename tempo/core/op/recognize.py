"""Recognition: a naive kernel source -> OpSpec, read from the declaration block it carries.

The operation is DECLARED in the naive source itself, inside a comment (format of the
reference's naive inputs, kernels/naive/gemm_fp16.cu:30-38; recogniser semantics of
tempo/core/op/recognize.py:41-141 -- the refusals below are the same, the parser is not):

    TEMPO-OP: gemm
      dtype: a=fp16 b=fp16 c=fp16 acc=fp32
      layout: a=k b=k c=n
      shape: M=* N=* K=*          ("*" = supplied when the spec is built)
      tol_rel_l2: 3e-3
      entry: naive_gemm_fp16
      signature: (const _Float16* A, ...)
    TEMPO-OP-END

Design: the block is cut out of the source as a region (header line to the END marker, at most
BLOCK_MAX_LINES lines), each line is stripped of its comment leader and split at the first ':'
into a field, and a per-field reader turns the value into data.  The entry check then looks for
the entry's DECLARATION in the source with the block region removed (so the block's own mention
of the name can never satisfy it) and counts the top-level parameters of that declaration with a
bracket-depth scan, which also copes with template arguments and function-pointer parameters.

Refusals (all NotRecognised; nothing unknown is guessed at):
  * the source has no TEMPO-OP block;
  * the block names no entry, or the source does not declare it;
  * the block's signature and the declaration disagree on the parameter count;
  * a shape declared "*" is not supplied.
"""
from __future__ import annotations

import re
from dataclasses import dataclass, field

from .spec import DIMS, OpSpec, validate

BLOCK_MAX_LINES = 40          # a declaration block longer than this is not read past its end
_HEADER = re.compile(r"TEMPO-OP\s*:\s*([A-Za-z_]\w*)")
_END = "TEMPO-OP-END"
_COMMENT_LEADERS = "/*#! \t"


class NotRecognised(Exception):
    """An unknown or inconsistently declared kernel is refused, not compiled badly."""


def _pairs(value: str) -> dict:
    """'a=fp16 b=fp16, c=fp16' -> {'a': 'fp16', ...} (keys lower-cased; unpaired words ignored)."""
    out = {}
    for word in value.replace(",", " ").split():
        key, eq, val = word.partition("=")
        if eq:
            out[key.strip().lower()] = val.strip()
    return out


def _text(value: str) -> str:
    return value.strip()


# field name -> reader; fields not listed here are ignored (forward compatible)
_READERS = {
    "dtype": _pairs, "layout": _pairs, "shape": _pairs,
    "tol_rel_l2": _text, "entry": _text, "signature": _text, "coverage": _text, "scale": _text,
}


@dataclass
class Declaration:
    """The parsed block: operation kind, its fields, and the source lines it occupied."""
    kind: str
    fields: dict = field(default_factory=dict)
    span: tuple = (0, 0)  # [first, last) line indices of the block in the source

    def get(self, name, default=None):
        return self.fields.get(name, default)


def read_declaration(text: str) -> Declaration:
    lines = text.split("\n")
    head = next((i for i, ln in enumerate(lines) if _HEADER.search(ln)), None)
    if head is None:
        raise NotRecognised("no TEMPO-OP block in the source: only declared operations are "
                            "recognised (there is no C++ parser here, by design)")
    decl = Declaration(kind=_HEADER.search(lines[head]).group(1))
    last = min(len(lines), head + 1 + BLOCK_MAX_LINES)
    end = last
    for i in range(head + 1, last):
        body = lines[i].strip().lstrip(_COMMENT_LEADERS).rstrip()
        if _END in body:
            end = i + 1
            break
        name, colon, value = body.partition(":")
        name = name.strip().lower()
        if not colon or not name.isidentifier() or not value.strip():
            continue
        reader = _READERS.get(name)
        if reader is not None:
            decl.fields[name] = reader(value)
    decl.span = (head, end)
    return decl


def _parameter_count(params: str) -> int:
    """Top-level comma-separated parameters of a C/C++ parameter list (without its parens)."""
    depth, count, seen = 0, 0, False
    for ch in params:
        if ch in "(<[{":
            depth += 1
        elif ch in ")>]}":
            depth -= 1
        elif ch == "," and depth == 0:
            count += 1
            continue
        if not ch.isspace():
            seen = True
    return count + 1 if seen else 0


def _declared_parameters(source: str, entry: str):
    """Parameter text of the first `entry(...)` in `source`, or None if it is not declared."""
    m = re.search(r"\b" + re.escape(entry) + r"\s*\(", source)
    if m is None:
        return None
    depth, start = 1, m.end()
    for i in range(start, len(source)):
        if source[i] == "(":
            depth += 1
        elif source[i] == ")":
            depth -= 1
            if depth == 0:
                return source[start:i]
    return source[start:]


def check_entry(decl: Declaration, text: str) -> None:
    entry = decl.get("entry")
    if not entry:
        raise NotRecognised("the TEMPO-OP block declares no entry")
    lines = text.split("\n")
    outside = "\n".join(lines[:decl.span[0]] + lines[decl.span[1]:])
    params = _declared_parameters(outside, entry)
    if params is None:
        raise NotRecognised("entry %r is named in the TEMPO-OP block but the source does not "
                            "declare it: the declaration has fallen behind the code" % entry)
    sig = decl.get("signature")
    if sig:
        inner = sig.strip()
        if inner.startswith("(") and inner.endswith(")"):
            inner = inner[1:-1]
        want, have = _parameter_count(inner), _parameter_count(params)
        if want != have:
            raise NotRecognised("the TEMPO-OP signature has %d parameters, the source's %s has %d"
                                % (want, entry, have))


def build_spec(decl: Declaration, shapes: dict = None) -> OpSpec:
    given = dict(shapes or {})
    declared = {k.upper(): v for k, v in decl.get("shape", {}).items()}
    resolved = {}
    if decl.kind not in DIMS:
        raise NotRecognised("operation %r is not declared; known: %s"
                            % (decl.kind, ", ".join(sorted(DIMS))))
    for dim in DIMS[decl.kind]:
        value = given.get(dim, declared.get(dim))
        if value is None or str(value).strip() == "*":
            raise NotRecognised("shape %s is declared '*' (set at run time) but was not given"
                                % dim)
        resolved[dim] = int(value)
    dt, lay = decl.get("dtype", {}), decl.get("layout", {})
    op = OpSpec(kind=decl.kind,
                dtype_a=dt.get("a", "fp16"), dtype_b=dt.get("b", "fp16"),
                dtype_c=dt.get("c", "fp16"), dtype_acc=dt.get("acc", "fp32"),
                layout_a=lay.get("a", "k"), layout_b=lay.get("b", "k"), layout_c=lay.get("c", "n"),
                shapes=resolved, scale=decl.get("scale"),
                tol_rel_l2=float(decl.get("tol_rel_l2", 0.0)),
                coverage=decl.get("coverage", "atomic_stamp"))
    validate(op)
    return op


def from_text(text: str, shapes: dict = None) -> OpSpec:
    decl = read_declaration(text)
    check_entry(decl, text)
    return build_spec(decl, shapes)


def from_file(path: str, shapes: dict = None) -> OpSpec:
    with open(path, encoding="utf-8") as f:
        return from_text(f.read(), shapes)
