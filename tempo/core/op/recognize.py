"""Recognition: naive source -> OpSpec, from its TEMPO-OP block only.

Reference: tempo/core/op/recognize.py:41-141.  Same block grammar, same refusals:
  * no TEMPO-OP block -> NotRecognised (there is no C++ parser, by design);
  * the declared entry must be DECLARED in the source (name followed by "("), and the
    signature's argument count must match that declaration;
  * a shape written "*" must be supplied at recognition time.
"""
from __future__ import annotations

import re

from .spec import OpSpec, validate

BLOCK_START = re.compile(r"TEMPO-OP\s*:\s*(\w+)")
KV = re.compile(r"^\s*(?://|#|\*)?\s*([A-Za-z_][\w]*)\s*:\s*(.+?)\s*$")


class NotRecognised(Exception):
    """An unknown kernel is refused, not compiled badly."""


def parse_block(text: str) -> dict:
    m = BLOCK_START.search(text)
    if not m:
        raise NotRecognised("no TEMPO-OP block in the source: only declared operations are "
                            "recognised")
    out = {"kind": m.group(1)}
    for ln in text[m.end():].split("\n")[:40]:
        if "TEMPO-OP-END" in ln:
            break
        km = KV.match(ln)
        if not km:
            continue
        key, val = km.group(1).lower(), km.group(2)
        if key in ("dtype", "layout", "shape"):
            sub = {}
            for pair in val.replace(",", " ").split():
                if "=" in pair:
                    a, b = pair.split("=", 1)
                    sub[a.strip().lower()] = b.strip()
            out[key] = sub
        elif key in ("tol_rel_l2", "entry", "signature", "coverage", "scale"):
            out[key] = val
    return out


def to_spec(block: dict, shapes: dict = None) -> OpSpec:
    d = block.get("dtype", {})
    lay = block.get("layout", {})
    s = dict(block.get("shape", {}))
    shapes = shapes or {}
    resolved = {}
    for k in ("M", "N", "K"):
        v = shapes.get(k, s.get(k, s.get(k.lower())))
        if v is None or str(v) == "*":
            if k in shapes:
                v = shapes[k]
            else:
                raise NotRecognised("shape %s is declared '*' (set at run time) but not given" % k)
        resolved[k] = int(v)
    op = OpSpec(kind=block["kind"], dtype_a=d.get("a", "fp16"), dtype_b=d.get("b", "fp16"),
                dtype_c=d.get("c", "fp16"), dtype_acc=d.get("acc", "fp32"),
                layout_a=lay.get("a", "k"), layout_b=lay.get("b", "k"), layout_c=lay.get("c", "n"),
                shapes=resolved, scale=block.get("scale"),
                tol_rel_l2=float(block.get("tol_rel_l2", 0.0)),
                coverage=block.get("coverage", "atomic_stamp"))
    validate(op)
    return op


def check_signature(block: dict, text: str) -> None:
    entry = block.get("entry")
    if not entry:
        raise NotRecognised("the TEMPO-OP block declares no entry")
    # look for a DECLARATION (name then "("), not any mention: the block itself names it
    if not re.search(re.escape(entry) + r"\s*\(", text):
        raise NotRecognised("entry %r is declared in TEMPO-OP but not in the source" % entry)
    sig = block.get("signature")
    if sig:
        args = [a.strip() for a in sig.strip("()").split(",") if a.strip()]
        m = re.search(re.escape(entry) + r"\s*\(([^)]*)\)", text)
        if m:
            real = [a.strip() for a in m.group(1).split(",") if a.strip()]
            if len(real) != len(args):
                raise NotRecognised("TEMPO-OP signature has %d arguments, the source %d"
                                    % (len(args), len(real)))


def from_file(path: str, shapes: dict = None) -> OpSpec:
    with open(path, encoding="utf-8") as f:
        text = f.read()
    block = parse_block(text)
    check_signature(block, text)
    return to_spec(block, shapes)
