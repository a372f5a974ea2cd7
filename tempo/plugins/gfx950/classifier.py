"""gfx950: ISA CLASSIFIER -- optional section 6, over AMDGPU assembly of OUR OWN builds.

Reads the text llvm-objdump prints for a gfx950 code object built here, and sorts each
instruction into the bound model's channels.  Control-field decoding is not offered
(NotSupported): the AMD ISA has no scheduling words to decode."""
from __future__ import annotations

import re
import subprocess
from pathlib import Path

from ..base import AtomClass, NotSupported

OBJDUMP = "/opt/rocm/llvm/bin/llvm-objdump"

_RULES = (
    (re.compile(r"^v_mfma_\w*32x32x16"), "MFMA", 32.0, 0, "MFMA32"),
    (re.compile(r"^v_mfma_\w*16x16x32"), "MFMA", 16.0, 0, "MFMA16"),
    (re.compile(r"^v_mfma"), "MFMA", 16.0, 0, "MFMA"),
    (re.compile(r"^ds_read_b128|^ds_load_b128"), "LDS", 1.0, 16, "LDS"),
    (re.compile(r"^ds_read_b64|^ds_load_b64"), "LDS", 1.0, 8, "LDS"),
    (re.compile(r"^ds_(read|write|load|store)"), "LDS", 1.0, 4, "LDS"),
    (re.compile(r"^global_load_lds_dwordx4"), "VMEM", 1.0, 16, "VMEM"),
    (re.compile(r"^(global|buffer)_load_dwordx4"), "VMEM", 1.0, 16, "VMEM"),
    (re.compile(r"^(global|buffer|flat)_(load|store)"), "VMEM", 1.0, 4, "VMEM"),
    (re.compile(r"^scratch_"), "SPILL", 1.0, 4, "VMEM"),
    (re.compile(r"^s_barrier"), "ISSUE", 1.0, 0, "BARRIER"),
    (re.compile(r"^s_"), "ISSUE", 1.0, 0, "SALU"),
    (re.compile(r"^v_"), "ISSUE", 1.0, 0, "VALU"),
)


class Gfx950Classifier:
    def classify(self, instr_text: str) -> AtomClass:
        mn = instr_text.strip().split()[0] if instr_text.strip() else ""
        for rx, ch, cyc, width, lat in _RULES:
            if rx.search(mn):
                return AtomClass(channel=ch, cycles=cyc, width_bytes=width, latency_class=lat,
                                 predicated=False)
        return AtomClass(channel="ISSUE", cycles=1.0, width_bytes=0, latency_class="OTHER",
                         predicated=False)

    def decode(self, binary: Path, kernel_regex: str):
        """Instruction mnemonics of the kernels whose symbol matches kernel_regex."""
        out = subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", str(binary)], capture_output=True,
                             text=True, check=True).stdout
        return parse_disasm(out, kernel_regex)

    def control_fields(self, word: int):
        raise NotSupported("gfx950 ISA carries no scheduling control words")


def parse_disasm(text: str, kernel_regex: str = ".*", operands: bool = False) -> dict:
    """{symbol: [mnemonic, ...]} from llvm-objdump -d output; with operands=True the entries are
    (mnemonic, operand text) pairs, the operand text cut at the encoding comment."""
    rx = re.compile(kernel_regex)
    cur, out = None, {}
    for line in text.splitlines():
        m = re.match(r"^[0-9a-f]+ <(.+)>:\s*$", line)
        if m:
            cur = m.group(1) if rx.search(m.group(1)) else None
            if cur:
                out[cur] = []
            continue
        if cur is None:
            continue
        m = re.match(r"^\s+([a-z_][a-z0-9_]*)\b(.*)$", line)
        if m:
            if operands:
                out[cur].append((m.group(1), m.group(2).split("//")[0].strip()))
            else:
                out[cur].append(m.group(1))
    return out
