"""gfx950: TOOLCHAIN -- section 8a: build, and read the build's own numbers (reference pattern
tempo/plugins/sm70/toolchain.py, which parses ptxas -v).

compile() builds a rendered kernel with hipcc for gfx950 and reports, per the contract's
BuildResult, the numbers the AMD toolchain gives for OUR build:
  * from the compiler's resource-usage remarks (-Rpass-analysis=kernel-resource-usage):
    VGPRs, AGPRs, spilled VGPRs/SGPRs, scratch bytes per lane, LDS bytes, occupancy;
  * from the code object (llvm-objdump of the device ELF): the instruction mix -- MFMA count,
    ds_read_b128 / LDS-DMA presence, and scratch_* instructions inside loops (the analogue of
    the reference's "LDL/STL in loops").
Nothing here reads any binary not built from this repository's sources.
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess
from pathlib import Path

from ..base import BuildResult, EnvReq
from .classifier import OBJDUMP, parse_disasm

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = ["-O3", "-std=c++17", "--offload-arch=%s" % ARCH,
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]

_REMARK = re.compile(r"remark: ([^:]+):(\d+):\d+: (.+?) \[-Rpass-analysis")


def source_flags(path) -> list:
    """Extra compiler flags a source declares for itself: "// tempo:flags <flags>" lines in its
    first 40 lines (the emitter writes one for kinds that need a particular scheduler)."""
    out = []
    with open(path, encoding="utf-8") as f:
        for i, line in enumerate(f):
            if i >= 40:
                break
            if line.startswith("// tempo:flags "):
                out += line[len("// tempo:flags "):].split()
    return out


def parse_resource_remarks(text: str) -> dict:
    """{kernel symbol: {field: value}} from -Rpass-analysis=kernel-resource-usage output."""
    out, cur = {}, None
    for line in text.splitlines():
        m = re.search(r"remark: .*?Function Name: (\S+)", line)
        if m:
            cur = m.group(1)
            out[cur] = {}
            continue
        if cur is None:
            continue
        m = re.search(r"remark: .*?\s([A-Za-z][A-Za-z /\[\]]+?): (\S+) \[-Rpass", line)
        if m:
            key, val = m.group(1).strip(), m.group(2)
            try:
                out[cur][key] = int(val)
            except ValueError:
                out[cur][key] = val
    return out


def _is_lds_dma(mn: str, ops: str) -> bool:
    """A global->LDS copy: the FLAT form global_load_lds_*, or a MUBUF load carrying the lds
    modifier (buffer_load_dword* ... lds), which writes LDS instead of VGPRs."""
    if mn.startswith("global_load_lds"):
        return True
    return mn.startswith("buffer_load") and re.search(r"(^|[\s,])lds($|\s)", ops) is not None


def isa_summary(instrs: list) -> dict:
    """Instruction mix of a disassembled kernel.  `instrs` holds mnemonics, or (mnemonic, operand
    text) pairs (parse_disasm(..., operands=True)); the LDS-DMA and buffer-load counts need the
    operands, since the MUBUF LDS copy differs from a register load only by its lds modifier."""
    pairs = [(x, "") if isinstance(x, str) else (x[0], x[1]) for x in instrs]
    dma = [_is_lds_dma(mn, ops) for mn, ops in pairs]
    return {
        "mfma": sum(1 for mn, _ in pairs if mn.startswith("v_mfma")),
        "ds_read_b128": sum(1 for mn, _ in pairs if mn in ("ds_read_b128", "ds_load_b128")),
        "lds_dma": sum(dma),
        "lds_dma_buffer": sum(1 for (mn, _), d in zip(pairs, dma)
                              if d and mn.startswith("buffer_load")),
        "buffer_load": sum(1 for (mn, _), d in zip(pairs, dma)
                           if not d and mn.startswith("buffer_load")),
        "global_load_dwordx4": sum(1 for mn, _ in pairs if mn == "global_load_dwordx4"),
        "scratch": sum(1 for mn, _ in pairs if mn.startswith("scratch_")),
        "barrier": sum(1 for mn, _ in pairs if mn == "s_barrier"),
        "total": len(pairs),
    }


class Gfx950Toolchain:
    def arch_flags(self) -> list:
        return list(FLAGS)

    def requirements(self) -> list:
        return [EnvReq("hipcc", shutil.which(HIPCC) or (HIPCC if os.path.exists(HIPCC) else None),
                       "HIP compiler with gfx950 support (ROCm >= 7)"),
                EnvReq("llvm-objdump", OBJDUMP if os.path.exists(OBJDUMP) else None,
                       "AMDGPU disassembler of our own builds"),
                EnvReq("rocprofv3", shutil.which("rocprofv3"), "kernel trace and PMC counters")]

    def compile(self, source: Path, out: Path, mode: str = "obj", extra: list = (),
                build_dir: Path = None) -> BuildResult:
        """mode: "obj" (host+device object), "device" (device-only code object, disassemblable),
        "exe" (link an executable)."""
        source, out = Path(source), Path(out)
        out.parent.mkdir(parents=True, exist_ok=True)
        cmd = ([HIPCC] + FLAGS + source_flags(source) + ["-Rpass-analysis=kernel-resource-usage"]
               + list(extra))
        if mode == "device":
            cmd += ["--cuda-device-only", "--no-gpu-bundle-output", "-c"]
        elif mode == "obj":
            cmd += ["-c"]
        elif mode != "exe":
            raise ValueError("mode %r" % mode)
        cmd += [str(source), "-o", str(out)]
        r = subprocess.run(cmd, capture_output=True, text=True,
                           cwd=str(build_dir) if build_dir else None)
        log = r.stdout + r.stderr
        if r.returncode != 0:
            return BuildResult(ok=False, binary=None, regs=0, spill_st=0, spill_ld=0, stack_frame=0,
                               smem_static=0, smem_dynamic=0, ldl_stl_in_loops=None, log=log)
        res = parse_resource_remarks(log)
        # the rendered file holds one instantiated kernel; take the largest numbers if several
        vg = max((k.get("VGPRs", 0) for k in res.values()), default=0)
        ag = max((k.get("AGPRs", 0) for k in res.values()), default=0)
        sp = max((k.get("VGPRs Spill", 0) for k in res.values()), default=0)
        ssp = max((k.get("SGPRs Spill", 0) for k in res.values()), default=0)
        scr = max((k.get("ScratchSize [bytes/lane]", 0) for k in res.values()), default=0)
        lds = max((k.get("LDS Size [bytes/block]", 0) for k in res.values()), default=0)
        scratch_in_code = None
        if mode == "device":
            scratch_in_code = isa_summary(
                sum(parse_disasm(self.disasm(out), operands=True).values(), []))["scratch"]
        return BuildResult(ok=True, binary=out, regs=int(vg + ag), spill_st=int(sp),
                           spill_ld=int(ssp), stack_frame=int(scr), smem_static=int(lds),
                           smem_dynamic=0, ldl_stl_in_loops=scratch_in_code, log=log)

    def disasm(self, binary: Path) -> str:
        r = subprocess.run([OBJDUMP, "-d", "--mcpu=%s" % ARCH, str(binary)], capture_output=True,
                           text=True)
        if r.returncode != 0:
            raise RuntimeError("llvm-objdump failed: %s" % r.stderr[-2000:])
        return r.stdout

    def resources(self, log: str) -> dict:
        return parse_resource_remarks(log)
