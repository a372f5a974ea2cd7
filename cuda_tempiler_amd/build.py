"""Build libtempo_gfx950.so in-tree (hipcc, gfx950 only).

    python3 -m cuda_tempiler_amd.build

Translation units: the two shipped deliveries' launch.hip (each instantiates its own ladder),
the FMHA unit and the C-ABI shim.  They compile in parallel, then link into one shared object
next to this file.  Before compiling, the shipped kernel.hip files are re-frozen from the
plugin skeletons and the dispatch tables regenerated from select.py, so a build always ships
what the skeletons and the ladders say.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
OUT = os.path.join(HERE, "libtempo_gfx950.so")
BUILD = os.path.join(HERE, "_build")
SHIPPED = os.path.join(ROOT, "kernels", "shipped")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 anywhere (their results are not trusted on this pool)
FLAGS = [
    "-O3", "-std=c++17", "--offload-arch=%s" % ARCH, "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]
INCLUDES = [
    "-I", os.path.join(ROOT, "include"),
    "-I", SHIPPED,
    "-I", os.path.join(ROOT, "kernels"),
    "-I", os.path.join(HERE, "csrc"),
    "-I", os.path.join(ROOT, "tempo", "plugins", "gfx950", "skeletons"),
]
UNITS = [
    os.path.join(SHIPPED, "gemm_fp16", "gfx950", "launch.hip"),
    os.path.join(SHIPPED, "gemm_fp16", "gfx950", "launch_prefill.hip"),
    os.path.join(SHIPPED, "gemm_w8a16", "gfx950", "launch.hip"),
    os.path.join(SHIPPED, "gemm_w8a16", "gfx950", "launch_prefill.hip"),
    os.path.join(HERE, "csrc", "fmha.hip"),
    os.path.join(HERE, "csrc", "gptq.hip"),
    os.path.join(HERE, "csrc", "capi.hip"),
]


def regenerate() -> None:
    """Freeze skeletons into the shipped kernel.hip files; regenerate dispatch.inc tables."""
    sys.path.insert(0, ROOT)
    from tempo.plugins.gfx950 import ship

    ship.write_all()
    for op in ("gemm_fp16", "gemm_w8a16"):
        d = os.path.join(SHIPPED, op, "gfx950")
        gens = [("dispatch.inc", []), ("dispatch_gate_up.inc", ["--gate-up"])]
        gens.append(("prefill.inc", ["--prefill"]))
        for name, args in gens:
            text = subprocess.run([sys.executable, os.path.join(d, "gen_dispatch.py")] + args,
                                  check=True, capture_output=True, text=True).stdout
            path = os.path.join(d, name)
            if not os.path.exists(path) or open(path).read() != text:
                with open(path, "w") as f:
                    f.write(text)


def unit_flags(src: str) -> list:
    """Flags a translation unit declares for itself ("// tempo:flags ..." in its first 40
    lines): launch_prefill.hip asks for the register-pressure-minimising scheduler."""
    out = []
    with open(src, encoding="utf-8") as f:
        for i, line in enumerate(f):
            if i >= 40:
                break
            if line.startswith("// tempo:flags "):
                out += line[len("// tempo:flags "):].split()
    return out


def _compile(src: str) -> str:
    name = os.path.relpath(src, ROOT).replace(os.sep, "_").replace(".hip", ".o")
    obj = os.path.join(BUILD, name)
    cmd = [HIPCC] + FLAGS + unit_flags(src) + INCLUDES + ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed on %s:\n%s\n%s" % (src, " ".join(cmd), r.stderr[-6000:]))
    return obj


# Delivery-only builds: each shipped delivery compiled from its own directory alone (-I there and
# nowhere else), linked with its ship_probe.hip into an executable.  This is what a host tree
# that vendors kernels/shipped/<op>/gfx950/ gets; tests run the probes on the GPU.
PROBE_OPS = ("gemm_fp16", "gemm_w8a16")
PROBE_FLAGS = ["-O3", "-std=c++17", "--offload-arch=%s" % ARCH,
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wno-unused-result"]


def probe_path(op: str) -> str:
    return os.path.join(BUILD, "ship_probe_%s" % op)


def _compile_delivery_unit(job):
    op, name = job
    d = os.path.join(SHIPPED, op, "gfx950")
    src = os.path.join(d, name)
    obj = os.path.join(BUILD, "delivery_%s_%s" % (op, name.replace(".hip", ".o")))
    cmd = [HIPCC] + PROBE_FLAGS + unit_flags(src) + ["-I", d, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True, cwd=d)
    if r.returncode != 0:
        raise RuntimeError("delivery-only compile of %s failed:\n%s\n%s"
                           % (src, " ".join(cmd), r.stderr[-6000:]))
    return obj


def delivery_units(op: str):
    d = os.path.join(SHIPPED, op, "gfx950")
    return [n for n in ("launch.hip", "launch_prefill.hip", "ship_probe.hip")
            if os.path.exists(os.path.join(d, n))]


def build_probes(ex) -> list:
    jobs = [(op, n) for op in PROBE_OPS for n in delivery_units(op)]
    objs = dict(zip(jobs, ex.map(_compile_delivery_unit, jobs)))
    out = []
    for op in PROBE_OPS:
        exe = probe_path(op)
        cmd = [HIPCC, "--offload-arch=%s" % ARCH, "-o", exe + ".tmp"] + \
            [objs[(op, n)] for n in delivery_units(op)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError("ship probe link failed for %s:\n%s" % (op, r.stderr[-4000:]))
        os.replace(exe + ".tmp", exe)
        out.append(exe)
    return out


# The measure stage's machine calibration probes (tempo/plugins/gfx950/calibrate.py): a library of
# their own, outside the product path.
CALIB_SRC = os.path.join(ROOT, "tempo", "plugins", "gfx950", "calib", "calib.hip")
CALIB_OUT = os.path.join(ROOT, "tempo", "plugins", "gfx950", "calib", "libgfx950_calib.so")


def build_calib() -> str:
    cmd = [HIPCC] + FLAGS + ["-shared", "-o", CALIB_OUT + ".tmp", CALIB_SRC]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed on %s:\n%s" % (CALIB_SRC, r.stderr[-4000:]))
    os.replace(CALIB_OUT + ".tmp", CALIB_OUT)
    return CALIB_OUT


def build(verbose: bool = False, probes: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    regenerate()
    with cf.ThreadPoolExecutor(max_workers=8) as ex:
        fut_probes = ex.submit(build_probes, ex) if probes else None
        fut_calib = ex.submit(build_calib)
        objs = list(ex.map(_compile, UNITS))
        cmd = [HIPCC, "--offload-arch=%s" % ARCH, "-shared", "-fPIC", "-o", OUT + ".tmp"] + objs
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError("link failed:\n%s" % r.stderr[-4000:])
        os.replace(OUT + ".tmp", OUT)
        if fut_probes is not None:
            fut_probes.result()
        fut_calib.result()
    if verbose:
        print(OUT)
    return OUT


if __name__ == "__main__":
    build(verbose=True)
