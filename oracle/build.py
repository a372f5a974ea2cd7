"""Build recipe for the CPU oracle (test infrastructure only): oracle/liboracle.so.

    python3 oracle/build.py

gcc on the one C file; x86-64-v3 (AVX2 + FMA + F16C) so the library built here also runs on
the GPU box's host CPU.  -ffp-contract=off keeps every rounding where the C source puts it
(the only fused operations are the explicit fmaf calls that restate the naive kernel's FMA).

The reference's own C/CUDA for this path is not built here: it is CUDA with sm_70 inline PTX
(kernels/naive/gemm_fp16.cu, ship_probe.cu) and needs nvcc, which this image does not have.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "tempo_oracle.c")
OUT = os.path.join(HERE, "liboracle.so")


def build(verbose: bool = False) -> str:
    cmd = [
        "gcc", "-O3", "-march=x86-64-v3", "-fopenmp", "-fPIC", "-shared",
        "-fno-fast-math", "-ffp-contract=off", "-std=c11", "-Wall",
        SRC, "-o", OUT + ".tmp", "-lm",
    ]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    os.replace(OUT + ".tmp", OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
