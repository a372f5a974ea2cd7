"""Run the delivery-only ship probes on the GPU (built by `python3 -m cuda_tempiler_amd.build`
from each delivery's own directory: kernels/shipped/<op>/gfx950/ship_probe.hip).  Each probe is a
separate process; it prints one line per shape and exits 0 when every shape passed the
reference's acceptance rule (kernels/shipped/gemm_fp16/sm_70/ship_probe.cu:35-98) and bit
equality with the exact closed form."""
import os
import subprocess

import pytest

from tests.gpu_util import say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("op", ["gemm_fp16", "gemm_w8a16"])
def test_ship_probe(gpu, op):
    from cuda_tempiler_amd import build as B

    exe = B.probe_path(op)
    assert os.path.exists(exe), "ship probe not built: run python3 -m cuda_tempiler_amd.build"
    say("ship probe", op)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=180)
    say(r.stdout)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-2000:]
    assert "FAIL 0" in r.stdout
