"""gfx950: METERS -- section 8b: counters through rocprofv3 (reference pattern
tempo/plugins/sm70/counters.py, which drives ncu).

Counter groups are the names rocprofv3 --list-avail prints on MI355X.  One --pmc pass may hold at
most 8 SQ_, 4 TCC_ (FETCH_SIZE alone takes 3, WRITE_SIZE 2), 4 TCP_, 2 TA_, 2 TD_ and 2 GRBM_
counters, so every group below fits one pass, and profile() runs one pass per call.
A resource share is not a time share: a busy counter says what was occupied, not what bound.
"""
from __future__ import annotations

import contextlib
import csv
import glob
import os
import shutil
import subprocess
import tempfile
from pathlib import Path

from ..base import NotSupported

GROUPS = {
    # matrix-core activity: MFMA_BUSY / (GRBM_GUI_ACTIVE * SIMDs) is the utilisation
    "mfma": ["SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU_MFMA_MOPS_F16", "GRBM_GUI_ACTIVE"],
    # HBM traffic (derived, KiB per dispatch): one pass each -- they do not fit together
    "hbm_read": ["FETCH_SIZE"],
    "hbm_write": ["WRITE_SIZE"],
    # LDS bank conflicts against LDS activity
    "lds": ["SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE", "SQ_INSTS_LDS", "GRBM_GUI_ACTIVE"],
    # memory pipeline occupancy
    "vmem": ["SQ_INSTS_VMEM_RD", "SQ_INSTS_VMEM_WR", "TA_BUSY_avr", "GRBM_GUI_ACTIVE"],
    # L2 behaviour
    "l2": ["TCC_HIT_sum", "TCC_MISS_sum"],
    # waves and stalls
    "waves": ["SQ_WAVES", "SQ_WAVE_CYCLES", "SQ_BUSY_CYCLES", "SQ_WAIT_INST_ANY"],
}


class Gfx950Meters:
    def counters(self, kind: str) -> list:
        if kind not in GROUPS:
            raise NotSupported("counter group %r not declared (known: %s)"
                               % (kind, ", ".join(sorted(GROUPS))))
        return list(GROUPS[kind])

    def profile(self, binary: Path, kernel: str, counters: list, args: list = ()) -> dict:
        """Run `binary args` once under rocprofv3 --pmc and return {counter: value} summed over
        the dispatches whose kernel name contains `kernel`.  Needs a GPU."""
        exe = shutil.which("rocprofv3")
        if exe is None:
            raise NotSupported("rocprofv3 not found")
        out = Path(tempfile.mkdtemp(prefix="tempo_pmc_", dir=os.environ.get("TMPDIR", "/tmp")))
        cmd = [exe, "--pmc"] + list(counters) + ["--output-format", "csv", "-d", str(out), "--",
                                                 str(binary)] + list(args)
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
        files = glob.glob(str(out / "**" / "*counter_collection.csv"), recursive=True)
        if not files:
            raise RuntimeError("rocprofv3 wrote no counter file (rc %d): %s" % (r.returncode, r.stderr[-2000:]))
        return parse_counter_csv(files[0], kernel)

    @contextlib.contextmanager
    def clock_lock(self, card: int, mhz: int):
        # Changing clocks needs privileges this deployment does not grant; the measure stage
        # records the clock it observed instead (CardState).
        raise NotSupported("clock locking is not available; clocks are recorded, not set")
        yield  # pragma: no cover


def parse_counter_csv(path: str, kernel: str = "") -> dict:
    """Sum Counter_Value per Counter_Name over rows whose Kernel_Name contains `kernel`."""
    out = {}
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            name = row.get("Kernel_Name", "")
            if kernel and kernel not in name:
                continue
            c = row.get("Counter_Name")
            try:
                v = float(row.get("Counter_Value", "nan"))
            except ValueError:
                continue
            out[c] = out.get(c, 0.0) + v
    return out
