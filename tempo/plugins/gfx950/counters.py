"""gfx950: METERS -- section 8b: counters through rocprofv3 (reference pattern
tempo/plugins/sm70/counters.py:74-104, which drives ncu; the measure stage's counter step is
tempo/core/measure/counters.py:38-43 in the reference).

Counter groups are the names rocprofv3 --list-avail prints on MI355X.  One --pmc pass may hold at
most 8 SQ_, 4 TCC_ (FETCH_SIZE alone takes 3, WRITE_SIZE 2), 4 TCP_, 2 TA_, 2 TD_ and 2 GRBM_
counters, so every group below fits one pass, and each pass is a run of its own.
A resource share is not a time share: a busy counter says what was occupied, not what bound.

How the raw numbers become the figures the measure stage reports (per dispatch):
  * HBM bytes = FETCH_SIZE (KiB) x 1024 x fetch_scale + WRITE_SIZE (KiB) x 1024 x write_scale.
    The scales come from a plain device copy of known size measured in the same pass
    (__amd_rocclr_copyBuffer: N bytes read and N written); on this part FETCH_SIZE counts half
    of the bytes read (scale 2.0) and WRITE_SIZE all of the bytes written (scale 1.0).
  * MFMA utilisation = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / XCDs x SIMDs) -- rocprofv3's
    own MfmaUtil expression; GRBM_GUI_ACTIVE is reported summed over the 8 XCDs.
  * engine clock = GRBM_GUI_ACTIVE / XCDs / dispatch duration (the counter run's timestamps).
    Under counter collection GRBM_GUI_ACTIVE also covers a fixed stretch around each dispatch
    (about 15k cycles on this part), so the clock and the GUI-based MFMA utilisation are only
    reported for dispatches of at least MIN_CLOCK_NS; shorter ones get the utilisation against
    the spec clock only.
  * MFMA utilisation at the spec clock = SQ_VALU_MFMA_BUSY_CYCLES / (duration x SPEC_GHZ x SIMDs):
    the share of the spec-peak matrix throughput the dispatch used, whatever clock it ran at.
  * LDS utilisation = SQ_LDS_IDX_ACTIVE / (GRBM_GUI_ACTIVE / XCDs x CUs) and bank conflicts per
    access = SQ_LDS_BANK_CONFLICT / (SQ_LDS_IDX_ACTIVE - SQ_LDS_BANK_CONFLICT): rocprofv3's own
    expressions (rocprofv3 -L prints them).
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
    # matrix-core activity: MFMA_BUSY / (GRBM_GUI_ACTIVE / XCDs * SIMDs) is the utilisation
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
    # where the wave-cycles go (SQ cycle counters count in units of 4 cycles; ratios to
    # SQ_WAVE_CYCLES of the waves group are unit-free)
    "stall": ["SQ_WAIT_ANY", "SQ_WAIT_INST_LDS", "SQ_ACTIVE_INST_ANY", "SQ_ACTIVE_INST_LDS",
              "SQ_ACTIVE_INST_VALU", "SQ_ACTIVE_INST_VMEM", "SQ_ACTIVE_INST_SCA", "SQ_INSTS_VALU",
              "GRBM_GUI_ACTIVE"],
    # issue mix: matrix cores busy and VALU work co-issued with them, scalar and memory issue
    "issue": ["SQ_VALU_MFMA_BUSY_CYCLES", "SQ_VALU_MFMA_COEXEC_CYCLES", "SQ_INST_CYCLES_SALU",
              "SQ_INST_CYCLES_VMEM_RD", "SQ_ACTIVE_INST_MISC", "SQ_ACTIVE_INST_FLAT",
              "SQ_WAVE_CYCLES", "GRBM_GUI_ACTIVE"],
    # the CU's memory intake: cycles the texture-address and LDS queues were full
    "fifo": ["SQ_VMEM_TA_ADDR_FIFO_FULL", "SQ_VMEM_TA_CMD_FIFO_FULL", "SQ_LDS_DATA_FIFO_FULL",
             "SQ_LDS_CMD_FIFO_FULL", "SQ_INSTS_VMEM", "SQ_WAVE_CYCLES", "GRBM_GUI_ACTIVE"],
}

COPY_KERNEL = "__amd_rocclr_copyBuffer"
XCDS = 8
CUS = 256
SIMDS = 1024  # 256 CUs x 4 SIMDs
SPEC_GHZ = 2.4  # the engine clock the published peaks assume
MIN_CLOCK_NS = 100_000


class Gfx950Meters:
    def counters(self, kind: str) -> list:
        if kind not in GROUPS:
            raise NotSupported("counter group %r not declared (known: %s)"
                               % (kind, ", ".join(sorted(GROUPS))))
        return list(GROUPS[kind])

    def profile(self, binary: Path, kernel: str, counters: list, args: list = ()) -> dict:
        """Run `binary args` once under rocprofv3 --pmc and return {counter: value} summed over
        the dispatches whose kernel name contains `kernel`.  Needs a GPU."""
        out = Path(tempfile.mkdtemp(prefix="tempo_pmc_", dir=os.environ.get("TMPDIR", "/tmp")))
        disp = self.run_pass([str(binary)] + list(args), counters, out)
        tot = {}
        for d in disp:
            if kernel and kernel not in d["kernel"]:
                continue
            for c, v in d["counters"].items():
                tot[c] = tot.get(c, 0.0) + v
        return tot

    def run_pass(self, argv: list, counters: list, out_dir, timeout: int = 600) -> list:
        """One rocprofv3 --pmc pass over the program `argv` (the program itself follows "--", no
        launcher in between); returns its dispatches in dispatch order (parse_dispatches).
        The caller's process must not have touched the GPU: it only starts the profiler."""
        exe = shutil.which("rocprofv3")
        if exe is None:
            raise NotSupported("rocprofv3 not found")
        out_dir = Path(out_dir)
        out_dir.mkdir(parents=True, exist_ok=True)
        cmd = ["timeout", "-s", "KILL", str(timeout), exe, "--pmc"] + list(counters) + [
            "--output-format", "csv", "-d", str(out_dir), "-o", "pass", "--"] + list(argv)
        with open(out_dir / "pass.log", "w") as log:
            r = subprocess.run(cmd, stdout=log, stderr=subprocess.STDOUT)
        files = glob.glob(str(out_dir / "**" / "*counter_collection.csv"), recursive=True)
        if not files:
            tail = open(out_dir / "pass.log", errors="replace").read()[-2000:]
            raise RuntimeError("rocprofv3 wrote no counter file (rc %d): %s" % (r.returncode, tail))
        return parse_dispatches(files[0])

    @contextlib.contextmanager
    def clock_lock(self, card: int, mhz: int):
        # Changing clocks needs privileges this deployment does not grant; the measure stage
        # records the clock it observed instead (CardState).
        raise NotSupported("clock locking is not available; clocks are recorded, not set")
        yield  # pragma: no cover


def parse_dispatches(path: str) -> list:
    """rocprofv3 counter CSV -> [{"id", "kernel", "grid", "start", "end", "counters": {...}}] in
    dispatch order (one CSV row per (dispatch, counter))."""
    by = {}
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            try:
                did = int(row["Dispatch_Id"])
                v = float(row.get("Counter_Value", "nan"))
            except (KeyError, ValueError):
                continue
            d = by.setdefault(did, dict(id=did, kernel=row.get("Kernel_Name", ""),
                                        grid=int(row.get("Grid_Size", 0) or 0),
                                        start=int(row.get("Start_Timestamp", 0) or 0),
                                        end=int(row.get("End_Timestamp", 0) or 0), counters={}))
            c = row.get("Counter_Name")
            d["counters"][c] = d["counters"].get(c, 0.0) + v
    return [by[k] for k in sorted(by)]


def parse_counter_csv(path: str, kernel: str = "") -> dict:
    """Sum of each counter over the dispatches whose kernel name contains `kernel`."""
    out = {}
    for d in parse_dispatches(path):
        if kernel and kernel not in d["kernel"]:
            continue
        for c, v in d["counters"].items():
            out[c] = out.get(c, 0.0) + v
    return out


def assign_segments(dispatches: list, segments: list, match: str) -> dict:
    """Attribute dispatches to the segments a counter-pass program declared, in order.

    segments: [{"label": str, "count": n, "copy_bytes": b (calibration segments only)}] in the
    order the program launched them; `count` is the number of DISPATCHES (launches x
    dispatches per launch).  A calibration segment takes the next `count` device-copy
    dispatches; any other segment takes the next `count` dispatches whose kernel name contains
    `match` (the library's namespace).  Other kernels (input generation) are skipped.
    Returns {label: [dispatch, ...]}; raises if the pass ran fewer dispatches than declared."""
    out, i = {}, 0
    for seg in segments:
        want = COPY_KERNEL if seg.get("copy_bytes") else match
        got = []
        while len(got) < seg["count"]:
            if i >= len(dispatches):
                raise RuntimeError("counter pass ended before segment %r was complete"
                                   % seg["label"])
            d = dispatches[i]
            i += 1
            if want in d["kernel"]:
                got.append(d)
        out[seg["label"]] = got
    return out


def _median(xs):
    xs = sorted(xs)
    n = len(xs)
    return 0.0 if n == 0 else (xs[n // 2] if n % 2 else 0.5 * (xs[n // 2 - 1] + xs[n // 2]))


def copy_scales(calib: list, copy_bytes: int) -> dict:
    """Scale factors that turn FETCH_SIZE / WRITE_SIZE (KiB) into bytes, from device copies of
    `copy_bytes` bytes (each reads and writes that many)."""
    out = {}
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        vals = [d["counters"][c] for d in calib if c in d["counters"]]
        if vals:
            out[c] = copy_bytes / (_median(vals) * 1024.0)
    return out


def derive(per_counter: dict, scales: dict, algorithmic_bytes: float = 0.0) -> dict:
    """Figures of one kernel from the per-dispatch medians of its counters (any subset)."""
    out = {}
    c = per_counter
    if "FETCH_SIZE" in c and "FETCH_SIZE" in scales:
        out["fetch_bytes"] = c["FETCH_SIZE"] * 1024.0 * scales["FETCH_SIZE"]
    if "WRITE_SIZE" in c and "WRITE_SIZE" in scales:
        out["write_bytes"] = c["WRITE_SIZE"] * 1024.0 * scales["WRITE_SIZE"]
    if "fetch_bytes" in out and "write_bytes" in out:
        out["hbm_bytes"] = out["fetch_bytes"] + out["write_bytes"]
        if algorithmic_bytes:
            out["traffic_over_algorithmic"] = out["hbm_bytes"] / algorithmic_bytes
    dur = c.get("_duration_ns", 0.0)
    if dur and "SQ_VALU_MFMA_BUSY_CYCLES" in c:
        out["mfma_util_spec_clock"] = c["SQ_VALU_MFMA_BUSY_CYCLES"] / (dur * SPEC_GHZ * SIMDS)
    gui = c.get("GRBM_GUI_ACTIVE")
    if gui:
        cycles = gui / XCDS
        out["gui_cycles"] = cycles
        if dur >= MIN_CLOCK_NS:
            out["sclk_ghz"] = cycles / dur
            if "SQ_VALU_MFMA_BUSY_CYCLES" in c:
                out["mfma_util"] = c["SQ_VALU_MFMA_BUSY_CYCLES"] / (cycles * SIMDS)
            if "SQ_LDS_IDX_ACTIVE" in c:  # rocprofv3's LDS utilisation expression
                out["lds_util"] = c["SQ_LDS_IDX_ACTIVE"] / (cycles * CUS)
    if "SQ_LDS_BANK_CONFLICT" in c and c.get("SQ_LDS_IDX_ACTIVE", 0) > c["SQ_LDS_BANK_CONFLICT"]:
        # conflict cycles per conflict-free LDS cycle (rocprofv3's bank-conflict expression)
        out["lds_conflicts_per_access"] = c["SQ_LDS_BANK_CONFLICT"] / (
            c["SQ_LDS_IDX_ACTIVE"] - c["SQ_LDS_BANK_CONFLICT"])
    for k, v in c.items():  # the raw per-launch medians as well
        if not k.startswith("_"):
            out[k] = v
    if "SQ_INSTS_VALU_MFMA_MOPS_F16" in c:
        out["mfma_flops"] = c["SQ_INSTS_VALU_MFMA_MOPS_F16"] * 512.0
    return out


def medians(dispatches: list, per_launch: int = 1) -> dict:
    """Per-counter median over launches, plus the median launch duration (ns).  A launch is
    `per_launch` consecutive dispatches (a split-K row dispatches its main kernel and then the
    reduction); its counters and durations are the sums over them."""
    launches = []
    for i in range(0, len(dispatches) - per_launch + 1, per_launch):
        grp = dispatches[i:i + per_launch]
        if [d["kernel"] for d in grp] != [d["kernel"] for d in dispatches[:per_launch]]:
            raise RuntimeError("launch %d dispatched %s, not the kernels of the first launch (%s)"
                               % (i // per_launch, [d["kernel"] for d in grp],
                                  [d["kernel"] for d in dispatches[:per_launch]]))
        cnt = {}
        for d in grp:
            for k, v in d["counters"].items():
                cnt[k] = cnt.get(k, 0.0) + v
        dur = sum(d["end"] - d["start"] for d in grp if d["end"] > d["start"])
        launches.append((cnt, dur))
    keys = set()
    for cnt, _ in launches:
        keys |= set(cnt)
    out = {k: _median([cnt[k] for cnt, _ in launches if k in cnt]) for k in keys}
    durs = [dur for _, dur in launches if dur > 0]
    if durs:
        out["_duration_ns"] = _median(durs)
    return out
