"""The card passport: the state of the GPU before and after a measurement.

The reference records, for every shipped number, the card index, its name, the clock it ran at
and the number of foreign processes on the card before and after the run
(kernels/shipped/gemm_fp16/sm_70/manifest.json:107-113), and its method counts the neighbours
before and after every measurement, judging a neighbour by what it draws, not by a utilisation
flag (docs/MEASURE_DISCIPLINE.md:70-77).  Its loader accepts a MEASURED rate only with a card
state showing no foreign process (tempo/plugins/registry.py:67-76).

Here clocks cannot be locked (the deployment grants no such privilege), so the passport records
the clocks it observes.  Sources, read without touching the GPU from this process:
  * `amd-smi metric --clock --power --temperature --json`: the engine clock of every XCD
    (gfx_0 ... gfx_7), the memory clock, socket power, temperatures, whether clocks are locked;
  * `amd-smi process --json` and /sys/class/kfd/kfd/proc/<pid>: the processes holding the GPU.
    A process is foreign when it is not this process, one of its ancestors or one of its
    descendants.  Inside a container only the container's processes are visible (on the pool's
    boxes amd-smi lists none and the kfd directory is hidden); the passport says which sources
    it could read;
  * the draw: a card that runs nobody's work sits at its idle engine clock, below the lowest
    working DPM level (500 MHz on MI355X; the pool's idle cards read 90-200 MHz).  `gfx_idle`
    records that, and clean() requires it of the state taken before a measurement starts, so a
    neighbour the process list cannot see is still caught by what it draws.
"""
from __future__ import annotations

import json
import os
import subprocess
import time
from typing import Optional

AMD_SMI = "amd-smi"
IDLE_MHZ = 500  # the lowest working engine-clock DPM level; an idle card sits below it


def _run(cmd, timeout=30) -> Optional[str]:
    try:
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    except Exception:
        return None
    return r.stdout if r.returncode == 0 else None


def _value(x):
    """amd-smi leaves are either {"value": v, "unit": u}, a bare number or "N/A"."""
    if isinstance(x, dict) and "value" in x:
        x = x["value"]
    if isinstance(x, (int, float)):
        return x
    try:
        return float(x)
    except (TypeError, ValueError):
        return None


def _gpu_entry(doc, index: int):
    """The record of GPU `index` in an amd-smi JSON document (a list of per-GPU records, or an
    object holding one under a top-level key)."""
    if isinstance(doc, dict):
        for k in ("gpu_data", "data", "gpus"):
            if isinstance(doc.get(k), list):
                doc = doc[k]
                break
        else:
            return doc
    if isinstance(doc, list):
        for e in doc:
            if isinstance(e, dict) and e.get("gpu") == index:
                return e
        return doc[index] if 0 <= index < len(doc) else None
    return None


def parse_metric(text: str, index: int = 0) -> dict:
    """Clocks, power and temperature of GPU `index` from `amd-smi metric ... --json` output."""
    out = {}
    try:
        e = _gpu_entry(json.loads(text), index)
    except (ValueError, TypeError):
        return out
    if not isinstance(e, dict):
        return out
    clk = e.get("clock") or {}
    gfx = [_value(v.get("clk")) for k, v in clk.items()
           if k.startswith("gfx") and isinstance(v, dict)]
    gfx = [g for g in gfx if g is not None]
    if gfx:
        out["gfx_clock_mhz"] = sum(gfx) / len(gfx)
        out["gfx_clock_mhz_min"] = min(gfx)
        out["gfx_clock_mhz_max"] = max(gfx)
    locked = [v.get("clk_locked") for k, v in clk.items()
              if k.startswith("gfx") and isinstance(v, dict)]
    if locked:
        out["clk_locked"] = locked[0]
    maxc = [_value(v.get("max_clk")) for k, v in clk.items()
            if k.startswith("gfx") and isinstance(v, dict)]
    maxc = [m for m in maxc if m is not None]
    if maxc:
        out["gfx_clock_max_mhz"] = max(maxc)
    mem = clk.get("mem_0")
    if isinstance(mem, dict) and _value(mem.get("clk")) is not None:
        out["mem_clock_mhz"] = _value(mem.get("clk"))
    pw = e.get("power") or {}
    for k in ("socket_power", "current_socket_power", "average_socket_power"):
        v = _value(pw.get(k))
        if v is not None:
            out["power_w"] = v
            break
    temp = e.get("temperature") or {}
    for k in ("hotspot", "edge"):
        v = _value(temp.get(k))
        if v is not None:
            out["temperature_c"] = v
            break
    return out


def parse_processes(text: str, index: int = 0) -> Optional[list]:
    """PIDs of the processes amd-smi lists on GPU `index` (None if the output has no list)."""
    try:
        doc = json.loads(text)
    except (ValueError, TypeError):
        return None
    e = _gpu_entry(doc, index)
    if not isinstance(e, dict):
        return None
    procs = e.get("process_list", e.get("processes"))
    if procs is None:
        return None
    pids = []
    for p in procs if isinstance(procs, list) else [procs]:
        if isinstance(p, dict):
            info = p.get("process_info", p)
            pid = info.get("pid") if isinstance(info, dict) else None
            if isinstance(pid, int):
                pids.append(pid)
    return pids


def kfd_pids() -> Optional[list]:
    """PIDs with the GPU driver open (/sys/class/kfd/kfd/proc lists one directory per process)."""
    d = "/sys/class/kfd/kfd/proc"
    try:
        return sorted(int(x) for x in os.listdir(d) if x.isdigit())
    except OSError:
        return None


def _parent(pid: int) -> Optional[int]:
    try:
        with open("/proc/%d/stat" % pid) as f:
            return int(f.read().rsplit(")", 1)[1].split()[1])
    except (OSError, IndexError, ValueError):
        return None


def own_tree() -> set:
    """This process, its ancestors and its descendants."""
    me = os.getpid()
    tree = {me}
    p = _parent(me)
    while p and p not in tree:
        tree.add(p)
        p = _parent(p)
    try:
        pids = [int(x) for x in os.listdir("/proc") if x.isdigit()]
    except OSError:
        pids = []
    tree.update(q for q in pids if _is_descendant(q, me))
    return tree


def _is_descendant(pid: int, root: int) -> bool:
    seen = set()
    p = pid
    while p and p not in seen:
        if p == root:
            return True
        seen.add(p)
        p = _parent(p)
    return False


def snapshot(index: int = 0) -> dict:
    """The card's state now: {index, time, clocks, power, temperature, foreign_procs, ...}."""
    out = {"index": index, "time": time.strftime("%Y-%m-%dT%H:%M:%S")}
    sources = []
    m = _run([AMD_SMI, "metric", "-g", str(index), "--clock", "--power", "--temperature",
              "--json"])
    if m is not None:
        got = parse_metric(m, index)
        if got:
            out.update(got)
            sources.append("amd-smi metric")
    if "gfx_clock_mhz_max" in out:
        out["gfx_idle"] = out["gfx_clock_mhz_max"] < IDLE_MHZ
    pids = set()
    seen_any = False
    p = _run([AMD_SMI, "process", "-g", str(index), "--json"])
    if p is not None:
        got = parse_processes(p, index)
        if got is not None:
            pids.update(got)
            seen_any = True
            sources.append("amd-smi process")
    k = kfd_pids()
    if k is not None:
        pids.update(k)
        seen_any = True
        sources.append("kfd proc")
    if seen_any:
        mine = own_tree()
        foreign = sorted(x for x in pids if x not in mine)
        out["foreign_procs"] = len(foreign)
        out["foreign_pids"] = foreign
    else:
        out["foreign_procs"] = None
    out["sources"] = sources
    return out


def wait_idle(index: int = 0, timeout_s: float = 10.0, poll_s: float = 0.5) -> dict:
    """Snapshots until the card is idle by its clock (work of an earlier step winds down over a
    second or two) or `timeout_s` passes; returns the last snapshot, with the wait recorded."""
    t0 = time.time()
    while True:
        s = snapshot(index)
        if s.get("gfx_idle", True) or time.time() - t0 >= timeout_s:
            s["waited_s"] = round(time.time() - t0, 1)
            return s
        time.sleep(poll_s)


def passport(before: dict, after: dict, name: str = "") -> dict:
    """The manifest's card block (reference manifest.json:107-113 keys, clocks observed rather
    than locked)."""
    def g(d, k):
        return d.get(k) if isinstance(d, dict) else None

    return {
        "index": g(before, "index"),
        "name": name,
        "clock_locked_mhz": None,
        "clk_locked": g(before, "clk_locked"),
        "gfx_clock_mhz_before": g(before, "gfx_clock_mhz"),
        "gfx_clock_mhz_after": g(after, "gfx_clock_mhz"),
        "gfx_clock_max_mhz": g(before, "gfx_clock_max_mhz"),
        "mem_clock_mhz": g(before, "mem_clock_mhz"),
        "power_w_before": g(before, "power_w"),
        "power_w_after": g(after, "power_w"),
        "gfx_idle_before": g(before, "gfx_idle"),
        "foreign_procs_before": g(before, "foreign_procs"),
        "foreign_procs_after": g(after, "foreign_procs"),
        "sources": g(before, "sources"),
        "time_before": g(before, "time"),
        "time_after": g(after, "time"),
    }


def clean(before: dict, after: dict) -> bool:
    """A measurement counts only when no foreign process was seen before or after it and, where
    the clock was readable, the card was idle (by its draw) before it started."""
    return (before.get("foreign_procs") == 0 and after.get("foreign_procs") == 0
            and before.get("gfx_idle", True) is True)


if __name__ == "__main__":
    print(json.dumps(snapshot(), indent=1))
