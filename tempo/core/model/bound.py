"""Time lower bound T >= max(ResMII, RecMII) over the plugin's channels (reference
tempo/core/model/bound.py:61-162).  No architecture name, no hardware number.

* A bound, not a prediction.
* The model may stay SILENT: if no channel with a usable capacity carries load, it says so
  instead of returning a quietly wrong number.
* SPEC capacities are refused (spec_forbidden_in_time_bound); NOT_MEASURED ones are skipped and
  listed.
"""
from __future__ import annotations

from dataclasses import dataclass, field

from tempo.plugins.base import spec_forbidden_in_time_bound


@dataclass
class Bound:
    T: float
    res_mii: float
    rec_mii: float
    binding: str
    per_channel: dict = field(default_factory=dict)
    silent: bool = False
    silent_reason: str = ""
    uses_not_measured: tuple = ()

    def render(self) -> str:
        if self.silent:
            return "MODEL SILENT: %s" % self.silent_reason
        head = "T >= %.2f cycles (ResMII %.2f, RecMII %.2f), bound by %s" % (
            self.T, self.res_mii, self.rec_mii, self.binding)
        if self.uses_not_measured:
            head += "\n  note: rests on NOT MEASURED rates: " + ", ".join(self.uses_not_measured)
        return head


def res_mii(atoms, channels, warps_per_sm: int = 1, schedulers: int = 1):
    from tempo.core.ir.atom import channel_load

    per, not_measured = {}, []
    for name, load in channel_load(atoms).items():
        ch = channels.get(name)
        if ch is None:
            continue
        cap = ch.capacity
        spec_forbidden_in_time_bound(cap)
        if cap.status == "NOT_MEASURED":
            not_measured.append(cap.symbol)
            continue
        if ch.scope == "sm":
            per[name] = (load * max(1, warps_per_sm)) / max(1e-12, cap.value)
        else:
            per[name] = load * cap.value
    return per, tuple(not_measured)


def rec_mii(atoms) -> float:
    """Maximum mean cycle of the loop-carried dependence graph (Karp)."""
    idx = {a.uid: i for i, a in enumerate(atoms)}
    edges = []
    for a in atoms:
        for d in a.deps:
            if d.src_uid in idx and int(d.distance) > 0:
                src = atoms[idx[d.src_uid]]
                edges.append((idx[d.src_uid], idx[a.uid], float(src.latency) + float(d.min_gap),
                              int(d.distance)))
    if not edges:
        return 0.0
    # ratio-weighted cycles: lambda = max over cycles of sum(w) / sum(distance); binary search
    # on lambda with Bellman-Ford positive-cycle detection (exact enough for a lower bound)
    n = len(atoms)

    def has_cycle(lam):
        dist = [0.0] * n
        for _ in range(n):
            changed = False
            for u, v, w, k in edges:
                if dist[u] + w - lam * k > dist[v] + 1e-12:
                    dist[v] = dist[u] + w - lam * k
                    changed = True
            if not changed:
                return False
        return True

    lo, hi = 0.0, sum(w for _, _, w, _ in edges) + 1.0
    if not has_cycle(lo):
        return 0.0
    for _ in range(60):
        mid = 0.5 * (lo + hi)
        if has_cycle(mid):
            lo = mid
        else:
            hi = mid
    return lo


def bound(atoms, channels, warps_per_sm: int = 1, schedulers: int = 1) -> Bound:
    per, nm = res_mii(atoms, channels, warps_per_sm, schedulers)
    if not per:
        return Bound(T=float("nan"), res_mii=float("nan"), rec_mii=float("nan"), binding="",
                     silent=True,
                     silent_reason="no loaded channel has a usable (measured or upper-bound) rate"
                     + (" (not measured: %s)" % ", ".join(nm) if nm else ""),
                     uses_not_measured=nm)
    binding = max(per, key=per.get)
    r = per[binding]
    rec = rec_mii(atoms)
    return Bound(T=max(r, rec), res_mii=r, rec_mii=rec,
                 binding=binding if r >= rec else "RECURRENCE", per_channel=per,
                 uses_not_measured=nm)


def headroom(measured_cycles: float, b: Bound) -> float:
    if b.silent or not b.T or b.T != b.T:
        return float("nan")
    return measured_cycles / b.T
