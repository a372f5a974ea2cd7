"""gfx950: MACHINE -- section 1 of the contract (reference pattern tempo/plugins/sm70/machine.py).

The closed rate table is data (data/machine.json); a symbol outside it is refused
(UnknownSymbol, gate G4), never defaulted.  Status discipline:
  SPEC          datasheet numbers (CU count, LDS size, peaks) -- never inside a time bound;
  UPPER_BOUND   issue ceilings derived from the ISA (MFMA flop per clock, LDS and L2->CU bytes
                per clock) -- legal as channel capacities because a rate ceiling gives a LOWER
                time bound;
  MODEL         estimates (latencies, register overhead);
  MEASURED      numbers taken on a clean card, with its CardState;
  NOT_MEASURED  declared, not yet taken (the bound skips and names them).
"""
from __future__ import annotations

import json
import os
from typing import Mapping

from ..base import CardState, Channel, Provenance, Rate, closed_table_get, not_measured, rate

HERE = os.path.dirname(os.path.abspath(__file__))
_TABLE = None


def _load_table() -> Mapping[str, Rate]:
    global _TABLE
    if _TABLE is None:
        with open(os.path.join(HERE, "data", "machine.json"), encoding="utf-8") as f:
            d = json.load(f)
        t = {}
        for sym, r in d["rates"].items():
            if r["status"] == "NOT_MEASURED" or r["value"] is None:
                t[sym] = not_measured(sym, r["units"], r.get("note", ""))
            else:
                t[sym] = rate(sym, r["value"], r["units"], r["status"], r.get("note", ""),
                              prov=_prov(r.get("prov")))
        _TABLE = t
    return _TABLE


def _prov(p):
    """Provenance of a rate as the table stores it (calibrate.py writes it for MEASURED rates)."""
    if not p:
        return None
    c = p.get("card")
    cs = None if c is None else CardState(index=int(c["index"]), clock_mhz=int(c["clock_mhz"]),
                                          foreign_procs=c["foreign_procs"], date=str(c["date"]))
    return Provenance(tool=p["tool"], counter=p.get("counter"), version=str(p["version"]),
                      date=str(p["date"]), who=p["who"], observability=p["observability"],
                      card=cs)


class Gfx950Machine:
    def arch(self) -> str:
        return "gfx950"

    def symbols(self) -> Mapping[str, Rate]:
        return dict(_load_table())

    def rate(self, symbol: str) -> Rate:
        return closed_table_get(_load_table(), symbol)

    def channels(self) -> Mapping[str, Channel]:
        """Channels of the bound model, all per compute unit (scope "sm"): footprints are per
        wave, the bound multiplies by resident waves and divides by the CU's per-clock
        capacity.  HBM is the device-wide floor: every CU carries 1/CUS of the operation's HBM
        bytes against its share of the HBM peak, so a grid spread over more CUs cannot bound
        itself below bytes / peak."""
        return {
            "MFMA": Channel("MFMA", "sm", self.rate("CAP.MFMA_F16")),
            "LDS": Channel("LDS", "sm", self.rate("CAP.LDS")),
            "VMEM": Channel("VMEM", "sm", self.rate("CAP.VMEM_L2")),
            "HBM": Channel("HBM", "sm", self.rate("CAP.HBM_SHARE")),
        }

    def latency(self, atom_class: str) -> Rate:
        return self.rate("LATENCY." + atom_class)

    def sms(self) -> Rate:
        return self.rate("GEOM.SMS")

    def schedulers_per_sm(self) -> Rate:
        return self.rate("GEOM.SCHEDULERS_PER_SM")

    def warp_slots_per_sm(self) -> Rate:
        return self.rate("GEOM.WARP_SLOTS_PER_SM")

    def threads_per_warp(self) -> Rate:
        return self.rate("GEOM.THREADS_PER_WARP")

    def smem_per_sm(self) -> Rate:
        return self.rate("GEOM.SMEM_PER_SM")

    def smem_per_cta_max(self) -> Rate:
        return self.rate("GEOM.SMEM_PER_CTA_MAX")

    def regfile_words_per_sm(self) -> Rate:
        return self.rate("GEOM.REGFILE_WORDS_PER_SM")

    def clock_mhz(self) -> Rate:
        return self.rate("CLOCK.SCLK_PEAK")

    def peak(self, kind: str) -> Rate:
        table = {
            "tensor_dense": "PEAK.TENSOR_FP16_DENSE",
            "tensor_fp8_dense": "PEAK.TENSOR_FP8_DENSE",
            "hbm_spec": "PEAK.HBM",
            "hbm_read_pure": "HBM.READ_PURE",
            "hbm_read": "HBM.READ",
            "hbm_copy": "HBM.COPY",
            "tensor_measured": "MFMA.F16",
            "l2": "CAP.VMEM_L2",
        }
        if kind not in table:
            from ..base import UnknownSymbol

            raise UnknownSymbol("peak kind %r is not declared (known: %s)"
                                % (kind, ", ".join(sorted(table))))
        return self.rate(table[kind])
