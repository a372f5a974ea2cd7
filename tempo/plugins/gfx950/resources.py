"""gfx950: RESOURCES AND OCCUPANCY -- section 4 (reference pattern tempo/plugins/sm70/resources.py).

CDNA4 register law: one unified file of 512 registers per lane per SIMD, shared by arch VGPRs and
AGPRs (accumulators), allocated in granules of 8.  A SIMD holds floor(512 / regs) waves (at most
8); a workgroup of T lanes puts ceil(T/64/4) waves on each SIMD.  __launch_bounds__(T, MINB)
tells the compiler how many waves per SIMD it must leave room for, which sets its budget:
512 / (ceil(T/256) * MINB), rounded down to the granule (arch VGPRs alone never exceed 256).

Verdict codes (contract): WALL_SMEM (LDS beyond 160 KiB: the launch cannot happen), NO_BUDGET
(no workgroup fits a CU), WALL_REG (even one wave per SIMD cannot hold max_live), SPILL (the
declared budget is below max_live + overhead: the compiler will use scratch), FITS.
"""
from __future__ import annotations

import math

from ..base import Occupancy, Rate, ResourceVerdict
from .machine import Gfx950Machine

_M = Gfx950Machine()


def _i(sym: str) -> int:
    return int(_M.rate(sym).value)


class Gfx950Resources:
    def reg_budget(self, warps_per_sm: int) -> int:
        """Registers per lane available when `warps_per_sm` waves share a CU's 4 SIMDs."""
        isa = _i("GEOM.REG_ISA_LIMIT")
        gran = _i("GEOM.REG_ALLOC_GRANULARITY")
        simds = _i("GEOM.SCHEDULERS_PER_SM")
        if warps_per_sm <= 0:
            return isa
        per_simd = max(1, math.ceil(warps_per_sm / simds))
        return min(isa, (isa // per_simd) // gran * gran)

    def spill_threshold(self, max_live: int) -> int:
        return int(max_live + _M.rate("REG.OVERHEAD").value)

    def free_spills(self) -> int:
        return int(_M.rate("REG.FREE_SPILLS").value)

    def spill_cost(self, n: int) -> Rate:
        if n <= self.free_spills():
            return Rate("SPILL.COST", 1.0, "x", "MODEL", note="no spill")
        step = _M.rate("REG.SPILL_STEP")
        return Rate("SPILL.COST", step.value, "x", "MODEL", note=step.note)

    def _alloc(self, regs: int) -> int:
        gran = _i("GEOM.REG_ALLOC_GRANULARITY")
        return max(gran, int(math.ceil(regs / gran)) * gran)

    def occupancy(self, regs: int, smem_bytes: int, threads: int) -> Occupancy:
        """Resident waves per CU: registers per SIMD, wave slots, LDS per workgroup.  `regs` is
        what one wave holds; callers that start from an estimate clamp it to the declared budget
        first (the compiler never allocates beyond it: it spills instead)."""
        tpw = _i("GEOM.THREADS_PER_WARP")
        simds = _i("GEOM.SCHEDULERS_PER_SM")
        isa = _i("GEOM.REG_ISA_LIMIT")
        waves_wg = max(1, math.ceil(threads / tpw))
        per_simd_wg = max(1, math.ceil(waves_wg / simds))  # waves of one workgroup on a SIMD
        by_reg_waves = min(_i("GEOM.WAVES_PER_SIMD_MAX"), isa // self._alloc(max(1, regs)))
        wg_by_reg = by_reg_waves // per_simd_wg
        wg_by_slots = _i("GEOM.WARP_SLOTS_PER_SM") // waves_wg
        wg_by_lds = (_i("GEOM.SMEM_PER_SM") // smem_bytes) if smem_bytes > 0 else wg_by_slots
        ctas = max(0, min(wg_by_reg, wg_by_slots, wg_by_lds))
        limiter = "regs"
        if wg_by_lds < wg_by_reg and wg_by_lds <= wg_by_slots:
            limiter = "lds"
        elif wg_by_slots <= min(wg_by_reg, wg_by_lds):
            limiter = "wave_slots"
        return Occupancy(warps_per_sm=int(ctas * waves_wg), ctas_per_sm=int(ctas),
                         regs_per_thread=int(regs), limiter=limiter)

    def declared_budget(self, threads: int, min_ctas_per_sm: int = 1, bound_threads: int = 0) -> int:
        """The register budget __launch_bounds__(max(threads, bound_threads), min_ctas_per_sm)
        gives the compiler."""
        tpw = _i("GEOM.THREADS_PER_WARP")
        waves = max(1, math.ceil(max(threads, bound_threads) / tpw)) * max(1, int(min_ctas_per_sm))
        return self.reg_budget(waves)

    def verdict(self, regs: int, max_live: int, smem_bytes: int, threads: int,
                min_ctas_per_sm: int = 1, bound_threads: int = 0) -> ResourceVerdict:
        isa = _i("GEOM.REG_ISA_LIMIT")
        lds_max = _i("GEOM.SMEM_PER_CTA_MAX")
        budget = self.declared_budget(threads, min_ctas_per_sm, bound_threads)
        # the compiler holds a wave to the declared budget (spilling the rest), so residency is
        # computed from min(estimate, budget): an estimate above the budget is a spill question,
        # never a "cannot launch" one
        occ = self.occupancy(min(regs, budget), smem_bytes, threads)
        if smem_bytes > lds_max:
            return ResourceVerdict(False, "WALL_SMEM", occ,
                                   "LDS %d B > %d B per workgroup" % (smem_bytes, lds_max))
        if occ.ctas_per_sm <= 0:
            return ResourceVerdict(False, "NO_BUDGET", occ, "no workgroup is resident on a CU")
        need = self.spill_threshold(max_live)
        if need > isa:
            return ResourceVerdict(False, "WALL_REG", occ,
                                   "max_live %d + overhead = %d > %d registers per lane (advisory: "
                                   "pessimistic edge of the estimate)" % (max_live, need, isa))
        if need > budget:
            over = need - budget
            return ResourceVerdict(over <= self.free_spills(), "SPILL", occ,
                                   "needs %d registers, declared budget %d: %d values to scratch, "
                                   "cost x%.1f" % (need, budget, over, self.spill_cost(over).value))
        return ResourceVerdict(True, "FITS", occ,
                               "needs %d registers even at the pessimistic edge; budget %d; %d "
                               "workgroup(s) per CU, limited by %s"
                               % (need, budget, occ.ctas_per_sm, occ.limiter))

    def wave_quantum(self, occ: Occupancy) -> int:
        """Workgroups that run concurrently on the whole part (the grid's useful multiple)."""
        return _i("GEOM.SMS") * max(1, occ.ctas_per_sm)

    def declared_bounds_required(self) -> bool:
        """True: the budget the compiler uses comes from __launch_bounds__."""
        return True
