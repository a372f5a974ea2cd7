"""Plugin gfx950 -- AMD Instinct MI355X (CDNA4) for the Tempolator pipeline, contract tempo/arch/1.

Sections (reference layout tempo/plugins/sm70/): machine.py (closed rate table,
data/machine.json), memory.py (LDS bank law), tensor.py (MFMA fragment maps), resources.py
(unified VGPR/AGPR file, LDS, wave64 occupancy, five verdict codes), sync.py (register-staged vs
LDS-DMA transactions), classifier.py (AMDGPU ISA of our own builds), space.py + lower.py
(skeletons: axes, legal hyperforms, atoms, render), toolchain.py (hipcc + resource remarks +
llvm-objdump), counters.py (rocprofv3).  Kernels: skeletons/; frozen deliveries:
kernels/shipped/{gemm_fp16,gemm_w8a16}/gfx950 (ship.py).

Self-test:  python3 -m tempo.plugins.gfx950
"""
from __future__ import annotations

from ..base import (CONTRACT, RESOURCE_CODES, OpSpec, Report, UnknownSymbol,
                    acc_regs_per_thread, operand_loads_per_mma)
from .classifier import Gfx950Classifier
from .counters import Gfx950Meters
from .lower import Gfx950Skeletons
from .machine import Gfx950Machine
from .memory import Gfx950Memory
from .resources import Gfx950Resources
from .sync import Gfx950Sync
from .tensor import Gfx950TensorUnit, result_map


class Gfx950Plugin:
    id = "gfx950"
    contract = CONTRACT
    description = ("AMD Instinct MI355X (gfx950, CDNA4): 256 CUs in 8 XCDs, wave64, MFMA "
                   "32x32x16/16x16x32 f16, 160 KiB LDS, LDS-DMA loads, 288 GB HBM3E.")

    def __init__(self):
        self.machine = Gfx950Machine()
        self.memory = Gfx950Memory()
        self.tensor = Gfx950TensorUnit()
        self.resources = Gfx950Resources()
        self.sync = Gfx950Sync()
        self.classifier = Gfx950Classifier()
        self.skeletons = Gfx950Skeletons()
        from .toolchain import Gfx950Toolchain

        self.toolchain = Gfx950Toolchain()
        self.meters = Gfx950Meters()

    def declared_stubs(self):
        return (
            "the bound's HBM channel uses each CU's share of the spec peak (CAP.HBM_SHARE, an "
            "upper bound); the MEASURED modes (HBM.READ_PURE / READ / COPY) are reported next "
            "to it, not used inside it, because a measured streaming rate is not an upper bound "
            "on what a kernel may reach",
            "clock locking (Meters.clock_lock) is not offered: clocks are recorded, not set",
            "classifier.control_fields: the AMD ISA has no scheduling control words",
            "the attention skeleton (skeletons/fmha_fwd) has one tile: its space holds one "
            "hyperform per head dimension (128 or 256) and mask",
            "the fused silu(gate)*up epilogue of the interleaved prefill kernels has no split-K "
            "form: mid-M gate/up shapes with few column tiles leave CUs idle",
        )

    def selftest(self) -> Report:
        r = Report("gfx950")
        M = self.machine
        syms = M.symbols()
        r.check("rate table is non-empty", len(syms) > 0, "%d symbols" % len(syms))
        bad = [s.symbol for s in syms.values() if s.status == "MEASURED" and
               (s.prov is None or s.prov.card is None or s.prov.card.foreign_procs != 0)]
        r.check("every MEASURED rate carries a clean card", not bad, ", ".join(bad[:3]))
        # bandwidth as three named modes, not one number (reference sm70/__init__.py:110-131)
        modes = ("hbm_read_pure", "hbm_read", "hbm_copy")
        rates = [M.peak(k) for k in modes]
        r.check("HBM bandwidth is declared as three MEASURED modes",
                all(x.status == "MEASURED" for x in rates),
                ", ".join("%s %s" % (x.symbol, x.status) for x in rates))
        vals = [x.value for x in rates]
        r.check("the three modes differ (else the symbols are redundant)", len(set(vals)) == 3,
                "%s" % vals)
        r.check("every mode names its access pattern", all("MODE:" in x.note for x in rates))
        r.check("the spec HBM peak is declared and differs from every mode",
                M.peak("hbm_spec").status == "SPEC" and M.peak("hbm_spec").value not in vals)
        # a measured rate above the declared ceiling of the same resource falsifies the ceiling
        lds = M.rate("LDS.READ")
        r.check("measured LDS rate within its UPPER_BOUND",
                lds.value <= M.rate("CAP.LDS").value,
                "%.1f vs %.1f B/clk/CU" % (lds.value, M.rate("CAP.LDS").value))
        mf = M.rate("MFMA.F16")
        sclk = M.rate("CLOCK.SCLK_MFMA_PROBE").value
        cap_tf = M.rate("GEOM.SMS").value * sclk * 1e6 * M.rate("CAP.MFMA_F16").value / 1e12
        r.check("measured MFMA rate within the issue ceiling at its own clock",
                mf.value <= cap_tf, "%.1f vs %.1f TFLOP/s at %d MHz" % (mf.value, cap_tf, sclk))
        try:
            M.rate("CAP.NONEXISTENT")
            r.check("closed table refuses an unknown symbol", False)
        except UnknownSymbol:
            r.check("closed table refuses an unknown symbol", True)
        caps = M.channels()
        r.check("no SPEC rate is a channel capacity",
                all(c.capacity.status != "SPEC" for c in caps.values()))
        peak = M.peak("tensor_dense")
        derived = M.rate("GEOM.SMS").value * M.rate("CLOCK.SCLK_PEAK").value * 1e6 * \
            M.rate("CAP.MFMA_F16").value / 1e12
        r.check("fp16 peak = CUs x clock x MFMA flop/clk", abs(derived - peak.value) < 1.0,
                "%.1f vs %.1f TFLOP/s" % (derived, peak.value))
        # tensor unit: result maps are bijections and acc counts follow from them
        for ms in (32, 16):
            rows, cols = result_map(ms)
            cells = {(a, b) for a, b in zip(rows.ravel(), cols.ravel())}
            r.check("MFMA %dx%d result map is a bijection" % (ms, ms), len(cells) == ms * ms)
        op32 = self.tensor.select(("fp16", "fp16"), "fp32")
        r.check("acc registers of a 128x128 wave tile = 256",
                acc_regs_per_thread((128, 128), op32) == 256)
        r.check("operand loads per MFMA of a 4x4 block tile = 0.5",
                operand_loads_per_mma((128, 128), op32) == 0.5)
        # resources: the five verdict codes are reachable
        R = self.resources
        codes = {
            R.verdict(256, 300, 200 * 1024, 256).code,       # LDS beyond 160 KiB
            R.verdict(128, 128, 64 * 1024, 40 * 64).code,    # more waves than a CU's slots
            R.verdict(400, 600, 64 * 1024, 256).code,        # max_live beyond 512
            R.verdict(128, 200, 64 * 1024, 512, 2).code,     # declared residency leaves 128
            R.verdict(128, 128, 64 * 1024, 256).code,
        }
        r.check("all five verdict codes are reachable", set(RESOURCE_CODES) <= codes,
                ",".join(sorted(codes)))
        occ = R.occupancy(512, 128 * 1024, 256)
        r.check("256x256 tile (512 regs, 128 KiB LDS) -> 1 workgroup per CU", occ.ctas_per_sm == 1)
        r.check("register budget at 4 waves/CU is 512, at 8 is 256",
                R.reg_budget(4) == 512 and R.reg_budget(8) == 256)
        # sync: the falsifier field differs between the two transaction kinds
        tk = {t.id: t.consumes_registers for t in self.sync.transactions()}
        r.check("LDS-DMA consumes no registers, register staging does",
                tk.get("gmem->lds:dma") is False and tk.get("gmem->vgpr->lds") is True)
        # skeletons: refusal and a non-empty space for the C1 shape
        op = OpSpec(kind="gemm", dtype_a="fp16", dtype_b="fp16", dtype_c="fp16", dtype_acc="fp32",
                    layout_a="k", layout_b="k", layout_c="n",
                    shapes={"M": 4096, "N": 15360, "K": 3840}, tol_rel_l2=3e-3)
        hs = list(self.skeletons.variants(op))
        r.check("C1 shape has legal hyperforms", len(hs) > 0, "%d" % len(hs))
        r.check("hyperform keys are injective", len({h.key for h in hs}) == len(hs))
        bad_op = OpSpec(kind="gemm", dtype_a="fp16", dtype_b="fp16", dtype_c="fp16",
                        dtype_acc="fp32", layout_a="k", layout_b="n", layout_c="n",
                        shapes={"M": 64, "N": 64, "K": 64})
        try:
            list(self.skeletons.variants(bad_op))
            r.check("layout b=n is refused structurally", False)
        except Exception as e:  # PluginCapabilityError
            r.check("layout b=n is refused structurally", type(e).__name__ == "PluginCapabilityError")
        src = self.skeletons.render(op, hs[0]).source
        r.check("render emits one explicit instantiation", src.count("template __global__") == 1)
        # the attention skeleton: one hyperform per head dimension and mask, rendered as the
        # shipped kernel's instantiation
        att = OpSpec(kind="attention", dtype_a="fp16", dtype_b="fp16", dtype_c="fp16",
                     dtype_acc="fp32", layout_a="d", layout_b="d", layout_c="d",
                     shapes={"B": 1, "H": 16, "HKV": 8, "SQ": 4096, "SK": 4096, "D": 256,
                             "CAUSAL": 1}, tol_rel_l2=3e-3)
        ah = list(self.skeletons.variants(att))
        r.check("attention (C5) has one hyperform", len(ah) == 1, ",".join(h.key for h in ah))
        asrc = self.skeletons.render(att, ah[0]).source
        r.check("attention renders fmha::k_fmha_fwd<256, true>",
                "template __global__ void fmha::k_fmha_fwd<256, true>(" in asrc)
        return r


def load():
    return Gfx950Plugin()
