"""CPU gates of the gfx950 plugin against the tempo/arch/1 contract, and the core drivers.

Patterns of the reference's tests/test_gates.py (G1 loader, G2 refusals are contract errors and
never AttributeError, G4 closed rate table, G5 self-test) and tests/test_pipeline.py (oracle
gate, coverage, registry), restated for the gfx950 plugin.
"""
import os

import pytest

from tempo.plugins import base, registry

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NAIVE = os.path.join(ROOT, "kernels", "naive", "gemm_fp16.hip")
C1 = {"M": 4096, "N": 15360, "K": 3840}


@pytest.fixture(scope="module")
def plug():
    return registry.load("gfx950")


def _op(**kw):
    d = dict(kind="gemm", dtype_a="fp16", dtype_b="fp16", dtype_c="fp16", dtype_acc="fp32",
             layout_a="k", layout_b="k", layout_c="n", shapes=dict(C1), tol_rel_l2=3e-3)
    d.update(kw)
    return base.OpSpec(**d)


# ---- G1: loader ------------------------------------------------------------------------------
def test_g1_registry_loads_gfx950(plug):
    assert "gfx950" in registry.available()
    assert plug.id == "gfx950"
    assert plug.contract.split("/")[0:2] == ["tempo", "arch"]
    for section in ("machine", "memory", "tensor", "resources", "sync", "classifier",
                    "skeletons", "toolchain", "meters"):
        assert hasattr(plug, section), section
    assert isinstance(plug.declared_stubs(), tuple)


def test_g1_every_rate_is_a_rate(plug):
    for sym, r in plug.machine.symbols().items():
        assert isinstance(r, base.Rate), sym
        assert r.status in base.STATUS


# ---- G2: refusals are contract errors --------------------------------------------------------
def test_g2_unknown_symbol(plug):
    with pytest.raises(base.UnknownSymbol):
        plug.machine.rate("CAP.NOT_A_RATE")


def test_g2_layout_refused_structurally(plug):
    with pytest.raises(base.PluginCapabilityError):
        list(plug.skeletons.variants(_op(layout_b="n")))
    with pytest.raises(base.PluginCapabilityError):
        list(plug.skeletons.variants(_op(dtype_acc="fp16")))
    with pytest.raises(base.PluginCapabilityError):
        list(plug.skeletons.variants(_op(dtype_b="fp8")))


def test_g2_clock_lock_not_supported(plug):
    with pytest.raises(base.NotSupported):
        with plug.meters.clock_lock(0, 2400):
            pass


# ---- G4: closed rate table, SPEC never a time bound ------------------------------------------
def test_g4_spec_is_not_a_channel_capacity(plug):
    for name, ch in plug.machine.channels().items():
        assert ch.capacity.status != "SPEC", name


def test_g4_spec_refused_in_time_bound():
    r = base.Rate("PEAK.X", 1.0, "x", "SPEC")
    with pytest.raises(base.ContractError):
        base.spec_forbidden_in_time_bound(r)


# ---- the loader's refusals (reference tempo/plugins/registry.py:41-76) -------------------------
def test_loader_refuses_what_breaks_the_contract():
    import types

    with pytest.raises(base.ContractError):
        registry.load("no_such_plugin")

    def plugin(contract="tempo/arch/1", rates=None, raises=False):
        def symbols():
            if raises:
                raise RuntimeError("table unavailable")
            return rates or {}
        return types.SimpleNamespace(contract=contract,
                                     machine=types.SimpleNamespace(symbols=symbols))

    card = base.CardState(index=0, clock_mhz=2400, foreign_procs=0, date="d")
    prov = base.Provenance("t", None, "1", "d", "w", "clean", card)
    busy = base.Provenance("t", None, "1", "d", "w", "clean",
                           base.CardState(index=0, clock_mhz=2400, foreign_procs=2, date="d"))
    ok = {"HBM.X": base.Rate("HBM.X", 1.0, "GB/s", "MEASURED", prov)}
    for check in registry.GATE:
        check(plugin(rates=ok), "p")  # a clean plugin passes every check
    bad = [plugin(contract=None), plugin(contract="tempo/arch2/1"), plugin(raises=True),
           plugin(rates={"X": 1.0}),                                                 # not a Rate
           plugin(rates={"X": base.Rate("X", 1.0, "u", "MEASURED")}),                # no card
           plugin(rates={"X": base.Rate("X", 1.0, "u", "MEASURED", busy)})]          # neighbours
    for p in bad:
        with pytest.raises(base.ContractError):
            for check in registry.GATE:
                check(p, "p")
    assert registry._contract_major("tempo/arch/7") == base.CONTRACT_MAJOR


# ---- G5: self-test -----------------------------------------------------------------------------
def test_g5_selftest_green(plug):
    rep = plug.selftest()
    assert rep.green, rep.render()


# ---- resources -------------------------------------------------------------------------------
def test_resource_verdicts(plug):
    R = plug.resources
    assert R.verdict(256, 300, 200 * 1024, 256).code == "WALL_SMEM"
    assert R.verdict(128, 128, 64 * 1024, 40 * 64).code == "NO_BUDGET"  # > 32 wave slots
    # an estimate above the declared budget is a spill question, never "cannot launch": the
    # compiler holds the wave to the budget
    v = R.verdict(600, 600, 64 * 1024, 1024)
    assert v.code == "WALL_REG" and v.occ.ctas_per_sm == 1
    v = R.verdict(152, 182, 128 * 1024, 1024)
    assert v.code == "SPILL" and v.occ.ctas_per_sm == 1
    # __launch_bounds__(512) on a kernel launched with 4 waves: the budget is the bound's
    assert R.declared_budget(256) == 512 and R.declared_budget(256, 1, 512) == 256
    assert R.verdict(100, 300, 0, 256, 1, 512).code == "SPILL"
    assert R.verdict(100, 300, 0, 256).code == "FITS"
    assert R.verdict(400, 600, 64 * 1024, 256).code == "WALL_REG"
    assert R.verdict(128, 200, 64 * 1024, 512, 2).code == "SPILL"
    v = R.verdict(128, 128, 64 * 1024, 256)
    assert v.code == "FITS" and v.ok
    # 256 threads at 128 registers: 4 waves per SIMD fit by registers, LDS 64 KiB -> 2 per CU
    assert R.occupancy(128, 64 * 1024, 256).ctas_per_sm == 2
    assert R.reg_budget(4) == 512 and R.reg_budget(16) == 128


# ---- space / prune / bound -------------------------------------------------------------------
def test_space_is_legal_and_injective(plug):
    from tempo.plugins.gfx950 import space

    hs = list(plug.skeletons.variants(_op()))
    assert len(hs) > 100
    assert len({h.key for h in hs}) == len(hs)
    for h in hs:
        p = dict(h.params)
        assert space.legal(p["kind"], p, 4096, 15360, 3840) is None
        assert space.lds_bytes(p["kind"], p) <= space.LDS_MAX


def test_decode_space_has_stream_kinds(plug):
    hs = list(plug.skeletons.variants(_op(dtype_b="int8", shapes={"M": 1, "N": 7168, "K": 5120})))
    kinds = {dict(h.params)["kind"] for h in hs}
    assert {"ring", "stream", "reg"} <= kinds and "dma" not in kinds


def test_prune_cuts_only_hard_codes(plug):
    from tempo.core.search import prune as P

    op = _op()
    hs = list(plug.skeletons.variants(op))
    cands = P.prune(plug, op, hs)
    assert len(cands) == len(hs)
    for c in cands:
        if not c.kept and c.verdict is not None and not c.verdict.ok:
            assert c.verdict.code in P.HARD_CODES
    kept = P.kept(cands)
    assert kept
    # the C1 winner's family is kept and its bound is MFMA-bound, not silent
    dma = [c for c in kept if c.hyper.key.startswith("dma_m256n256k64")]
    assert dma and all(c.bound is not None and not c.bound.silent for c in dma)
    assert all(c.bound.binding == "MFMA" for c in dma)


def test_bound_is_a_lower_bound_on_flops(plug):
    """T >= flops per CU / MFMA capacity: the C1 bound can never beat the MFMA peak."""
    from tempo.core.model.bound import bound

    op = _op()
    h = next(h for h in plug.skeletons.variants(op) if h.key.startswith("dma_m256n256k64"))
    atoms = plug.skeletons.estimate_atoms(op, h)
    regs, max_live, lds = plug.skeletons.resources_of(op, h)
    lau = plug.skeletons.launch_of(op, h)
    occ = plug.resources.occupancy(regs, lds, lau.threads)
    b = bound(atoms, plug.machine.channels(), warps_per_sm=occ.warps_per_sm)
    cap = plug.machine.rate("CAP.MFMA_F16").value
    per_cu_flops = 2 * 4096 * 15360 * 3840 / 256
    assert b.T >= per_cu_flops / cap * 0.999


# ---- emit + build (hipcc, CPU only) -----------------------------------------------------------
def test_render_and_build_one_hyperform(plug, tmp_path):
    from tempo.core.emit import render as R
    from tempo.plugins.gfx950.classifier import parse_disasm
    from tempo.plugins.gfx950.toolchain import isa_summary

    op = _op()
    h = next(h for h in plug.skeletons.variants(op)
             if h.key == "dma_m256n256k64_w4x4_s2_z2_g8_x1_f16")
    path = R.emit(plug, op, h, str(tmp_path))
    assert os.path.exists(path)
    obj = tmp_path / "k.o"
    b = plug.toolchain.compile(path, obj, mode="device")
    assert b.ok, b.log[-2000:]
    assert b.spill_st == 0 and b.stack_frame == 0
    assert b.smem_static == 2 * (256 + 256) * 64 * 2
    isa = isa_summary(sum(parse_disasm(plug.toolchain.disasm(obj)).values(), []))
    assert isa["mfma"] >= 32 and isa["lds_dma"] > 0 and isa["scratch"] == 0
    assert isa["ds_read_b128"] > 0
    assert plug.skeletons.entry_probe(h).startswith("tempo::gen::k_gemm_dma<256, 256, 64")


# ---- recognize ---------------------------------------------------------------------------------
def test_recognize_naive_input():
    from tempo.core.op import recognize

    op = recognize.from_file(NAIVE, C1)
    assert (op.kind, op.dtype_a, op.dtype_b, op.dtype_c, op.dtype_acc) == \
        ("gemm", "fp16", "fp16", "fp16", "fp32")
    assert (op.layout_a, op.layout_b, op.layout_c) == ("k", "k", "n")
    assert op.tol_rel_l2 == pytest.approx(3e-3)


def test_recognize_refuses_mismatched_signature(tmp_path):
    from tempo.core.op import recognize

    text = open(NAIVE, encoding="utf-8").read().replace("naive_gemm_fp16(", "other_name(", 1)
    p = tmp_path / "bad.hip"
    p.write_text(text)
    with pytest.raises(recognize.NotRecognised):
        recognize.from_file(str(p), C1)


def test_recognize_refusals():
    """The refusals of the reference's recogniser (tempo/core/op/recognize.py:41-141)."""
    from tempo.core.op import recognize as R

    good = open(NAIVE, encoding="utf-8").read()
    with pytest.raises(R.NotRecognised):            # no block at all
        R.from_text("__global__ void k(int* x) {}", C1)
    with pytest.raises(R.NotRecognised):            # block names no entry
        R.from_text(good.replace("entry: naive_gemm_fp16", "entry_x: y"), C1)
    with pytest.raises(R.NotRecognised):            # '*' shape not supplied
        R.from_text(good, {"M": 4, "N": 8})
    # the block's own mention of the entry never counts as its declaration
    body = good.split("TEMPO-OP-END", 1)[0] + "TEMPO-OP-END\n"
    with pytest.raises(R.NotRecognised):
        R.from_text(body, C1)
    # parameter counting is bracket-aware: a template argument's comma is not a parameter
    tmpl = good.replace("int M, int N, int K)", "int M, int N, Pair<int, int> K)", 1)
    assert R.from_text(tmpl, C1).shapes == {"M": 4096, "N": 15360, "K": 3840}
    extra = good.replace("int M, int N, int K)", "int M, int N, int K, int L)", 1)
    with pytest.raises(R.NotRecognised):
        R.from_text(extra, C1)
    # given shapes override declared ones; declared numbers are used when none is given
    fixed = good.replace("shape: M=* N=* K=*", "shape: M=7 N=8 K=16")
    assert R.from_text(fixed).shapes == {"M": 7, "N": 8, "K": 16}
    assert R.from_text(fixed, {"M": 9}).shapes == {"M": 9, "N": 8, "K": 16}


# ---- core oracle gate / coverage / ratio ------------------------------------------------------
def test_oracle_gate_needs_named_independent_path():
    from tempo.core.op.oracle import OracleResult

    r = OracleResult(rel_l2=1e-4, tol=3e-3, independent_rel_l2=2e-4, independent_path="")
    assert r.necessary_ok and not r.ok
    r.independent_path = "fp64 dot products on 2048 sampled cells"
    assert r.ok
    r.independent_rel_l2 = 1e-2
    assert not r.ok


def test_coverage_from_poison():
    import numpy as np

    from tempo.core.op.coverage import from_poison

    cells = np.zeros(100, np.uint16)
    assert from_poison(cells).ok
    cells[17] = 0x7f7f
    assert not from_poison(cells).ok


def test_median_ratio():
    from tempo.core.measure.ratio import median_ratio

    r = median_ratio([(1.0, 2.0), (1.0, 2.2), (1.0, 1.8)])
    assert r == pytest.approx(2.0, rel=1e-6) or r == pytest.approx(0.5, rel=1e-6)


# ---- toolchain remark parsing -----------------------------------------------------------------
def test_parse_resource_remarks():
    from tempo.plugins.gfx950.toolchain import parse_resource_remarks

    text = """k.hip:3:1: remark: k.hip:3:0: Function Name: _Z1kPf [-Rpass-analysis=kernel-resource-usage]
k.hip:3:1: remark: k.hip:3:0:     TotalSGPRs: 18 [-Rpass-analysis=kernel-resource-usage]
k.hip:3:1: remark: k.hip:3:0:     VGPRs: 130 [-Rpass-analysis=kernel-resource-usage]
k.hip:3:1: remark: k.hip:3:0:     AGPRs: 64 [-Rpass-analysis=kernel-resource-usage]
k.hip:3:1: remark: k.hip:3:0:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
k.hip:3:1: remark: k.hip:3:0:     LDS Size [bytes/block]: 65536 [-Rpass-analysis=kernel-resource-usage]
"""
    r = parse_resource_remarks(text)
    assert r["_Z1kPf"]["VGPRs"] == 130 and r["_Z1kPf"]["AGPRs"] == 64
    assert r["_Z1kPf"]["LDS Size [bytes/block]"] == 65536


def test_tensor_result_maps_are_bijections(plug):
    from tempo.plugins.gfx950.tensor import result_map

    for ms in (32, 16):
        rows, cols = result_map(ms)
        assert len({(a, b) for a, b in zip(rows.ravel(), cols.ravel())}) == ms * ms


# ---- meters: the counter step's parsing and attribution (no GPU) ------------------------------
def _csv(path, dispatches):
    import csv

    cols = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id",
            "Grid_Size", "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size",
            "Scratch_Size", "VGPR_Count", "Accum_VGPR_Count", "SGPR_Count", "Counter_Name",
            "Counter_Value", "Start_Timestamp", "End_Timestamp"]
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, cols)
        w.writeheader()
        for did, (name, cnt, t0, t1) in enumerate(dispatches, 1):
            for c, v in cnt.items():
                w.writerow({"Dispatch_Id": did, "Kernel_Name": name, "Grid_Size": 256,
                            "Counter_Name": c, "Counter_Value": v, "Start_Timestamp": t0,
                            "End_Timestamp": t1})


def test_counter_step_attribution_and_figures(tmp_path):
    from tempo.plugins.gfx950 import counters as C

    copy = "__amd_rocclr_copyBuffer"
    ours = "void tempo::gen::k_gemm_ilv<256, 256>(...)"
    gib = 1 << 30
    rows = [("at::native::fill", {"FETCH_SIZE": 5.0}, 0, 10)]
    rows += [(copy, {"FETCH_SIZE": gib / 2048.0, "WRITE_SIZE": gib / 1024.0}, 0, 10)] * 3
    rows += [("at::native::normal", {"FETCH_SIZE": 1.0}, 0, 10)]
    for k in range(3):  # shape 1: three launches, the middle one the median
        rows.append((ours, {"FETCH_SIZE": 1000.0 + k, "WRITE_SIZE": 500.0,
                            "GRBM_GUI_ACTIVE": 8 * 400000.0,
                            "SQ_VALU_MFMA_BUSY_CYCLES": 0.5 * 400000 * 1024}, 0, 200000))
    rows.append(("at::native::normal", {"FETCH_SIZE": 1.0}, 0, 10))
    rows += [(ours, {"FETCH_SIZE": 10.0, "WRITE_SIZE": 1.0}, 0, 10)] * 3
    path = tmp_path / "c.csv"
    _csv(path, rows)
    disp = C.parse_dispatches(str(path))
    assert len(disp) == len(rows) and [d["id"] for d in disp] == sorted(d["id"] for d in disp)
    segs = [dict(label="calibration", count=3, copy_bytes=gib), dict(label="a", count=3),
            dict(label="b", count=3)]
    got = C.assign_segments(disp, segs, "tempo")
    assert [len(got[k]) for k in ("calibration", "a", "b")] == [3, 3, 3]
    sc = C.copy_scales(got["calibration"], gib)
    assert abs(sc["FETCH_SIZE"] - 2.0) < 1e-12 and abs(sc["WRITE_SIZE"] - 1.0) < 1e-12
    fig = C.derive(C.medians(got["a"]), sc, algorithmic_bytes=1001 * 2048 + 500 * 1024)
    assert fig["fetch_bytes"] == 1001 * 1024 * 2.0 and fig["write_bytes"] == 500 * 1024
    assert abs(fig["traffic_over_algorithmic"] - 1.0) < 1e-12
    assert abs(fig["mfma_util"] - 0.5) < 1e-12
    assert abs(fig["sclk_ghz"] - 2.0) < 1e-12   # 400k cycles per XCD in 200 us
    # busy half the cycles at 2.0 GHz = 2.0 / 2.4 x 0.5 of the spec-clock matrix throughput
    assert abs(fig["mfma_util_spec_clock"] - 0.5 * 2.0 / 2.4) < 1e-12
    # a short dispatch: the profiler's fixed stretch in GRBM_GUI_ACTIVE would dominate its clock
    short = C.derive({"GRBM_GUI_ACTIVE": 8 * 30000.0, "SQ_VALU_MFMA_BUSY_CYCLES": 1024 * 1000.0,
                      "_duration_ns": 5000.0}, sc)
    assert "sclk_ghz" not in short and "mfma_util" not in short
    assert abs(short["mfma_util_spec_clock"] - 1000.0 / (5000 * 2.4)) < 1e-12
    # a split-K launch is two dispatches (main kernel, reduction): summed per launch
    two = [dict(id=i, kernel=ours, grid=1, start=0, end=100 * (i + 1),
                counters={"FETCH_SIZE": float(10 * (i % 2) + 1)}) for i in range(6)]
    m2 = C.medians(two, per_launch=2)
    assert m2["FETCH_SIZE"] == 12.0 and m2["_duration_ns"] == 700
    # a launch whose kernels differ from the first launch's means the grouping slipped
    two[3] = dict(two[3], kernel="tempo::gen::k_splitk_reduce<8>")
    with pytest.raises(RuntimeError):
        C.medians(two, per_launch=2)
    # a pass that ran fewer launches than it declared is an error, not a silent shift
    import pytest as _pt

    with _pt.raises(RuntimeError):
        C.assign_segments(disp, segs + [dict(label="c", count=1)], "tempo")
