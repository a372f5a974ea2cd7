"""CPU checks of the shipped deliveries and the C-ABI library (no GPU calls).

"One source, two consumers" (reference kernels/shipped/gemm_fp16/sm_70/test_gate.py:102-146):
select.py is the ladder, dispatch.inc is generated from it, and the compiled dispatcher must
pick the same row as select.py for every shape.  The library must export every symbol that
include/tempo_gfx950.h declares.
"""
import importlib.util
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SHIPPED = os.path.join(ROOT, "kernels", "shipped")
HEADER = os.path.join(ROOT, "include", "tempo_gfx950.h")
OPS = ("gemm_fp16", "gemm_w8a16")


def _select(op):
    path = os.path.join(SHIPPED, op, "gfx950", "select.py")
    spec = importlib.util.spec_from_file_location("select_%s" % op, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.mark.parametrize("op", OPS)
@pytest.mark.parametrize("table", ["dispatch.inc", "dispatch_gate_up.inc"])
def test_dispatch_inc_is_generated_from_select(op, table):
    d = os.path.join(SHIPPED, op, "gfx950")
    args = ["--gate-up"] if table == "dispatch_gate_up.inc" else []
    text = subprocess.run([sys.executable, os.path.join(d, "gen_dispatch.py")] + args,
                          check=True, capture_output=True, text=True).stdout
    with open(os.path.join(d, table), encoding="utf-8") as f:
        assert f.read() == text, "%s is stale: re-run the build" % table


@pytest.mark.parametrize("op,kind", [("gemm_fp16", "ilv"), ("gemm_w8a16", "ilv8")])
def test_prefill_inc_is_generated_from_select(op, kind):
    d = os.path.join(SHIPPED, op, "gfx950")
    text = subprocess.run([sys.executable, os.path.join(d, "gen_dispatch.py"), "--prefill"],
                          check=True, capture_output=True, text=True).stdout
    with open(os.path.join(d, "prefill.inc"), encoding="utf-8") as f:
        assert f.read() == text, "prefill.inc is stale: re-run the build"
    # every interleaved row of the ladder is instantiated there, once per distinct launcher, and
    # nothing else
    import importlib.util as iu

    spec = iu.spec_from_file_location("gd_" + op, os.path.join(d, "gen_dispatch.py"))
    gd = iu.module_from_spec(spec)
    spec.loader.exec_module(gd)
    insts = {gd.instantiation(r[3], r[4]) for r in _select(op).LADDER if r[3] == kind}
    plain = [ln for ln in text.splitlines()
             if ln.startswith("template hipError_t launch_%s" % kind) and "_gu" not in ln]
    assert insts and len(plain) == len(insts)
    assert all(i in text for i in insts)


@pytest.mark.parametrize("op", ["gemm_fp16", "gemm_w8a16"])
def test_prefill_unit_declares_its_scheduler(op):
    from cuda_tempiler_amd import build

    flags = build.unit_flags(os.path.join(SHIPPED, op, "gfx950", "launch_prefill.hip"))
    assert flags == ["-mllvm", "-amdgpu-sched-strategy=iterative-minreg"]
    assert build.unit_flags(os.path.join(SHIPPED, op, "gfx950", "launch.hip")) == []


def test_frozen_kernels_match_skeletons():
    from tempo.plugins.gfx950 import ship

    assert ship.stale() == []


def test_delivery_layout():
    for op in OPS:
        d = os.path.join(SHIPPED, op, "gfx950")
        for f in ("kernel.hip", "launch.h", "launch.hip", "dispatch.inc", "dispatch_gate_up.inc",
                  "select.py", "gen_dispatch.py", "manifest.json"):
            assert os.path.exists(os.path.join(d, f)), "%s/%s missing" % (op, f)
    for op in OPS:
        for f in ("launch_prefill.hip", "prefill.inc"):
            assert os.path.exists(os.path.join(SHIPPED, op, "gfx950", f)), (op, f)


def _declared():
    with open(HEADER, encoding="utf-8") as f:
        text = f.read()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(tempo_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    from cuda_tempiler_amd import capi

    declared = _declared()
    assert len(declared) >= 10
    L = capi.lib()
    missing = [s for s in declared if not hasattr(L, s)]
    assert not missing
    assert set(declared) == set(capi.EXPORTS), "ctypes table and header disagree"


def test_abi_version():
    from cuda_tempiler_amd import capi

    assert capi.lib().tempo_abi_version() >= 1


SWEEP_M = (1, 2, 8, 16, 17, 31, 32, 33, 64, 128, 255, 256, 257, 1000, 2048, 4096)
SWEEP_NK = ((15360, 3840), (3840, 15360), (7168, 5120), (5120, 6144), (34816, 5120),
            (5120, 17408), (1024, 5120), (5120, 5120), (512, 384), (520, 384), (384, 100),
            (4096, 192), (4096, 320),
            # the line kernel's tail grid: one slab left, none left, one per CU left, too many
            # waves per CU, fmt 2 metadata past the LDS, more rounds
            (16400, 256), (16384, 384), (36864, 128), (69632, 5120), (34816, 16384),
            (32784, 256), (49152, 5120),
            # the phase-ordered rows: 136 / 144 / 24 / 20 rows per CU, K % 1024, the gate/up width
            (36864, 2048), (6144, 1024), (5120, 3072), (34816, 3840), (17408, 5120),
            (18432, 1024), (17408, 3840))


def test_compiled_route_agrees_with_select_fp16():
    from cuda_tempiler_amd import capi

    sel = _select("gemm_fp16")
    for (N, K) in SWEEP_NK:
        for M in SWEEP_M:
            r = sel.select("gemm", M, N, K)
            assert capi.route(0, M, N, K) == (r["tag"] if r else ""), (M, N, K)


@pytest.mark.parametrize("fmt", [1, 2])
def test_compiled_route_agrees_with_select_w8a16(fmt):
    from cuda_tempiler_amd import capi

    sel = _select("gemm_w8a16")
    for (N, K) in SWEEP_NK:
        for M in SWEEP_M:
            r = sel.select("gemm_w8a16", M, N, K, fmt=fmt, group=128)
            assert capi.route(fmt, M, N, K) == (r["tag"] if r else ""), (M, N, K, fmt)


def test_compiled_route_agrees_with_select_gate_up():
    from cuda_tempiler_amd import capi

    s16, s8 = _select("gemm_fp16"), _select("gemm_w8a16")
    for (N, K) in SWEEP_NK:
        for M in SWEEP_M:
            r = s16.select_gate_up("gemm_gate_up", M, N, K)
            assert capi.route(3, M, N, K) == (r["tag"] if r else ""), (M, N, K)
            for fmt in (1, 2):
                r = s8.select_gate_up("gemm_w8a16_gate_up", M, N, K, fmt=fmt, group=128)
                assert capi.route(3 + fmt, M, N, K) == (r["tag"] if r else ""), (M, N, K, fmt)
    assert capi.route(3, 64, 17408, 5120) == "gi128x256k64s3"  # prefill: the interleaved kernel
    assert capi.route(4, 300, 17408, 5120) == "gi8x256w1x4k64s3t"
    assert capi.route(3, 64, 1000, 512) == ""  # N % 128 != 0 past the decode band: fallback


def test_route_unknown_op_is_empty():
    from cuda_tempiler_amd import capi

    assert capi.route(7, 64, 64, 64) == ""
    assert capi.route(6, 1, 64, 64) == ""


def test_rows_fall_through_when_the_first_row_does_not_fit():
    from cuda_tempiler_amd import capi

    assert capi.route(0, 8, 15360, 3840) == "l1r1n4d4"
    assert capi.route(0, 8, 12304, 3840) == "l1r1d4"      # N % 64 != 0: the unshared line row
    assert capi.route(0, 8, 15360, 65792) == "s16r1u4"    # K > 65536: past the line rows
    assert capi.route(1, 16, 34816, 5120) == "p1n9d4"    # 256 workgroups of 136 rows
    assert capi.route(1, 16, 34816, 3840) == "l1r1n4d2t"  # K % 1024 != 0
    assert capi.route(1, 16, 34816, 12288) == "l1r1n4d2t"  # long K: past the phase rows
    assert capi.route(2, 32, 34816, 5120) == "p2n9d4"
    assert capi.route(2, 1, 34816, 5120) == "p0n9d3"
    assert capi.route(2, 1, 5120, 17408) == "p0n2d3"      # uint8, long K: the whole-K phase row
    assert capi.route(2, 1, 5120, 24576) == "l0r1d2k8"    # past the row's K band
    assert capi.route(1, 1, 34816, 5120) == "l0r1d2w"     # int8 at M = 1: the line row
    assert capi.route(1, 16, 15360, 5120) == "l1r1n4d3"  # too few slabs for the tail grid
    assert capi.route(1, 16, 69632, 5120) == "l1r1n4d3"  # 5 workgroups of 4 waves per CU
    assert capi.route(2, 16, 5120, 17408) == "p1n10d4k8"    # long K: the k-sliced phase row
    assert capi.route(2, 32, 5120, 17408) == "p2n10d4k8"
    assert capi.route(2, 16, 5120, 12416) == "l1r1n4d2k8"   # K % 1024 != 0: the k-slice row
    assert capi.route(1, 16, 5120, 17408) == "l1r1n4d2k8"   # int8: the k-sliced phase row is uint8 only
    assert capi.route(2, 16, 5120, 8192) != "p1n10d4k8"     # K < 12288: under the row's band
    assert capi.route(2, 16, 5120, 6144) == "l1r1n2d2"
    assert capi.route(2, 16, 1024, 5120) == "l1r1d2k8"     # narrow N
    assert capi.route(1, 32, 5120, 5120) == "l2r1n2d4"     # K < 6144: past the k-slice row
    assert capi.route(1, 32, 34816, 5120) == "l2r1n8d2t"
    assert capi.route(2, 32, 34816, 16384) == "l2r1n4d4"  # fmt 2 metadata: not co-resident
    assert capi.route(2, 32, 34816, 65536 + 256) == "h32r1u4n2"
    assert capi.route(0, 1, 15360, 3840) == "l0r1d2w"
    assert capi.route(0, 1, 3840, 15360) == "l0r1d2"    # long K
    assert capi.route(1, 1, 5120, 5120) == "p0n2d2"      # 20 rows per CU, K % 1024 == 0
    assert capi.route(2, 1, 5120, 5120) == "p0n2d2"
    assert capi.route(1, 1, 5120, 3840) == "l0r1n2d2"    # K % 1024 != 0
    assert capi.route(1, 1, 7168, 5120) == "l0r1d2w"     # N = 7168: past the narrow phase row
    assert capi.route(1, 1, 5120, 17408) == "l0r1d2k8"  # long K: k slices
    assert capi.route(1, 1, 7168, 5120) == "l0r1d2w"    # past the narrow row's N band
    assert capi.route(1, 1, 1024, 5120) == "l0r1d2"     # narrow N
    assert capi.route(1, 1, 5120, 65536 + 512) == "s1a_r1u8"
    assert capi.route(1, 1, 5120, 65536 + 256) == "s1a_r1u4"   # K % 512 != 0, K % 256 == 0
    assert capi.route(0, 4096, 15360, 3840) == "i256x256k64w4r8"
    assert not capi.route(0, 4096, 15360, 3872)  # K % 64 != 0: no prefill row fits, fallback


def test_gptq_repack_refuses_before_any_launch():
    """Shapes and groups the repack does not cover are refused on the host (no GPU touched)."""
    from cuda_tempiler_amd import capi

    L = capi.lib()
    p = capi._p(4096)  # never dereferenced: every case below is refused before a launch
    s = capi._p(0)
    assert L.tempo_gptq_repack_u8(p, p, p, 5120, 6144, 64, p, p, p, s) == capi.TEMPO_FALLBACK
    assert L.tempo_gptq_repack_u8(p, p, p, 5120 + 32, 6144, 128, p, p, p, s) == capi.TEMPO_FALLBACK
    assert L.tempo_gptq_repack_u8(p, p, p, 5120, 6144 + 4, 128, p, p, p, s) == capi.TEMPO_FALLBACK
    assert L.tempo_gptq_repack_u8(p, p, p, 0, 6144, 128, p, p, p, s) == capi.TEMPO_FALLBACK
    assert L.tempo_gptq_repack_u8(None, p, p, 5120, 6144, 128, p, p, p, s) != 0


# ---- delivery-only build (reference kernels/shipped/gemm_fp16/sm_70/test_gate.py:230-285) ------
@pytest.mark.parametrize("op", ["gemm_fp16", "gemm_w8a16"])
def test_delivery_builds_from_its_own_directory(op, tmp_path):
    """A host tree that vendors kernels/shipped/<op>/gfx950/ compiles it with -I pointing there and
    nowhere else, and links a launcher: the ship probe links against the delivery's objects."""
    import concurrent.futures as cf
    import subprocess

    from cuda_tempiler_amd import build as B

    d = os.path.join(ROOT, "kernels", "shipped", op, "gfx950")
    units = B.delivery_units(op)
    assert units[-1] == "ship_probe.hip" and "launch.hip" in units

    def cc(name):
        src = os.path.join(d, name)
        obj = str(tmp_path / name.replace(".hip", ".o"))
        cmd = [B.HIPCC] + B.PROBE_FLAGS + B.unit_flags(src) + ["-I", d, "-c", src, "-o", obj]
        r = subprocess.run(cmd, capture_output=True, text=True, cwd=str(tmp_path))
        assert r.returncode == 0, r.stderr[-3000:]
        return obj

    with cf.ThreadPoolExecutor(len(units)) as ex:
        objs = list(ex.map(cc, units))
    exe = str(tmp_path / "probe")
    r = subprocess.run([B.HIPCC, "--offload-arch=gfx950", "-o", exe] + objs,
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    assert os.path.getsize(exe) > 0


def test_tail_rule_of_the_two_part_row():
    """The W8A16 TAIL row splits N only where the last round of 256 x 256 tiles is at most a
    quarter full and the whole rounds are whole column blocks (select.tail_split mirrors
    launch_ilv8_tail; the GPU ladder cases at (512 | 500 | 300, 34816, 1024) run both parts)."""
    sel = _select("gemm_w8a16")
    assert sel.tail_split(2048, 34816) == 32768   # 1088 tiles: four rounds, then 64
    assert sel.tail_split(512, 34816) == 32768    # 272 tiles: one round, then 16
    assert sel.tail_split(300, 34816) == 32768
    assert sel.tail_split(2048, 5120) == 0        # 160 tiles: no whole round
    assert sel.tail_split(2048, 7168) == 0        # 224 tiles
    assert sel.tail_split(4096, 34816) == 0       # 2176 tiles: the last round half full
    assert sel.tail_split(2048, 32768) == 0       # 1024 tiles: whole rounds only


def test_fill_rule_of_the_192_row_tiles():
    """The W8A16 FILL row (192 x 256 tiles) takes a grid only where one round of its tiles holds
    it and it has more tiles than 256 x 256 tiles would (select.fill_fits mirrors
    ilv8_fill_fits of launch.h; the compiled-route sweep above checks the two agree)."""
    sel = _select("gemm_w8a16")
    assert sel.fill_fits(2048, 5120, 192, 256)       # 220 tiles against 160
    assert sel.fill_fits(1536, 7168, 192, 256)       # 224 against 168
    assert sel.fill_fits(512, 17408, 192, 256)       # 204 against 136
    assert not sel.fill_fits(2048, 7168, 192, 256)   # 308 tiles: a second round
    assert not sel.fill_fits(4096, 5120, 192, 256)   # 440 tiles
    assert not sel.fill_fits(192, 5120, 192, 256)    # one tile row either way
    assert not sel.fill_fits(384, 5120, 192, 256)    # two tile rows either way
    assert not sel.fill_fits(257, 5120, 192, 256)
    assert sel.select("gemm_w8a16", 2048, 5120, 5120, fmt=1)["tag"] == "i8x192x256w1x4k64s3f"
    assert sel.select("gemm_w8a16", 2048, 7168, 5120, fmt=2)["tag"] == "i8x256w1x4k64s3t"
