"""The verify stage reads what ships: LDS-DMA in either encoding, and no spill in a shipped row.

Reference: the build stage records spill and stack bytes per build
(tempo/plugins/sm70/toolchain.py:102-112) and the contract's BuildResult carries a loop-spill
field (tempo/plugins/base.py:534).  Here manifest.gate_build() refuses a shipped row that spills,
uses scratch, or -- for the kinds that copy by LDS-DMA -- has no LDS-DMA instruction.  CPU only
(hipcc cross-compiles; nothing runs on a GPU).
"""
import os

import pytest

from tempo.plugins.gfx950 import load, manifest
from tempo.plugins.gfx950.classifier import parse_disasm
from tempo.plugins.gfx950.toolchain import isa_summary

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# A disassembly excerpt in llvm-objdump's layout: the MUBUF LDS copy differs from a register
# load only by its lds modifier
DISASM = """
0000000000001000 <k>:
	buffer_load_dwordx4 v1, s[8:11], s4 offen lds                // 000000001000: E05D1000 04020001
	buffer_load_dword v2, s[8:11], 0 offen lds                  // 000000001008: E0511000 80020002
	buffer_load_dwordx4 v[4:7], v3, s[8:11], 0 offen            // 000000001010: E05C1000 80020403
	global_load_lds_dwordx4 v[8:9], off                         // 000000001018: DDF48000 007F0008
	global_load_dwordx4 v[10:13], v[8:9], off                   // 000000001020: DD5C8000 0A7F0008
	v_mfma_f32_16x16x32_f16 a[0:3], v[4:7], v[10:13], a[0:3]    // 000000001028: D3D48000 04021504
	scratch_store_dword off, v4, off                            // 000000001030: DC700000 007F0400
	s_barrier                                                   // 000000001038: BF8A0000
"""


def test_isa_summary_counts_both_lds_dma_forms():
    isa = isa_summary(parse_disasm(DISASM, operands=True)["k"])
    assert isa["lds_dma"] == 3 and isa["lds_dma_buffer"] == 2
    assert isa["buffer_load"] == 1 and isa["global_load_dwordx4"] == 1
    assert isa["mfma"] == 1 and isa["scratch"] == 1 and isa["barrier"] == 1
    # mnemonics alone cannot see the buffer form's modifier: only the FLAT copy is counted
    assert isa_summary(parse_disasm(DISASM)["k"])["lds_dma"] == 1


def test_gate_build_refuses_spill_scratch_and_a_lost_dma_copy():
    good = dict(tag="r", kind="ilv", vgpr_spill=0, sgpr_spill=0, scratch_bytes_per_lane=0,
                scratch_insts=0, lds_dma=40)
    assert manifest.gate_build({"r": good}) == []
    for bad in (dict(good, vgpr_spill=2), dict(good, scratch_bytes_per_lane=12),
                dict(good, scratch_insts=4), dict(good, lds_dma=0)):
        fails = manifest.gate_build({"r": bad})
        assert len(fails) == 1 and fails[0].startswith("r: ")
    # a register-staged kind has no DMA copy to lose; a waiver names the row it covers
    assert manifest.gate_build({"m": dict(good, kind="mfma", lds_dma=0)}) == []
    assert manifest.gate_build({"r": dict(good, vgpr_spill=2)}, waivers={"r": "why"}) == []


PLANTED = r"""
#include <hip/hip_runtime.h>
// 96 values live across a loop under a 32-VGPR cap: the allocator must spill
extern "C" __global__ __attribute__((amdgpu_num_vgpr(32))) void planted(const float* x, float* y,
                                                                       int n) {
  float v[96];
#pragma unroll
  for (int i = 0; i < 96; ++i) v[i] = x[threadIdx.x + 64 * i];
  for (int k = 0; k < n; ++k)
#pragma unroll
    for (int i = 0; i < 96; ++i) v[i] = v[i] * v[(i + 1) % 96] + 1.0f;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 96; ++i) s += v[i];
  y[threadIdx.x] = s;
}
"""


def test_planted_spilling_kernel_fails_the_gate(tmp_path):
    plug = load()
    src = tmp_path / "planted.hip"
    src.write_text(PLANTED)
    got = manifest.source_numbers(plug, str(src), "line", "planted")
    assert got["vgpr_spill"] > 0 and got["scratch_insts"] > 0
    fails = manifest.gate_build({"planted": got})
    assert len(fails) == 1 and "spills" in fails[0] and "scratch" in fails[0]
    assert "without an LDS-DMA copy" in fails[0]


@pytest.mark.parametrize("op,tag,fmt", [("gemm_fp16", "i256x256k64w4r8", 0),
                                        ("gemm_w8a16", "i8x256w1x4k64s3t", 1),
                                        ("gemm_w8a16", "gi8x256w1x4k64s3t", 2)])
def test_shipped_rows_pass_the_gate(op, tag, fmt):
    """The C1 row copies by buffer LDS-DMA (counted), and the W8A16 prefill rows that used to
    spill 2 VGPRs compile clean."""
    from tempo.plugins.base import Hyperform, OpSpec

    plug = load()
    sel = manifest._select(op)
    db = {0: "fp16", 1: "int8", 2: "uint8"}[fmt]
    spec = OpSpec(kind="gemm", dtype_a="fp16", dtype_b=db, dtype_c="fp16", dtype_acc="fp32",
                  layout_a="k", layout_b="k", layout_c="n",
                  shapes={"M": 4096, "N": 15360, "K": 3840})
    row = next(r for r in manifest.ladder_rows(sel) if r[2] == tag)
    _, _, _, kind, p, epi = row
    h = Hyperform(plugin="gfx950", params=manifest.hyper_params(kind, p, fmt, epi), key=tag)
    got = manifest.row_numbers(plug, spec, h, kind, tag)
    assert got["lds_dma_buffer"] > 0 and got["buffer_load"] == 0
    assert manifest.gate_build({tag: got}) == []
