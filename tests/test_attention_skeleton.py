"""The attention operation in the pipeline (CPU): the naive input declares it, the core counts
its work, the gfx950 plugin enumerates, bounds, renders and compiles its skeleton.

The operation is the profiled forward of the reference (bottom-right causal mask
attn_fwd_cutlass.cu:137, GQA :193, LSE volta_fwd_ws.cuh:1063); its naive input is
kernels/naive/fmha_fwd.hip and the shipped kernel k_fmha_fwd (skeletons/fmha_fwd) behind
tempo_fmha_fwd_launch.  The skeleton's tile is fixed (128 query rows, 32-key blocks, 4 waves), so
its space is one hyperform per head dimension and mask; these tests hold that hyperform to what
the shipped launcher runs and to what the compiler builds.
"""
import os
import tempfile

import pytest

from tempo.core.op import recognize
from tempo.core.op.spec import describe, flops, visible_pairs
from tempo.core.search.prune import prune
from tempo.plugins.base import PluginCapabilityError
from tempo.plugins.gfx950 import load

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NAIVE = os.path.join(ROOT, "kernels", "naive", "fmha_fwd.hip")
C5 = {"B": 1, "H": 16, "HKV": 8, "SQ": 4096, "SK": 4096, "D": 256, "CAUSAL": 1}


def _op(**over):
    return recognize.from_file(NAIVE, dict(C5, **over))


def test_naive_input_declares_attention():
    op = _op()
    assert op.kind == "attention"
    assert (op.dtype_a, op.dtype_b, op.dtype_c, op.dtype_acc) == ("fp16", "fp16", "fp16", "fp32")
    assert dict(op.shapes) == C5
    assert describe(op).startswith("attention[B=1 H=16 HKV=8 SQ=4096 SK=4096 D=256 CAUSAL=1]")
    with pytest.raises(Exception):   # a dimension left '*' must be given
        recognize.from_file(NAIVE, {k: v for k, v in C5.items() if k != "SK"})
    with pytest.raises(ValueError):  # query heads must group over the key/value heads
        _op(H=12, HKV=8)


def test_visible_pairs_and_work_count():
    def brute(sq, sk, causal):
        off = sk - sq
        return sum(1 for i in range(sq) for j in range(sk) if not causal or j <= i + off)

    for sq, sk in [(1, 1), (4, 4), (3, 7), (7, 3), (5, 1), (1, 5), (33, 64), (64, 33)]:
        for c in (0, 1):
            assert visible_pairs(sq, sk, c) == brute(sq, sk, c), (sq, sk, c)
    # C5: 4 D flops per visible pair per head (the bench's FMHA TFLOP/s uses the same count)
    assert flops(_op()) == 4.0 * 16 * 256 * (4096 * 4097 // 2)
    assert flops(_op(CAUSAL=0)) == 4.0 * 16 * 256 * 4096 * 4096


def test_space_holds_the_shipped_hyperform():
    plug = load()
    for D, causal in ((256, 1), (128, 0)):
        op = _op(D=D, CAUSAL=causal)
        hs = list(plug.skeletons.variants(op))
        assert [h.key for h in hs] == ["fmha_d%d_c%d_q128_kv32_w4" % (D, causal)]
        cands = prune(plug, op, hs)
        assert cands[0].kept, cands[0].reason
        lau = plug.skeletons.launch_of(op, hs[0])
        # what cuda_tempiler_amd/csrc/fmha.hip launches: one 256-thread workgroup per
        # (128 query rows, head, batch), the four K and four V slots of 32 keys in LDS
        assert (lau.grid_ctas, lau.threads, lau.smem_bytes) == (32 * 16, 256, 8 * 32 * D * 2)
    with pytest.raises(PluginCapabilityError):
        list(plug.skeletons.variants(_op(D=64)))


def test_rendered_skeleton_compiles_within_its_estimate():
    plug = load()
    for D, causal in ((256, 1), (128, 0)):
        op = _op(D=D, CAUSAL=causal)
        h = next(iter(plug.skeletons.variants(op)))
        r = plug.skeletons.render(op, h)
        assert ("template __global__ void fmha::k_fmha_fwd<%d, %s>(" % (D, "true" if causal else "false")
                in r.source)
        d = tempfile.mkdtemp()
        src = os.path.join(d, r.filename)
        with open(src, "w") as f:
            f.write(r.source)
        b = plug.toolchain.compile(src, os.path.join(d, "k.o"), mode="device")
        assert b.ok, b.log[-2000:]
        regs, max_live, lds = plug.skeletons.resources_of(op, h)
        assert b.spill_st == 0 and b.stack_frame == 0, "the skeleton spills VGPRs"
        assert b.smem_static == lds
        # the estimate's two edges bracket the compiler's count (one wave per SIMD: <= 512)
        assert regs <= b.regs <= max_live <= 512, (regs, b.regs, max_live)
