"""Every row of every shipped ladder is reachable, and some GPU parity case reaches it.

Reference pattern: the dispatch consistency gate of the sm_70 delivery
(kernels/shipped/gemm_fp16/sm_70/test_gate.py:102-146), which checks that the generated
dispatcher and select.py agree row for row.  Here two more properties are checked on the CPU:

  * reachability -- a brute-force search over shapes finds, for every row (and every weight
    format it is instantiated for), a shape that the ladder routes to it.  A row shadowed by the
    rows in front of it is dead code in the library and a row no test can run;
  * coverage -- every reachable row is named by a case of tests/ladder_cases.py, and every case
    routes to the row it names, so the GPU parity suite (tests/test_gpu_ladder_rows.py) runs
    every row the dispatcher can pick.
"""
import importlib.util
import os

import pytest

from tests import ladder_cases as LC

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _select(op):
    path = os.path.join(ROOT, "kernels", "shipped", op, "gfx950", "select.py")
    spec = importlib.util.spec_from_file_location("sel_cov_" + op, path)
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


F16 = _select("gemm_fp16")
W8S = _select("gemm_w8a16")

# name -> (ladder rows, route function (M, N, K) -> tag or None, cases)
LADDERS = {
    "fp16": (F16.LADDER, lambda M, N, K: F16.select("gemm", M, N, K), LC.FP16),
    "fp16_gate_up": (F16.LADDER_GATE_UP,
                     lambda M, N, K: F16.select_gate_up("gemm_gate_up", M, N, K), LC.FP16_GATE_UP),
}
for _f in (1, 2):
    LADDERS["w8_fmt%d" % _f] = (
        [r for r in W8S.LADDER if _f in r[4].get("fmts", W8S.FORMATS)],
        (lambda f: lambda M, N, K: W8S.select("gemm_w8a16", M, N, K, fmt=f))(_f), LC.W8[_f])
    LADDERS["w8_gate_up_fmt%d" % _f] = (
        [r for r in W8S.LADDER_GATE_UP if _f in r[4].get("fmts", W8S.FORMATS)],
        (lambda f: lambda M, N, K: W8S.select_gate_up("gemm_w8a16_gate_up", M, N, K, fmt=f))(_f),
        LC.W8_GATE_UP[_f])

# the search grid: band edges of M, every multiple of 8 below 4200 for N plus the neighbourhoods
# of the N thresholds (32768: one round of 8-slab workgroups of the line kernel's tail grid;
# 34816: whole rounds of 128 x 128 tiles and a quarter round more; 17408: the gate/up output
# width, 68 columns per CU for the phase-ordered rows; 5120: 160 rows per row group of the
# k-sliced phase rows), and K over the divisibility
# classes the rows test (K > 65536 is past the line rows; 12288: the long-K rows; 5120: a
# multiple of 1024 below 12288, the phase-ordered rows' class)
_M = (1, 2, 8, 9, 16, 17, 32, 33, 64, 65, 128, 129, 256, 257, 2048)
_N = sorted(set(range(8, 4200, 8)) | {n + d for n in (5120, 6144, 8192, 12288, 16384, 17408, 32768, 34816)
                                        for d in range(-64, 72, 8)})
_K = (64, 128, 192, 256, 384, 512, 3840, 5120, 5184, 12288, 17408) + tuple(65536 + 64 * j for j in range(1, 9))


def _tag(route, M, N, K):
    r = route(M, N, K)
    return None if r is None else r["tag"]


@pytest.mark.parametrize("name", sorted(LADDERS))
def test_every_row_is_reachable(name):
    rows, route, _ = LADDERS[name]
    want = {r[2] for r in rows}
    seen = set()
    for M in _M:
        for K in _K:
            for N in _N:
                t = _tag(route, M, N, K)
                if t is not None:
                    seen.add(t)
            if seen >= want:
                return
    assert not (want - seen), "%s: rows no shape reaches: %s" % (name, sorted(want - seen))


@pytest.mark.parametrize("name", sorted(LADDERS))
def test_cases_route_as_named(name):
    _, route, cases = LADDERS[name]
    wrong = [(c, _tag(route, *c[1:4])) for c in cases if _tag(route, *c[1:4]) != c[0]]
    assert not wrong, "%s: cases routed elsewhere: %s" % (name, wrong)


@pytest.mark.parametrize("name", sorted(LADDERS))
def test_every_row_has_a_gpu_case(name):
    rows, _, cases = LADDERS[name]
    missing = sorted({r[2] for r in rows} - {c[0] for c in cases})
    assert not missing, "%s: ladder rows no GPU parity case runs: %s" % (name, missing)


def test_strided_cases_route_as_named():
    for tag, M, N, K, pa, pb, pc in LC.FP16_STRIDED:
        assert _tag(LADDERS["fp16"][1], M, N, K) == tag
        assert pa % 8 == 0 and pb % 8 == 0 and pc % 4 == 0  # the launcher's stride rule
