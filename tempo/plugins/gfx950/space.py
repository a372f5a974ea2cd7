"""gfx950: SEARCH SPACE -- axes and legal hyperforms (reference pattern tempo/plugins/sm70/space.py).

The skeleton kinds, each a kernel family of tempo/plugins/gfx950/skeletons:
  ilv     gemm_mfma/k_gemm_ilv      fp16 x fp16, one wave per SIMD, large wave tiles, LDS-DMA
                                    copies and fragment reads interleaved with the MFMAs by hand
  ilv8    gemm_mfma/k_gemm_ilv8     int8 / uint8 weights (W8A16 prefill): k_gemm_ilv with the
                                    weight tile as bytes, dequantised after its fragment reads
  dma     gemm_mfma/k_gemm_dma      fp16 x fp16, LDS-DMA multi-stage pipeline (prefill, M > 32)
  reg     gemm_mfma/k_gemm          any weight format, register-staged copy that can dequantise
                                    on the way into LDS (W8A16 prefill, fp16 fallback)
  line    gemv_stream/k_stream_line decode (M <= 32): whole 128-byte weight lines by nontemporal
                                    LDS-DMA into per-wave rings, fragments read back swizzled;
                                    with row tiles (MT = 1) also 32 < M <= 128, 8-bit weights
  ring    gemv_stream/k_stream_dma  decode (M <= 32): per-wave LDS-DMA ring of k-steps
  fmha    fmha_fwd/k_fmha_fwd       attention forward (op kind 'attention'), one hyperform per
                                    head dimension and mask (fixed 128-row / 32-key tile)
  stream  gemv_stream/k_stream      decode, register-staged prefetch (kept as a measured arm)

Legality here means "compiles and launches": LDS within 160 KiB, tiles divide the shape, the
vmcnt-counted depth fits the 6-bit counter.  Register pressure is NOT legality -- it is the
resource verdict's business (tempo/plugins/gfx950/resources.py).
"""
from __future__ import annotations

from typing import Iterator

from ..base import Axis, Hyperform, OpSpec, PluginCapabilityError

LDS_MAX = 160 * 1024
MFMA_FLOPS = {32: 32 * 32 * 16 * 2, 16: 16 * 16 * 32 * 2}

AXES = (
    Axis("kind", frozenset({"LDS", "VMEM", "regs"})),
    Axis("block_tile", frozenset({"LDS", "VMEM", "hbm", "waves"})),
    Axis("wave_tile", frozenset({"LDS", "regs"})),
    Axis("bk", frozenset({"LDS", "barriers"})),
    Axis("stages", frozenset({"LDS", "latency"})),
    Axis("swizzle", frozenset({"LDS"})),
    Axis("group", frozenset({"l2", "hbm"})),
    Axis("xcd", frozenset({"l2"})),
    Axis("mfma_shape", frozenset({"MFMA", "regs"})),
    Axis("rows_per_wave", frozenset({"VMEM", "regs"})),
    Axis("ring_depth", frozenset({"LDS", "latency", "hbm"})),
)

DOMAINS = {
    "ilv": dict(BM=(64, 128, 256), BN=(128, 192, 256), BK=(32, 64), STAGES=(2, 3, 4),
                GROUP=(4, 8, 16), XCD=(0, 1), WAVES=((2, 2), (2, 4), (4, 2), (1, 4)),
                RSP=(0, 8, 12), SW=(0, 128, 256, 512)),
    "ilv8": dict(TILES=((256, 256, 2, 2), (256, 256, 1, 4), (192, 256, 1, 4), (128, 256, 1, 4),
                        (128, 128, 2, 2), (128, 128, 1, 4)),
                 BK=(64, 128),
                 STAGES=(2, 3, 4),
                 GROUP=(4, 8, 16), XCD=(0, 1), RSP=(4, 8, 12), SW=(0, 128, 256, 512)),
    "dma": dict(BM=(32, 64, 128, 256), BN=(64, 128, 192, 256), BK=(32, 64, 128, 256), STAGES=(2, 3, 4), SWZ=(0, 1, 2),
                GROUP=(4, 8, 16), XCD=(0, 1), WAVES=((2, 2), (2, 4), (4, 2), (4, 4)), MS=(16, 32)),
    "reg": dict(BM=(64, 128, 256), BN=(64, 128, 256), BK=(64,), MS=(16, 32), SWZ=(1, 2), GROUP=(8,),
                XCD=(1,)),
    "line": dict(R=(1, 2, 4), D=(2, 3, 4, 5, 6), W=(1024, 2048, 4096), SN=(1, 2, 4, 8), TL=(0, 1),
                 KS=(1, 4, 8, 16)),
    # row tiles (MT = 1): 16 MB rows of A per workgroup, S waves splitting K (64 < M <= 128)
    "line_mt": dict(MB=(1, 2, 4), R=(1, 2), D=(2, 3, 4), S=(2, 4, 8)),
    "ring": dict(R=(1, 2, 4), D=(4, 5, 6, 8, 10, 12, 14, 16)),
    "stream": dict(R=(1, 2, 4), U=(2, 4, 8), ALDS=(0, 1)),
    "shared": dict(R=(1, 2), U=(2, 4), SN=(2, 4, 8)),
    # phase-ordered decode kernel (8-bit weights, wide N): ring depth; NS follows from N
    "phase": dict(D=(2, 3, 4), KS=(1, 8)),
}
PHASE_WAVES = 8  # k_stream_phase: waves (k chunks) per workgroup, one workgroup per CU
PHASE_CUS = 256

BFMT_OF = {("fp16", "fp16"): 0, ("fp16", "int8"): 1, ("fp16", "uint8"): 2}
SPLIT_MINKT = 8  # split-K rows keep at least this many k-tiles per split


def split_count(tiles: int, ktiles: int, slots: int, minkt: int) -> int:
    """Splits of a split-K row, as the shipped launchers compute them (split_count in
    skeletons/common/splitk_host.h): the most splits with tiles x splits <= `slots` workgroups,
    at least `minkt` k-tiles per split, no split empty; 1 = no split."""
    if slots <= 0 or minkt <= 0 or 2 * tiles > slots:
        return 1
    sp = min(slots // tiles, ktiles // minkt)
    if sp <= 1:
        return 1
    per = -(-ktiles // sp)
    return -(-ktiles // per)


def splits_of(kind: str, p: dict, M: int, N: int, K: int) -> int:
    """Split count of an ilv / ilv8 hyperform at this shape (1 for every other kind)."""
    if kind not in ("ilv", "ilv8") or not p.get("SW", 0):
        return 1
    tiles = -(-M // p["BM"]) * (N // p["BN"])
    return split_count(tiles, K // p["BK"], p["SW"], p.get("MINKT", SPLIT_MINKT))


def bfmt(op: OpSpec) -> int:
    key = (op.dtype_a, op.dtype_b)
    if key not in BFMT_OF:
        raise PluginCapabilityError("gfx950 skeletons take A fp16 with B fp16|int8|uint8; got %s x %s"
                                    % key)
    return BFMT_OF[key]


def line_paired(p: dict) -> bool:
    """The fused gate/up line kernel with SN >= 2 pairs its slab waves (gate, up)."""
    return bool(p.get("EPI")) and p.get("SN", 1) >= 2


def line_geometry(p: dict):
    """(copies per step per wave, weight slot bytes, activation slot bytes) of the line kernel,
    as skeletons/gemv_stream declares them."""
    rr = 2 * p["R"] if p.get("EPI") and not line_paired(p) else p["R"]
    eb = 2 if p["BFMT"] == 0 else 1
    sn = p.get("SN", 1)
    la = 4 * p["MB"] if p["MB"] else sn
    return 2 * rr * eb + la // sn, rr * eb * 2048, (p["MB"] * 16 * 256 if p["MB"] else 256)


LINE_CUS = 256  # one round of the tail grid: the part's CUs
LINE_MIN_STEPS = 8  # k slices keep at least this many 128-k steps


def line_kslices(wgs: int, K: int, KS: int) -> int:
    """k slices across workgroups of a line hyperform that allows up to KS, as the shipped
    launchers choose them (line_kslices in kernels/shipped/*/gfx950/launch.h): the count whose
    wgs x ks workgroups fill whole rounds of LINE_CUS most evenly, each slice whole steps and at
    least LINE_MIN_STEPS of them; taken only when it lifts the evenness by 0.08 over no split."""
    steps = K // 128

    def even(ks):
        w = wgs * ks
        return w / (-(-w // LINE_CUS) * LINE_CUS)

    best = 1
    for ks in range(2, KS + 1):
        if steps % ks == 0 and steps // ks >= LINE_MIN_STEPS and even(ks) > even(best) + 1e-9:
            best = ks
    return best if even(best) >= even(1) + 0.08 else 1


def _line_lds(rings: int, red: int, S: int, paired: bool) -> int:
    """StreamLine::lds: with S > 1 k chunks the partial sums (red bytes) are added through LDS,
    in the rings' own bytes once every wave is past its loop, except in the paired epilogue,
    which keeps them apart."""
    if S <= 1:
        return rings
    return rings + red if paired else max(rings, red)


def line_mt_split(K: int, p: dict):
    """(S, steps per wave, LDS bytes, 1) of a row-tiled line hyperform (MT = 1), as
    kernels/shipped/gemm_w8a16/gfx950/launch.h line_mt_config chooses them: the most waves, at
    most p["S"], each taking an equal count of whole 128-k steps, whose rings (+ fmt 2 metadata of
    those steps) fit the LDS; None if none does."""
    steps = K // 128
    _, wslot, aslot = line_geometry(p)
    for S in range(min(p["S"], steps), 0, -1):
        per = -(-steps // S)
        s2 = -(-steps // per)
        meta = -(-(p["R"] * 16 * per * 3) // 16) * 16 if p["BFMT"] == 2 else 0
        wave = -(-(p["D"] * (wslot + aslot) + meta) // 1024) * 1024
        lds = _line_lds(s2 * wave, s2 * p["R"] * p["MB"] * 1024, s2, False)
        if lds <= LDS_MAX:
            return s2, per, lds, 1
    return None


def line_tail_grid(N: int, K: int, p: dict):
    """(workgroups of SN slabs, grid) of the line kernel's tail grid (TL = 1), or None: q >= 1
    whole rounds of LINE_CUS workgroups, then one single-wave workgroup per remaining slab (at
    most one per CU), a CU's q workgroups and one tail resident together.  As
    kernels/shipped/gemm_w8a16/gfx950/launch.h line_tail_grid."""
    slabs, sn = N // (16 * p["R"]), p.get("SN", 1)
    q = slabs // (LINE_CUS * sn)
    tail = slabs - q * LINE_CUS * sn
    split = line_split(N, K, p)
    if q < 1 or tail > LINE_CUS or split is None:
        return None
    if (q + 1) * split[2] > LDS_MAX or (q + 1) * sn > 16:
        return None
    return q * LINE_CUS, q * LINE_CUS + tail


def line_split(N: int, K: int, p: dict):
    """(S, steps per wave, LDS bytes, k slices across workgroups) as the shipped launchers
    compute them; None if none fits."""
    rr = 2 * p["R"] if p.get("EPI") and not line_paired(p) else p["R"]
    sn = p.get("SN", 1)
    if p.get("MT"):  # row tiles: the most waves, at most S, whose rings fit (line_mt_config)
        return line_mt_split(K, p)
    if p.get("TL"):  # one k chunk; LDS of the shared-ring body or the tail body, the larger
        steps = K // 128
        _, wslot, aslot = line_geometry(p)
        meta = -(-(rr * 16 * steps * 3) // 16) * 16 if p["BFMT"] == 2 else 0
        wave_big = -(-(p["D"] * wslot + meta) // 1024) * 1024
        act = -(-((p["D"] + 1) * aslot) // 1024) * 1024
        wave_one = -(-(p["D"] * (wslot + aslot) + meta) // 1024) * 1024
        lds = max(sn * wave_big + act, wave_one)
        return (1, steps, lds, 1) if lds <= LDS_MAX else None
    wgs = N // (16 * p["R"] * (sn // 2 if line_paired(p) else sn))
    ks = line_kslices(wgs, K, p["KS"]) if p.get("KS", 1) > 1 else 1
    steps = K // 128 // ks
    _, wslot, aslot = line_geometry(p)
    tpb = p.get("TPB", 1024)  # the kernel's launch bound
    S = max(1, min(tpb // 64 // sn, steps, -(-p["W"] // max(1, wgs * ks * sn))))

    def lds(s_, per):
        meta = -(-(rr * 16 * per * 3) // 16) * 16 if p["BFMT"] == 2 else 0
        wave = -(-(p["D"] * (wslot + (aslot if sn == 1 else 0)) + meta) // 1024) * 1024
        act = -(-((p["D"] + 1) * aslot) // 1024) * 1024 if sn > 1 else 0  # D+1 shared slots
        return _line_lds(s_ * (sn * wave + act), s_ * sn * rr * max(1, p["MB"]) * 1024, s_,
                         line_paired(p))

    while True:
        per = -(-steps // S)
        s2 = -(-steps // per)
        if lds(s2, per) <= LDS_MAX and (sn == 1 or steps % s2 == 0):
            return s2, per, lds(s2, per), ks
        if S == 1:
            return None
        S -= 1


def phase_lds(K: int, p: dict) -> int:
    """LDS of k_stream_phase (StreamPhase::lds of the skeleton): D-slot weight rings of the 8
    waves, the activation staging (after the loop: the chunk partial sums), the output image of
    NS slabs, the metadata of 16 NS rows (fmt 1: row scales; fmt 2: zero-points and scales of
    every group)."""
    mb, ns, d, ks = p["MB"], p["NS"], p["D"], p.get("KS", 1)
    mbe = max(1, mb)
    G, S = K // 128, K // (128 * ks)
    stg = 4 * mb * 1024 if mb else -(-S // PHASE_WAVES) * 256  # M = 1: every phase's slice
    kib = lambda b: -(-b // 1024) * 1024  # noqa: E731
    meta = ((kib(ns * 16 * 4 * S) * 2 if ks > 1 else kib(ns * 16 * G) + kib(ns * 32 * G))
            if p["BFMT"] == 2 else kib(ns * 32))
    return (PHASE_WAVES * d * 2048 + max(PHASE_WAVES * stg, 2 * PHASE_WAVES * mbe * 1024)
            + (0 if ks > 1 else kib(mbe * 16 * ns * 16 * 2)) + meta)


def phase_ns(N: int, ks: int = 1):
    """Slabs per workgroup of k_stream_phase for width N and ks k slices (None: N does not split
    into 256 / ks row groups of a multiple of 4 rows)."""
    groups = PHASE_CUS // ks
    if N % groups or (N // groups) % 4:
        return None
    return -(-(N // groups) // 16)


def lds_bytes(kind: str, p: dict) -> int:
    if kind in ("dma", "ilv"):
        return p["STAGES"] * (p["BM"] + p["BN"]) * p["BK"] * 2
    if kind == "ilv8":  # fp16 A tile, byte weight tile, fmt 2 metadata per stage; fmt 1 scales
        mrows = max(p["BN"], 64 * p["WM"] * p["WN"])  # metadata slots: 64 rows per wave
        meta = mrows * 8 if p["BFMT"] == 2 else 0
        return (p["STAGES"] * (p["BM"] * p["BK"] * 2 + p["BN"] * p["BK"] + meta)
                + (mrows * 4 if p["BFMT"] == 1 else 0))
    if kind == "reg":
        return 2 * (p["BM"] + p["BN"]) * p["BK"] * 2
    if kind == "ring":
        wb = 2 if p["BFMT"] == 0 else 1
        per_wave = p["D"] * (p["R"] * wb + 2 * p["MB"]) * 1024 + (p["R"] * 16 * 64 * 3 if p["BFMT"] == 2 else 0)
        return p.get("S", 1) * per_wave + (p.get("S", 1) * p["R"] * p["MB"] * 1024 if p.get("S", 1) > 1 else 0)
    if kind == "stream":
        return p.get("S", 1) * p["R"] * p["MB"] * 1024 if p.get("S", 1) > 1 else 0
    if kind == "shared":
        sk = p.get("S", 1)
        return sk * 2 * 16 * p["MB"] * 128 * p["U"] + (p["SN"] * sk * p["R"] * p["MB"] * 1024
                                                       if sk > 1 else 0)
    raise KeyError(kind)


def stream_split(N: int, K: int, R: int, step_k: int, bfmt_: int = 0, per_wave_lds: int = 0):
    """Waves per workgroup S and k chunk, as the shipped launchers compute them."""
    slabs = N // (16 * R)
    steps = K // step_k
    S = min(8, max(1, -(-2048 // max(1, slabs))), steps)
    while bfmt_ == 2 and -(-K // S) > 8192 and S < 8:
        S += 1

    def fix(s_):
        per = -(-steps // s_)
        return -(-steps // per), per * step_k

    S, chunk = fix(S)
    while per_wave_lds and S > 1 and S * per_wave_lds > LDS_MAX:
        S, chunk = fix(S - 1)
    return S, chunk


def shared_split(N: int, K: int, MB: int, R: int, U: int, SN: int, TPB: int = 1024):
    """(SK, chunk, lds bytes) of the shared-activation kernel, as the shipped launchers compute."""
    stages = K // (64 * U)
    wgs = max(1, N // (16 * R * SN))
    SK = min(TPB // 64 // SN, max(1, -(-2048 // (wgs * SN))))
    stage = 16 * MB * 128 * U

    def lds(sk):
        return sk * 2 * stage + (SN * sk * R * MB * 1024 if sk > 1 else 0)

    while SK > 1 and (stages % SK or lds(SK) > LDS_MAX):
        SK -= 1
    return SK, stages // SK * 64 * U, lds(SK)


def tag(kind: str, p: dict) -> str:
    sw = "_sw%d" % p["SW"] if p.get("SW", 0) else ""
    if kind == "ilv":
        return "ilv_m%dn%dk%d_w%dx%d_s%d_g%d_x%d_r%d%s" % (
            p["BM"], p["BN"], p["BK"], p["WM"], p["WN"], p["STAGES"], p["GROUP"], p["XCD"], p["RSP"],
            sw)
    if kind == "ilv8":
        return "ilv8_m%dn%dk%d_w%dx%d_s%d_g%d_x%d_r%d_b%d%s%s" % (
            p["BM"], p["BN"], p["BK"], p["WM"], p["WN"], p["STAGES"], p["GROUP"], p["XCD"], p["RSP"],
            p["BFMT"], sw, {0: "", 1: "_t", 2: "_t2"}[p.get("TAIL", 0)])
    if kind == "dma":
        return "dma_m%dn%dk%d_w%dx%d_s%d_z%d_g%d_x%d_f%d" % (
            p["BM"], p["BN"], p["BK"], p["WM"], p["WN"], p["STAGES"], p["SWZ"], p["GROUP"], p["XCD"],
            p.get("MS", 32))
    if kind == "reg":
        return "reg_m%dn%dk%d_w%dx%d_f%d_z%d_b%d" % (p["BM"], p["BN"], p["BK"], p["WM"], p["WN"],
                                                   p["MS"], p["SWZ"], p["BFMT"])
    if kind == "fmha":
        return "fmha_d%d_c%d_q%d_kv%d_w%d" % (p["D"], p["CAUSAL"], p["BQ"], p["BKV"], p["WAVES"])
    if kind == "line" and p.get("MT"):
        return "line_mb%d_r%d_d%d_mt%d_b%d" % (p["MB"], p["R"], p["D"], p["S"], p["BFMT"])
    if kind == "line":
        return "line_mb%d_r%d_n%d_d%d_w%d_b%d%s%s%s" % (
            p["MB"], p["R"], p.get("SN", 1), p["D"], p["W"], p["BFMT"],
            "_e1" if p.get("EPI") else "", "_tl" if p.get("TL") else "",
            "_ks%d" % p["KS"] if p.get("KS", 1) > 1 else "")
    if kind == "ring":
        return "ring_mb%d_r%d_d%d_b%d" % (p["MB"], p["R"], p["D"], p["BFMT"])
    if kind == "phase":
        return "phase_mb%d_n%d_d%d_b%d%s%s" % (p["MB"], p["NS"], p["D"], p["BFMT"],
                                              "_e1" if p.get("EPI") else "",
                                              "_ks%d" % p["KS"] if p.get("KS", 1) > 1 else "")
    if kind == "shared":
        return "shared_mb%d_r%d_u%d_b%d_n%d" % (p["MB"], p["R"], p["U"], p["BFMT"], p["SN"])
    return "stream_mb%d_r%d_u%d_b%d_a%d" % (p["MB"], p["R"], p["U"], p["BFMT"], p.get("ALDS", 0))


def legal(kind: str, p: dict, M: int, N: int, K: int):
    """None when the hyperform compiles and launches for this shape, else the reason."""
    if kind == "ilv":
        BM, BN, BK, WM, WN = p["BM"], p["BN"], p["BK"], p["WM"], p["WN"]
        if N % BN or K % max(64, BK):
            return "tile %dx%d / even substep count does not divide N=%d / K=%d" % (BN, BK, N, K)
        if BK not in (32, 64):
            return "substeps per k-tile must be 1 or 2"
        if (BM // WM) % 16 or (BN // WN) % 16:
            return "wave tile not a multiple of 16"
        rpb, nw = 1024 // (BK * 2), WM * WN
        if BM % (rpb * nw) or BN % (rpb * nw):
            return "copy blocks do not divide among waves"
        r256 = 1 if BK * 2 >= 256 else 256 // (BK * 2)
        if (16 // r256) % (BK // 8) or (nw * rpb // r256) % (BK // 8):
            return "blocks do not share the swizzle key"
        L = (BM + BN) // (rpb * nw)
        if (p["STAGES"] - 1) * L >= 64:
            return "vmcnt depth"
        if nw * 64 > 1024:
            return "more than 1024 lanes"
        if lds_bytes(kind, p) > LDS_MAX:
            return "LDS %d B > 160 KiB" % lds_bytes(kind, p)
        return None
    if kind == "ilv8":
        BM, BN, BK, WM, WN = p["BM"], p["BN"], p["BK"], p["WM"], p["WN"]
        if (BM, BN, BK, WM, WN) not in ((256, 256, 64, 2, 2), (256, 256, 64, 1, 4), (192, 256, 64, 1, 4),
                                        (128, 256, 64, 1, 4), (128, 128, 64, 2, 2),
                                        (128, 256, 128, 1, 4), (128, 128, 128, 2, 2),
                                        (128, 128, 128, 1, 4)):
            return ("the int8 interleaved kernel takes 256 x 256 (2 x 2 waves), 192 x 256 and "
                    "128 x 256 (1 x 4 waves) or 128 x 128 (2 x 2 waves) tiles of 64 k, and the "
                    "last two also of 128 k")
        if p["BFMT"] not in (1, 2):
            return "weights must be int8 (fmt 1) or uint8 group-128 (fmt 2)"
        if N % BN or K % 128:
            return "N %% %d / K %% 128 (one scale group = two k-tiles)" % BN
        L = BM // (512 // BK) // 4 + BN // (1024 // BK) // 4 + (2 if p["BFMT"] == 2 else 0)
        if (p["STAGES"] - 1) * L >= 64:
            return "vmcnt depth"
        if BM * BN * 2 > p["STAGES"] * (BM * BK * 2 + BN * BK):
            return "the C tile does not fit the stages"
        if lds_bytes(kind, p) > LDS_MAX:
            return "LDS %d B > 160 KiB" % lds_bytes(kind, p)
        return None
    if kind == "phase":
        mb, ns, d = p["MB"], p["NS"], p["D"]
        if p["BFMT"] not in (1, 2):
            return "weights must be int8 (fmt 1) or uint8 group-128 (fmt 2)"
        if M > 16 * max(1, mb) or (mb == 0 and M != 1):
            return "M > 16*MB (MB = 0: M = 1)"
        ks = p.get("KS", 1)
        if ks > 1 and (p.get("EPI") or not p.get("KSL")):
            return "k slices: the KSL instantiation, plain epilogue"
        if phase_ns(N, ks) != ns:
            return "N is not 256 / %d row groups of a multiple of 4 rows in %d slabs" % (ks, ns)
        if K % (128 * ks) or K // (128 * ks) < PHASE_WAVES or (ks == 1 and K % (PHASE_WAVES * 128)):
            return "K: whole 128-k steps per slice, at least one per wave"
        if (mb > 0 and ns < d) or d < 2 or (d - 1) * 2 + (4 * mb if mb else 1) >= 64:
            return "ring depth: 2 <= D (<= NS where activations ride the ring), vmcnt range"
        if phase_lds(K, p) > LDS_MAX:
            return "LDS %d B > 160 KiB" % phase_lds(K, p)
        return None
    if kind in ("dma", "reg"):
        BM, BN, BK = p["BM"], p["BN"], p["BK"]
        if N % BN or K % BK:
            return "tile %dx%d does not divide N=%d / K=%d" % (BN, BK, N, K)
        WM, WN = p["WM"], p["WN"]
        ms = p.get("MS", 32)
        if (BM // WM) % ms or (BN // WN) % ms:
            return "wave tile not a multiple of the MFMA shape"
        if kind == "dma":
            rpb = 1024 // (BK * 2)
            nw = WM * WN
            if BM % (rpb * nw) or BN % (rpb * nw):
                return "DMA blocks do not divide among waves"
            L = (BM + BN) // (rpb * nw)
            if (p["STAGES"] - 2 + p.get("XT", 0)) * L >= 64:
                return "vmcnt depth"
            if nw * 64 > 1024:
                return "more than 1024 lanes"
        if lds_bytes(kind, p) > LDS_MAX:
            return "LDS %d B > 160 KiB" % lds_bytes(kind, p)
        return None
    R = p["R"]
    if N % (16 * R):
        return "N %% %d" % (16 * R)
    if kind == "line" and p.get("MT"):
        if p["MB"] < 1 or p.get("SN", 1) != 1 or p.get("EPI") or p.get("TL") or p.get("KS", 1) > 1:
            return "row tiles: MB >= 1, one slab wave, plain epilogue, whole k"
        if K % 128 or K > 65536:
            return "K % 128 / K > 65536"
        L, _, _ = line_geometry(p)
        if (p["D"] - 1) * L >= 64:
            return "vmcnt depth"
        if p.get("TPB") != 64 * p["S"]:
            return "row tiles: the launch bound is 64 S threads"
        if line_mt_split(K, p) is None:
            return "LDS"
        return None
    if kind == "line":
        sn = p.get("SN", 1)
        if M > max(1, 16 * p["MB"]):
            return "M > 16*MB (MB = 0: M = 1)"
        sno = sn // 2 if line_paired(p) else sn
        if N % (16 * R * sno):
            return "N %% %d" % (16 * R * sno)
        if K % 128 or K > 65536:
            return "K % 128 / K > 65536"
        if (4 * p["MB"] if p["MB"] else sn) % sn or (not p["MB"] and sn not in (1, 2, 4)):
            return "activation copies do not split over the slab waves"
        L, _, _ = line_geometry(p)
        if (p["D"] - 1) * L >= 64 or p["D"] < 2:
            return "vmcnt depth"
        if p.get("KS", 1) > 1 and (p.get("TL") or p.get("EPI")):
            return "k slices: plain epilogue, no tail grid"
        if p.get("TL"):
            if sn == 1 or p.get("EPI"):
                return "tail grid: SN > 1, plain epilogue"
            if line_tail_grid(N, K, p) is None:
                return "tail grid: no whole round, > 1 tail slab per CU, or not co-resident"
            return None
        if line_split(N, K, p) is None:
            return "LDS"
        return None
    if M > 16 * p["MB"]:
        return "M > 16*MB"
    if kind == "shared":
        if N % (16 * R * p["SN"]) or K % (64 * p["U"]) or p["U"] < 2:
            return "shape does not divide into slab groups / stages"
        if (2 * p["MB"] * p["U"]) % p["SN"]:
            return "activation copy blocks do not split over the slab waves"
        return None
    if kind == "ring":
        wb = 2 if p["BFMT"] == 0 else 1
        if K % 64:
            return "K % 64"
        if (p["D"] - 1) * (R * wb + 2 * p["MB"]) >= 64:
            return "vmcnt depth"
        if p["D"] < 3:
            return "ring depth < 3"
        if lds_bytes(kind, dict(p, S=1)) > LDS_MAX:
            return "LDS"
        return None
    if K % (64 * p["U"]):
        return "K %% %d" % (64 * p["U"])
    if p.get("ALDS", 0) and M * (2 * K + 16) > 96 * 1024:
        return "activations do not fit the LDS budget"
    return None


def _with_split(p: dict, sw: int) -> dict:
    """An ilv / ilv8 hyperform with split-K towards `sw` workgroups: the kernel's SPLIT template
    parameter plus the launch-time rule (SW, MINKT); sw = 0 leaves the hyperform unsplit."""
    if sw:
        p.update(SW=sw, MINKT=SPLIT_MINKT, SPLIT=1)
    return p


# The attention skeleton (fmha_fwd/k_fmha_fwd): its tile is fixed by its design -- 4 waves of 32
# query rows (128 per workgroup), 32-key blocks, four LDS slots per operand -- so one hyperform
# per (head dimension, mask) is what the space holds; D 128 or 256 (the skeleton's two forms).
FMHA_TILE = dict(BQ=128, BKV=32, WAVES=4)
FMHA_D = (128, 256)


def attention_variants(op: OpSpec) -> Iterator[Hyperform]:
    D, causal = int(op.shapes["D"]), int(op.shapes["CAUSAL"])
    if D not in FMHA_D:
        raise PluginCapabilityError("gfx950 attention skeleton takes head dimension %s; declared "
                                    "D = %d" % (" or ".join(map(str, FMHA_D)), D))
    p = dict(kind="fmha", D=D, CAUSAL=causal, **FMHA_TILE)
    yield Hyperform(plugin="gfx950", params=p, key=tag("fmha", p))


def fmha_lds(D: int) -> int:
    """LDS of one workgroup of the attention skeleton: four K and four V slots of 32 keys x D."""
    return 8 * FMHA_TILE["BKV"] * D * 2


def variants(op: OpSpec) -> Iterator[Hyperform]:
    if op.kind == "attention":
        return attention_variants(op)
    if op.kind != "gemm":
        raise PluginCapabilityError("gfx950 skeletons take 'gemm' and 'attention'; declared %r"
                                    % op.kind)
    return _gemm_variants(op)


def _gemm_variants(op: OpSpec) -> Iterator[Hyperform]:
    M, N, K = int(op.shapes["M"]), int(op.shapes["N"]), int(op.shapes["K"])
    b = bfmt(op)
    out = []
    if M <= 128:
        MB = 1 if M <= 16 else 2 if M <= 32 else 4 if M <= 64 else 8
        d = DOMAINS["line"]
        for R in d["R"]:
            for D in d["D"]:
                for W in d["W"]:
                    for SN, TL, KS in ((sn, tl, ks) for sn in d["SN"] for tl in d["TL"]
                                       for ks in d["KS"]):
                        if TL and (SN == 1 or W != 2048 or MB >= 4 or M > 32):
                            continue  # the tail grid ignores W; decode rows only
                        if TL and KS > 1:
                            continue  # the tail grid takes whole k
                        q = dict(MB=0 if M == 1 else MB, R=R, D=D, W=W, BFMT=b)
                        if SN > 1:
                            q["SN"] = SN
                        if TL:
                            q["TL"] = 1
                        if KS > 1:
                            q["KS"] = KS
                        if MB >= 4 and M > 32:  # the shipped launchers' bound: 256 VGPRs
                            q["SN"] = SN
                            q["TPB"] = 512
                        out.append(("line", q))
        if b and M > 16:  # row tiles of 16 MB rows, at least two of them (8-bit weights)
            d = DOMAINS["line_mt"]
            for MBT in (m for m in d["MB"] if 16 * m < M):
                for R in d["R"]:
                    for D in d["D"]:
                        for S in d["S"]:
                            out.append(("line", dict(MB=MBT, R=R, D=D, MT=1, S=S, BFMT=b,
                                                     TPB=64 * S)))
    if M <= 32:
        MB = 1 if M <= 16 else 2
        for R in DOMAINS["ring"]["R"]:
            for D in DOMAINS["ring"]["D"]:
                out.append(("ring", dict(MB=MB, R=R, D=D, BFMT=b)))
        for R in DOMAINS["stream"]["R"]:
            for U in DOMAINS["stream"]["U"]:
                for AL in DOMAINS["stream"]["ALDS"]:
                    out.append(("stream", dict(MB=MB, R=R, U=U, BFMT=b, ALDS=AL)))
        for R in DOMAINS["shared"]["R"]:
            for U in DOMAINS["shared"]["U"]:
                for SN in DOMAINS["shared"]["SN"]:
                    out.append(("shared", dict(MB=MB, R=R, U=U, BFMT=b, SN=SN, TPB=1024)))
        if b:  # the phase-ordered kernel: 8-bit weights, N in 256 / KS row groups
            for ks in DOMAINS["phase"]["KS"]:
                if not phase_ns(N, ks):
                    continue
                for D in DOMAINS["phase"]["D"]:
                    q = dict(MB=0 if M == 1 else MB, NS=phase_ns(N, ks), D=D, BFMT=b)
                    if ks > 1:
                        q.update(KS=ks, KSL=1)
                    out.append(("phase", q))
    if b == 0:
        d = DOMAINS["ilv"]
        for BM in d["BM"]:
            for BN in d["BN"]:
                for BK in d["BK"]:
                    for ST in d["STAGES"]:
                        for G in d["GROUP"]:
                            for X in d["XCD"]:
                                for (WM, WN) in d["WAVES"]:
                                    for RS in d["RSP"]:
                                        for SW in d["SW"]:
                                            out.append(("ilv", _with_split(dict(
                                                BM=BM, BN=BN, BK=BK, WM=WM, WN=WN, STAGES=ST,
                                                GROUP=G, XCD=X, RSP=RS), SW)))
        d = DOMAINS["dma"]
        for BM in d["BM"]:
            for BN in d["BN"]:
                for BK in d["BK"]:
                    for ST in d["STAGES"]:
                        for SW in d["SWZ"]:
                            for G in d["GROUP"]:
                                for X in d["XCD"]:
                                    for (WM, WN) in d["WAVES"]:
                                        for MS in d["MS"]:
                                            out.append(("dma", dict(
                                                BM=BM, BN=BN, BK=BK, WM=WM, WN=WN, STAGES=ST,
                                                SWZ=SW, GROUP=G, XCD=X, XT=0, MINB=1, MS=MS)))
    if b in (1, 2) and M > 32:
        d = DOMAINS["ilv8"]
        for (BM, BN, WM, WN) in d["TILES"]:
            for BK in d["BK"]:
                for ST in d["STAGES"]:
                    for G in d["GROUP"]:
                        for X in d["XCD"]:
                            for RS in d["RSP"]:
                                for SW in d["SW"]:
                                    out.append(("ilv8", _with_split(dict(
                                        BM=BM, BN=BN, BK=BK, WM=WM, WN=WN, STAGES=ST, GROUP=G,
                                        XCD=X, RSP=RS, BFMT=b), SW)))
                                    # N in two parts (select.py TAIL): quarter-size tail
                                    # tiles behind 256 x 256, split-K tail behind 128 x 128 x 128
                                    tl = (1 if BM == 256 else
                                          2 if (BM, BN, BK) == (128, 128, 128) else 0)
                                    if tl and not SW:
                                        out.append(("ilv8", dict(
                                            BM=BM, BN=BN, BK=BK, WM=WM, WN=WN, STAGES=ST,
                                            GROUP=G, XCD=X, RSP=RS, BFMT=b, TAIL=tl)))
    d = DOMAINS["reg"]
    for BM in d["BM"]:
        for BN in d["BN"]:
            for MS in d["MS"]:
                for SW in d["SWZ"]:
                    out.append(("reg", dict(BM=BM, BN=BN, BK=64, WM=2, WN=2, MS=MS, SWZ=SW,
                                            GROUP=8, XCD=1, BFMT=b)))
    for kind, p in out:
        if legal(kind, p, M, N, K) is None:
            params = dict(p, kind=kind)
            yield Hyperform(plugin="gfx950", params=params, key=tag(kind, p))


def axes():
    return AXES
