"""Shipped dispatcher for gemm_fp16 on gfx950: (op, M, N, K, dtypes, arch) -> kernel id or None.

None means "caller's own path" (the fallback).  Same contract as the reference's
kernels/shipped/gemm_fp16/sm_70/select.py:23-58; this file is the ONE source of the M-band
ladder -- dispatch.inc is generated from it by gen_dispatch.py and a test checks they agree.

Rows are tried in order; the first row whose band holds (M, N) -- M <= M_max and N >= N_min --
AND whose kernel fits the shape (divisibility) is taken.  No such row: None, the caller's own
path.  (The reference stops at the first band that holds M; here a row that does not fit falls
through to the next one, so a narrower row can sit in front of a general one.)
  * M <= 32   line / stream: the weight-streaming decode kernels (HBM-bound; one pass over B);
              16 < M <= 32 at wide N: dma tiles of 64 weight rows and 256 k per stage.
              line = whole 128-byte weight lines by nontemporal LDS-DMA into per-wave rings
              (needs K % 128 and K <= 65536); stream (register-pipelined) takes the rest.  A = 1
              stages the activations in LDS once per workgroup (M = 1).
  * 32 < M <= 64  dma tiles of 128 k at wide N, then line rows with more activation blocks;
              narrow N (< 6144) takes the interleaved
              kernel with split-K (64 x 192 tiles).
  * 64 < M <= 256  narrow N (< 6144 for M <= 128): the interleaved kernel with split-K (128 x 128
              or 128 x 256 tiles); otherwise dma: k_gemm_dma tiles (64x64 to 128x128, 4-stage
              LDS-DMA ring), tile chosen by M and N; a line row takes N % 64 != 0.
  * M > 256   ilv: the interleaved 4-wave kernel (128 x 128 wave tiles, LDS-DMA copies,
              hand-pipelined substeps).
"""

ARCH = "gfx950"

# (M_max, N_min, tag, kind, template params).  First row that holds (M, N) and fits wins.
LADDER = [
    # M = 1, long K: a two-step ring (1.05x three steps at (1, 3840, 15360))
    (1, 0, "l0r1d2", "line", dict(MB=0, R=1, D=2, W=1024, KMIN=12288)),
    # two ring steps (1.03x three at (1, 15360, 3840))
    (1, 0, "l0r1d2w", "line", dict(MB=0, R=1, D=2, W=2048)),
    (1, 0, "s1a_r1u4", "stream", dict(MB=1, R=1, U=4, A=1)),
    # four ring steps (1.07x three at M = 8 and 16, (15360, 3840))
    (16, 12288, "l1r1n4d4", "line", dict(MB=1, R=1, D=4, SN=4, W=2048)),
    # narrow N, long K: k slices across workgroups (KS, fp32 partials reduced in slice order)
    # spread the 60 four-slab workgroups of N = 3840 over the part (1.10x the row below at
    # (16, 3840, 15360); 0.99x at M = 8)
    (16, 0, "l1r1n4d4k8", "line", dict(MB=1, R=1, D=4, SN=4, W=2048, KS=8, KMIN=12288)),
    (16, 0, "l1r1d4", "line", dict(MB=1, R=1, D=4, W=2048)),
    (16, 0, "s16r1u4", "stream", dict(MB=1, R=1, U=4, A=0)),
    # 16 < M <= 32, wide N: LDS-DMA tiles of 64 weight rows that take 256 k per stage (512
    # contiguous bytes of each weight row per copy), one workgroup per 64 rows: 1.01 / 1.03 /
    # 1.08x the ring row below at M = 24, 32 (15360, 3840) and 32 (12288, 4096); at M <= 16
    # the ring rows above stay ahead (0.96-0.97x)
    (32, 12288, "d32x64k256s3", "dma",
     dict(BM=32, BN=64, BK=256, WM=2, WN=4, STAGES=3, SWZ=1, GROUP=8, XCD=1, MS=16)),
    # four ring stages (1.08-1.12x three at M = 24-32, N = 12288-15360)
    (32, 12288, "l2r1n4d4", "line", dict(MB=2, R=1, D=4, SN=4, W=2048)),
    # k slices as above (1.28x the row below at (32, 3840, 15360)), four ring steps (1.07x /
    # 1.07x / 1.09x three at M = 24 / 32 (K = 15360) and M = 32 (K = 12288), N = 3840)
    (32, 0, "l2r1n4d4k8", "line", dict(MB=2, R=1, D=4, SN=4, W=2048, KS=8, KMIN=12288)),
    (32, 0, "l2r1d4", "line", dict(MB=2, R=1, D=4, W=2048)),
    (32, 0, "s32r1u4", "stream", dict(MB=2, R=1, U=4, A=0)),
    # 32 < M <= 64, wide N: 64 x 64 LDS-DMA tiles of 128 k (1.04x the four-slab ring row
    # l4r1n4d3 they replace, at M = 48 and 64, (15360, 3840); that row needed the same N % 64
    # and K % 128)
    (64, 12288, "d64x64k128s3", "dma",
     dict(BM=64, BN=64, BK=128, WM=2, WN=2, STAGES=3, SWZ=1, GROUP=8, XCD=1, MS=16)),
    # narrow N, long K: split-K over the interleaved kernel's tiles (fp32 partials in the
    # workspace, reduced in order) gives the 20 column tiles of N = 3840 enough workgroups;
    # measured by the variant driver (tempo/plugins/gfx950/tune.py) at (64|128|256, 3840, 15360);
    # at M <= 64 the 64 x 128 tiles on four stages (1.06x the 64 x 192 three-stage row)
    (64, 0, "i64x128k64s4w256", "ilv",
     dict(BM=64, BN=128, BK=64, WM=2, WN=2, STAGES=4, GROUP=8, XCD=1, RSP=8, SW=256, MINKT=8,
          NMAX=6144)),
    (64, 0, "l4r1d3", "line", dict(MB=4, R=1, D=3, W=2048)),
    # 64 < M <= 256: LDS-DMA tiles with a 4-stage ring.  Per CU they keep more operand bytes in
    # flight than the line kernel (which re-reads the activations per slab wave) or the
    # register-staged tiles.  Narrow N gives few workgroups (N = 3840: 60 column tiles)
    # 128-k stages (256 contiguous bytes of each weight row per copy): 1.01-1.06x the 64-k
    # four-stage row at M = 100, 128 (15360, 3840) and 128 (12288, 4096); at M = 200-256 the
    # 128 x 128 tiles of 128 k lose (0.92-0.97x), so the M <= 256 rows keep 64 k
    (128, 12288, "d128x64k128s3", "dma",
     dict(BM=128, BN=64, BK=128, WM=2, WN=2, STAGES=3, SWZ=1, GROUP=8, XCD=1, MS=16)),
    (128, 12288, "d128x64k64s4", "dma",
     dict(BM=128, BN=64, BK=64, WM=2, WN=2, STAGES=4, SWZ=1, GROUP=8, XCD=1, MS=16)),
    (128, 0, "i128x128k64s3w256", "ilv",
     dict(BM=128, BN=128, BK=64, WM=2, WN=2, STAGES=3, GROUP=8, XCD=1, RSP=8, SW=256, MINKT=8,
          NMAX=6144)),
    (128, 0, "d64x64k64s4", "dma",
     dict(BM=64, BN=64, BK=64, WM=2, WN=2, STAGES=4, SWZ=1, GROUP=8, XCD=1, MS=16)),
    (128, 0, "l8r1n2d3", "line", dict(MB=8, R=1, D=3, SN=2, W=2048)),
    (256, 12288, "d128x128k64s4", "dma",
     dict(BM=128, BN=128, BK=64, WM=2, WN=2, STAGES=4, SWZ=1, GROUP=8, XCD=1, MS=16)),
    (256, 6144, "d128x64k64s4", "dma",
     dict(BM=128, BN=64, BK=64, WM=2, WN=2, STAGES=4, SWZ=1, GROUP=8, XCD=1, MS=16)),
    (256, 0, "i128x256k64s3w256", "ilv",
     dict(BM=128, BN=256, BK=64, WM=1, WN=4, STAGES=3, GROUP=8, XCD=1, RSP=8, SW=256, MINKT=8)),
    (256, 0, "d64x64k64s4", "dma",
     dict(BM=64, BN=64, BK=64, WM=2, WN=2, STAGES=4, SWZ=1, GROUP=8, XCD=1, MS=16)),
    (1 << 30, 0, "i256x256k64w4r8", "ilv",
     dict(BM=256, BN=256, BK=64, WM=2, WN=2, STAGES=2, GROUP=8, XCD=1, RSP=8)),
]

# Fused gate/up ladder (C = silu(A.B[0..N)^T) * (A.B[N..2N)^T), N = output width): the decode
# kernels with EPI = 1 (shared: the slab waves pair up, gate and up; stream: each wave carries
# the gate and the up row groups of its slab), rows measured on (N, K) = (17408, 5120) and
# (7680, 3840) against the plain GEMM + a separate silu*mul kernel; then the interleaved prefill
# kernel with EPI = 1 (each tile holds BN/2 gate and the BN/2 matching up rows of B, and pairs
# them in the epilogue) for every M.
LADDER_GATE_UP = [
    (1, 0, "gl0r1n2d3", "line", dict(MB=0, R=1, D=3, SN=2, W=2048)),
    (16, 12288, "gl1r1n4d3", "line", dict(MB=1, R=1, D=3, SN=4, W=2048)),
    (16, 0, "gl1r1d3", "line", dict(MB=1, R=1, D=3, W=2048)),
    (32, 12288, "gl2r1n4d3", "line", dict(MB=2, R=1, D=3, SN=4, W=2048)),
    (32, 0, "gl2r1d3", "line", dict(MB=2, R=1, D=3, W=2048)),
    (1, 0, "gh1r1u2n2", "shared", dict(MB=1, R=1, U=2, SN=2, TPB=512)),
    (16, 0, "gh16r1u4n2", "shared", dict(MB=1, R=1, U=4, SN=2, TPB=512)),
    (32, 0, "gh32r1u4n4", "shared", dict(MB=2, R=1, U=4, SN=4, TPB=1024)),
    (32, 0, "g32r1u4", "stream", dict(MB=2, R=1, U=4, A=0)),
    (128, 0, "gi128x256k64s3", "ilv",
     dict(BM=128, BN=256, BK=64, WM=1, WN=4, STAGES=3, GROUP=8, XCD=1, RSP=8)),
    # TAIL: where the last round of tiles (128 output columns each) is at most a quarter full
    # ((2048, 17408): 1088 tiles), the whole rounds, then the rest on ILV_TAIL tiles
    (1 << 30, 0, "gi256x256k64w4r8t", "ilv",
     dict(BM=256, BN=256, BK=64, WM=2, WN=2, STAGES=2, GROUP=8, XCD=1, RSP=8, TAIL=1)),
]

# the tail tiles of the gate/up TAIL row: BM, BN, BK, WM, WN, STAGES of k_gemm_ilv (no split)
ILV_TAIL = {1: (128, 128, 64, 2, 2, 3)}

# Divisibility each kind needs (checked at run time by dispatch.inc, mirrored here).
STREAM_K_STEP = 64  # k per pipeline step of the stream kernel
STREAM_N_ROWS = 16  # weight rows per MFMA row group (times R)
LINE_K_STEP = 128   # k per step of the line kernel (one 128-byte line of an int8 row)
LINE_K_MAX = 65536  # the line kernel's LDS holds one wave's metadata (fmt 2): bounded k


def _fits_gate_up(kind, p, M, N, K):
    # N is the output width; the slab waves of the shared kernel and of the line kernel with
    # SN >= 2 pair up (SN/2 output slabs per workgroup)
    if kind == "line" and p.get("SN", 1) >= 2:
        return (N % (STREAM_N_ROWS * p["R"] * p["SN"] // 2) == 0 and K % LINE_K_STEP == 0
                and K <= LINE_K_MAX)
    if kind == "shared":
        return (p["SN"] % 2 == 0 and N % (STREAM_N_ROWS * p["R"] * p["SN"] // 2) == 0
                and K % (STREAM_K_STEP * p["U"]) == 0)
    if kind == "ilv":  # a tile covers BN/2 output columns
        return N % (p["BN"] // 2) == 0 and K % max(64, p["BK"]) == 0 and K <= ilv_ld_max(p)
    return _fits(kind, p, M, N, K)


def ilv_ld_max(p):
    """Largest leading dimension the interleaved kernel takes: its copies address a BM- or
    BN-row panel with 31-bit byte offsets."""
    return (2 ** 31 - 1) // (2 * max(p["BM"], p["BN"]))


def _fits(kind, p, M, N, K):
    if kind == "line":  # NMAX / KMIN (optional): the row holds narrower N / longer K only
        return (N % (STREAM_N_ROWS * p["R"] * p.get("SN", 1)) == 0 and K % LINE_K_STEP == 0
                and K <= LINE_K_MAX and N < p.get("NMAX", 1 << 30) and K >= p.get("KMIN", 0))
    if kind == "ilv":  # NMAX (optional): the row holds narrower N only
        return (N % p["BN"] == 0 and K % max(64, p["BK"]) == 0 and K <= ilv_ld_max(p)
                and N < p.get("NMAX", 1 << 30))
    if kind == "stream":
        return N % (STREAM_N_ROWS * p["R"]) == 0 and K % (STREAM_K_STEP * p["U"]) == 0
    if kind == "shared":
        return (N % (STREAM_N_ROWS * p["R"] * p["SN"]) == 0
                and K % (STREAM_K_STEP * p["U"]) == 0)
    # mfma: NMAX (optional) as for the line rows
    return N % p["BN"] == 0 and K % p["BK"] == 0 and N < p.get("NMAX", 1 << 30)


def select(op, M, N, K, dtype_a="fp16", dtype_b="fp16", dtype_c="fp16", arch=ARCH):
    if op != "gemm" or arch != ARCH:
        return None
    if (dtype_a, dtype_b, dtype_c) != ("fp16", "fp16", "fp16"):
        return None
    if M <= 0 or N <= 0 or K <= 0 or N % 8 or K % 8:
        return None
    return _first(LADDER, M, N, K)


def _first(ladder, M, N, K, fits=_fits):
    for m_max, n_min, tag, kind, p in ladder:
        if M <= m_max and N >= n_min and fits(kind, p, M, N, K):
            return dict(tag=tag, kind=kind, **p)
    return None


def select_gate_up(op, M, N, K, dtype_a="fp16", dtype_b="fp16", dtype_c="fp16", arch=ARCH):
    """The fused gate/up row for output width N (B has 2N rows), or None."""
    if op != "gemm_gate_up" or arch != ARCH:
        return None
    if (dtype_a, dtype_b, dtype_c) != ("fp16", "fp16", "fp16"):
        return None
    if M <= 0 or N <= 0 or K <= 0 or N % 8 or K % 8:
        return None
    return _first(LADDER_GATE_UP, M, N, K, _fits_gate_up)
