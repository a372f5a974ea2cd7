"""Shipped dispatcher for gemm_w8a16 on gfx950: (op, M, N, K, fmt, group) -> kernel id or None.

Same contract as kernels/shipped/gemm_fp16/gfx950/select.py (reference pattern:
kernels/shipped/gemm_fp16/sm_70/select.py:23-58).  The weight formats:
  fmt 1  int8 symmetric, fp16 scale per output channel
  fmt 2  uint8 asymmetric, fp16 scale + uint8 zero-point per (row, group of `group` k)
Every row of the ladder is instantiated for both formats; dispatch.inc is generated from this
file by gen_dispatch.py, and so is prefill.inc (the instantiations of the interleaved int8
prefill kernel, built in their own translation unit, launch_prefill.hip).
"""

ARCH = "gfx950"
FORMATS = (1, 2)

# (M_max, N_min, tag, kind, template params).  Rows are tried in order; the first row whose band
# holds (M, N) -- M <= M_max and N >= N_min -- whose weight format is listed (params "fmts";
# absent = both) and whose kernel fits the shape is taken.
LADDER = [
    # M = 1, long K: k slices across workgroups (KS, fp32 partials reduced in slice order) spread
    # the 320 slabs of N = 5120 evenly over the part; two ring steps (1.04x / 1.12x the rows
    # below at (1, 5120, 17408), int8 / uint8)
    # M = 1, uint8, long K on N = 4096..7168: the phase-ordered kernel over the whole K (17
    # phases dealt 3 or 2 per wave at K = 17408), three ring steps: 1.06x the k-slice row below
    # at (1, 5120, 17408) (int8 1.02x, not taken)
    (1, 4096, "p0n2d3", "phase", dict(MB=0, NS=2, D=3, NMAX=7168, KMIN=13312, KMAX=20480,
                                      fmts=(2,))),
    (1, 0, "l0r1d2k8", "line", dict(MB=0, R=1, D=2, W=2048, KS=8, KMIN=12288)),
    # M = 1 on N = 4096..7168, K < 12288, K % 1024 == 0: the phase-ordered kernel, 20-24 rows
    # per CU (a slab of 16 and one of 4-8), no tail: 1.08x / 1.10x the row below at (1, 5120,
    # 5120), 1.00x / 1.03x at (1, 5120, 6144), int8 / uint8 (at N = 7168: 0.95x, not taken)
    (1, 4096, "p0n2d2", "phase", dict(MB=0, NS=2, D=2, NMAX=7168, KMAX=12288)),
    # M = 1 on N = 4096..6144: two slab waves per activation ring, two ring steps (1.10-1.14x
    # the five-step row it replaced at N = 5120, K = 5120-6144)
    (1, 4096, "l0r1n2d2", "line", dict(MB=0, R=1, D=2, SN=2, W=2048, NMAX=6145)),
    # M = 1, narrow N: two ring steps (1.24x four at (1, 1024, 5120))
    (1, 0, "l0r1d2", "line", dict(MB=0, R=1, D=2, W=2048, NMAX=4096)),
    # M = 1, wider N: two ring steps; where a CU holds 4+ slab waves (8.5 at N = 34816) two steps
    # per wave already keep ~35 KiB per CU in flight.  1.06x / 1.02x the four-step row it
    # replaced at (1, 34816, 5120) and 1.10x / 1.05x at (1, 7168, 5120), int8 / uint8
    # M = 1, uint8, wide N: the phase-ordered kernel (k loop outside the slab loop, one
    # workgroup per CU, the workgroup's metadata staged once by LDS-DMA): 1.06x the row below at
    # (1, 34816, 5120) (int8: 1.01x, the row below stays)
    (1, 12288, "p0n9d3", "phase", dict(MB=0, NS=9, D=3, KMAX=12288, fmts=(2,))),
    (1, 0, "l0r1d2w", "line", dict(MB=0, R=1, D=2, W=2048)),
    # M <= 16 / 32, wide N: the tail grid -- whole rounds of 4- / 8-slab workgroups (one ring of
    # activations each) and one single-wave workgroup per remaining slab, so the slabs per CU
    # differ by at most one (1.10-1.19x / 1.29-1.31x the rows after them at (34816, 5120))
    # M <= 16, wide N: the phase-ordered kernel -- each CU reads the activations once, a phase
    # (128 k) ahead of their use, and its ring carries weights only: 1.11x / 1.17x the tail grid
    # below at (16, 34816, 5120), int8 / uint8
    (16, 12288, "p1n9d4", "phase", dict(MB=1, NS=9, D=4, KMAX=12288)),
    (16, 12288, "l1r1n4d2t", "line", dict(MB=1, R=1, D=2, SN=4, W=2048, TL=1)),
    (16, 12288, "l1r1n4d3", "line", dict(MB=1, R=1, D=3, SN=4, W=2048)),
    # uint8, long K: the phase-ordered kernel with 8 k slices over all 256 CUs (32 row groups of
    # 160 rows, 17 steps of 128 k each): 1.05x the row below at (16, 5120, 17408) (int8 1.00x)
    (16, 0, "p1n10d4k8", "phase", dict(MB=1, NS=10, D=4, KS=8, KMIN=12288, fmts=(2,))),
    # long K: k slices (1.17x / 1.25x the row below at (16, 5120, 17408))
    (16, 0, "l1r1n4d2k8", "line", dict(MB=1, R=1, D=2, SN=4, W=2048, KS=8, KMIN=12288)),
    # narrow N: one slab wave per ring, k slices over the part (1.43-1.47x the two-slab
    # four-step row at (16, 1024, 5120))
    (16, 0, "l1r1d2k8", "line", dict(MB=1, R=1, D=2, W=2048, KS=8, NMAX=2048)),
    # two ring steps (1.10-1.11x four at (16, 5120 | 7168, 5120))
    (16, 0, "l1r1n2d2", "line", dict(MB=1, R=1, D=2, SN=2, W=2048)),
    # M <= 32, uint8: 1.05x the tail grid below at (32, 34816, 5120) (int8: 1.00x, it stays)
    (32, 12288, "p2n9d4", "phase", dict(MB=2, NS=9, D=4, KMAX=12288, fmts=(2,))),
    (32, 12288, "l2r1n8d2t", "line", dict(MB=2, R=1, D=2, SN=8, W=2048, TL=1)),
    (32, 12288, "l2r1n4d4", "line", dict(MB=2, R=1, D=4, SN=4, W=2048)),
    # long K: k slices, eight slab waves per activation ring (1.37x / 1.46x the row below at
    # (32, 5120, 17408), int8 / uint8)
    (32, 0, "l2r1n8d3k8", "line", dict(MB=2, R=1, D=3, SN=8, W=1024, KS=8, KMIN=12288, fmts=(1,))),
    # uint8: the phase-ordered kernel with 8 k slices, 1.07x the row below at (32, 5120, 17408)
    (32, 0, "p2n10d4k8", "phase", dict(MB=2, NS=10, D=4, KS=8, KMIN=12288, fmts=(2,))),
    (32, 0, "l2r1n8d2k8", "line", dict(MB=2, R=1, D=2, SN=8, W=2048, KS=8, KMIN=12288, fmts=(2,))),
    # narrow N: one slab wave per ring, k slices (1.53-1.62x at (32, 1024, 5120))
    (32, 0, "l2r1d2k8", "line", dict(MB=2, R=1, D=2, W=2048, KS=8, NMAX=2048)),
    # four slab waves per ring, two steps, k slices where they even out the grid (1.20x / 1.30x
    # the two-slab four-step row at (32, 5120, 6144); at K = 5120 the slices leave the grid
    # uneven and the row below stays ahead)
    (32, 0, "l2r1n4d2k8", "line", dict(MB=2, R=1, D=2, SN=4, W=2048, KS=8, KMIN=6144)),
    (32, 0, "l2r1n2d4", "line", dict(MB=2, R=1, D=4, SN=2, W=2048)),
    (1, 0, "s1a_r1u8", "stream", dict(MB=1, R=1, U=8, A=1)),
    (1, 0, "s1a_r1u4", "stream", dict(MB=1, R=1, U=4, A=1)),
    (8, 0, "s8r2u4", "stream", dict(MB=1, R=2, U=4, A=0)),
    (16, 0, "h16r1u4n2", "shared", dict(MB=1, R=1, U=4, SN=2)),
    (16, 0, "s16r1u4", "stream", dict(MB=1, R=1, U=4, A=0)),
    (32, 0, "h32r1u4n2", "shared", dict(MB=2, R=1, U=4, SN=2, TPB=512)),
    (64, 12288, "l4r1n4d3", "line", dict(MB=4, R=1, D=3, SN=4, W=2048)),
    # 32 < M <= 64, narrow N and long K: the int8 interleaved kernel on 128 x 256 tiles of 128 k
    # (whole weight lines) with split-K (1.09x the 64-k tile row at (64, 5120, 17408), which was
    # 1.3x the line row)
    (64, 0, "i8x128x256k128s2w256", "ilv8",
     dict(BM=128, BN=256, BK=128, WM=1, WN=4, STAGES=2, GROUP=8, XCD=1, RSP=8, SW=256, MINKT=8,
          NMAX=12288, KMIN=12288)),
    # 32 < M <= 64, narrow N: 128 x 128 tiles of 128 k, split-K (1.23x the line row below at
    # (64, 7168, 5120))
    (64, 0, "i8x128x128w1x4k128s2w256", "ilv8",
     dict(BM=128, BN=128, BK=128, WM=1, WN=4, STAGES=2, GROUP=8, XCD=1, RSP=8, SW=256, MINKT=8,
          NMAX=12288)),
    (64, 0, "l4r1n2d3", "line", dict(MB=4, R=1, D=3, SN=2, W=2048)),
    # 64 < M <= 128, narrow N (< 2048): the line kernel on row tiles of 32 rows, each workgroup
    # one row tile x 16 weight rows over the whole K on four waves (k chunks summed through LDS);
    # the weight rows of one slab group are read by the row tiles on one XCD, from its L2 after
    # the first (1.50x / 1.41x the line row with eight activation blocks and k slices across
    # workgroups it replaced, at (128, 1024, 5120), int8 / uint8)
    (128, 0, "l2r1d2m4", "line", dict(MB=2, R=1, D=2, MT=1, S=4, NMAX=2048)),
    # 64 < M <= 128, N < 12288, uint8 and long K: 128 x 256 tiles of 128 k, split-K (1.11x the
    # 64-k row at (128, 5120, 17408))
    (128, 0, "i8x128x256k128s2w256", "ilv8",
     dict(BM=128, BN=256, BK=128, WM=1, WN=4, STAGES=2, GROUP=8, XCD=1, RSP=8, SW=256, MINKT=8,
          NMAX=12288, KMIN=12288, fmts=(2,))),
    # 64 < M <= 128, N < 12288: 128 x 128 tiles of 128 k -- every k-tile takes whole 128-byte
    # lines of the weight rows -- two stages, split-K (1.04-1.21x the 64-k tile rows at N =
    # 5120-7168, both formats); 1 x 4 waves of 128 x 32, each dequantising only its own weight
    # rows (1.03-1.08x 2 x 2 waves of 64 x 64)
    (128, 0, "i8x128x128w1x4k128s2w256", "ilv8",
     dict(BM=128, BN=128, BK=128, WM=1, WN=4, STAGES=2, GROUP=8, XCD=1, RSP=8, SW=256, MINKT=8,
          NMAX=12288)),
    # 64 < M <= 128, wide N, uint8, where 128 x 128 tiles make whole rounds and at most a quarter
    # round more ((128, 34816): 256 tiles, then 16): the whole rounds unsplit on three stages,
    # the remaining columns split-K (TAIL = 2); 1.10x the 128 x 256 row below, whose 136 tiles
    # leave 120 CUs idle (int8: 0.94x, the row below stays)
    (128, 12288, "i8x128x128w1x4k128s3t2", "ilv8",
     dict(BM=128, BN=128, BK=128, WM=1, WN=4, STAGES=3, GROUP=8, XCD=1, RSP=8, TAIL=2,
          fmts=(2,))),
    # 64 < M <= 128: 128 x 256 tiles (one tile row), split-K where the column tiles are too few
    # to fill the part (the variant driver's rows: 1.5-2.9x the line and register-staged rows)
    (128, 0, "i8x128x256s3w256", "ilv8",
     dict(BM=128, BN=256, BK=64, WM=1, WN=4, STAGES=3, GROUP=8, XCD=1, RSP=8, SW=256, MINKT=8)),
    (128, 0, "l8r1n2d3", "line", dict(MB=8, R=1, D=3, SN=2, W=2048, NMAX=12288)),
    (256, 0, "m128x128k64", "mfma",
     dict(BM=128, BN=128, BK=64, WM=2, WN=2, MS=32, SWZ=1, GROUP=8, XCD=1)),
    # narrow N (fewer than 8 tiles of 256 columns): 256x256 tiles leave most CUs idle; 128 x 128
    # tiles of 128 k with split-K fill the part (1.08x the 128 x 256 64-k row at (2048, 1024,
    # 5120), which was 1.97x the 128 x 128 register-staged row behind them)
    (1 << 30, 0, "i8x128x128w1x4k128s2w256", "ilv8",
     dict(BM=128, BN=128, BK=128, WM=1, WN=4, STAGES=2, GROUP=8, XCD=1, RSP=8, SW=256, MINKT=8,
          NMAX=2048)),
    # what the 128-k tiles leave at narrow N: K % 128 == 64 (int8 only; uint8 groups are whole
    # 128-k)
    (1 << 30, 0, "m128x128k64s16", "mfma",
     dict(BM=128, BN=128, BK=64, WM=2, WN=2, MS=16, SWZ=1, GROUP=8, XCD=1, NMAX=2048, fmts=(1,))),
    # FILL: where one round of 192 x 256 tiles holds the whole grid and has more tiles than the
    # 256 x 256 grid (220 against 160 tiles at (2048, 5120)), the 192-row tiles fill more of the
    # part: 1.05-1.10x the row below at (2048, 5120, 5120 | 6144 | 17408) in both formats,
    # 1.07-1.26x at M = 512-1536 (variant driver, paired rounds); a 192-row tile's M past the
    # last row is predicated like any other
    (1 << 30, 0, "i8x192x256w1x4k64s3f", "ilv8",
     dict(BM=192, BN=256, BK=64, WM=1, WN=4, STAGES=3, GROUP=8, XCD=1, RSP=8, FILL=1)),
    # TAIL: where the last round of 256 x 256 tiles is at most a quarter full (four rounds and
    # 64 tiles at (2048, 34816)), the columns of the whole rounds run on these tiles and the rest
    # of N on ILV8_TAIL_TILE tiles, one round of their own; any other grid runs this row plain
    # 1 x 4 waves (wave tiles of 256 x 64): each wave dequantises only its own 64 weight rows,
    # where 2 x 2 waves dequantise every weight fragment twice (1.04-1.05x at M = 2048)
    (1 << 30, 0, "i8x256w1x4k64s3t", "ilv8",
     dict(BM=256, BN=256, BK=64, WM=1, WN=4, STAGES=3, GROUP=8, XCD=1, RSP=8, TAIL=1)),
    (1 << 30, 0, "m256x256k64", "mfma",
     dict(BM=256, BN=256, BK=64, WM=2, WN=2, MS=32, SWZ=1, GROUP=8, XCD=1, fmts=(1,))),
]

# Fused gate/up ladder (C = silu(A.deq(W)[0..N)^T) * (A.deq(W)[N..2N)^T), N = output width): the
# decode kernels with EPI = 1 (shared: paired gate/up slab waves), rows measured on the
# production gate_up shape (N, K) = (17408, 5120), both formats; then the interleaved int8
# kernel with EPI = 1 for every M.
LADDER_GATE_UP = [
    # the phase-ordered kernel with the gate/up epilogue (a workgroup's 68 output columns take
    # its 136 rows: the gate rows and the matching up rows), wide N: at (17408 x 2, 5120) uint8
    # 1.04x the paired line row at M = 1 (int8 1.01x: not taken)
    (1, 12288, "gp0n9d4", "phase", dict(MB=0, NS=9, D=4, KMAX=12288, fmts=(2,))),
    # two ring steps at M = 1 and M = 32 (1.05-1.08x / 1.02-1.06x four, both formats)
    (1, 0, "gl0r1n2d2", "line", dict(MB=0, R=1, D=2, SN=2, W=2048)),
    # M <= 16 / 32, wide N: the tail grid -- whole rounds of paired workgroups (SN/2 output
    # slabs each), then one gate, up pair of waves per remaining output slab; at
    # (17408 x 2, 5120), one process: M = 32 39.5 / 41.6 us (int8 / uint8) against 46.9 / 48.8
    # for the paired row below, and 1.18x / 1.13x the tail grid with one wave carrying both
    # halves of a tail slab; M = 16 36.9 / 38.9 us against 38.4 / 40.3 for the row below
    # M <= 16: 1.11x / 1.15x the tail grid below at (17408 x 2, 5120), int8 / uint8
    (16, 12288, "gp1n9d4", "phase", dict(MB=1, NS=9, D=4, KMAX=12288)),
    (16, 12288, "gl1r1n4d2t", "line", dict(MB=1, R=1, D=2, SN=4, W=2048, TL=1)),
    (16, 12288, "gl1r1n4d3", "line", dict(MB=1, R=1, D=3, SN=4, W=2048)),
    (16, 0, "gl1r1n2d4", "line", dict(MB=1, R=1, D=4, SN=2, W=2048)),
    # M <= 32, uint8: 1.04x the tail grid below (int8 1.01x: not taken)
    (32, 12288, "gp2n9d4", "phase", dict(MB=2, NS=9, D=4, KMAX=12288, fmts=(2,))),
    (32, 12288, "gl2r1n8d2t", "line", dict(MB=2, R=1, D=2, SN=8, W=2048, TL=1)),
    (32, 12288, "gl2r1n4d2", "line", dict(MB=2, R=1, D=2, SN=4, W=2048)),
    (32, 0, "gl2r1n2d4", "line", dict(MB=2, R=1, D=4, SN=2, W=2048)),
    (1, 0, "g1a_r1u2", "stream", dict(MB=1, R=1, U=2, A=1, fmts=(1,))),
    (1, 0, "g1a_r1u8", "stream", dict(MB=1, R=1, U=8, A=1, fmts=(2,))),
    (1, 0, "g1a_r1u4", "stream", dict(MB=1, R=1, U=4, A=1, fmts=(2,))),
    (16, 0, "gh16r1u2n2", "shared", dict(MB=1, R=1, U=2, SN=2, TPB=512, fmts=(1,))),
    (16, 0, "gh16r1u4n2", "shared", dict(MB=1, R=1, U=4, SN=2, TPB=512, fmts=(2,))),
    (32, 0, "gh32r1u2n4", "shared", dict(MB=2, R=1, U=2, SN=4, TPB=1024, fmts=(1,))),
    (32, 0, "gh32r1u4n4", "shared", dict(MB=2, R=1, U=4, SN=4, TPB=512, fmts=(2,))),
    (32, 0, "g32r1u4", "stream", dict(MB=2, R=1, U=4, A=0)),
    # M > 32 (and what the decode rows leave): the interleaved int8 kernel with EPI = 1 -- each
    # tile holds BN/2 gate and the BN/2 matching up weight rows and pairs them in the epilogue
    (128, 0, "gi8x128x256k128s2", "ilv8",
     dict(BM=128, BN=256, BK=128, WM=1, WN=4, STAGES=2, GROUP=8, XCD=1, RSP=8)),
    # TAIL = 1 as in the plain ladder: where the last round of tiles (128 output columns each) is
    # at most a quarter full ((2048, 17408): 1088 tiles), the rest on 128 x 128 tiles of 128 k
    (1 << 30, 0, "gi8x256w1x4k64s3t", "ilv8",
     dict(BM=256, BN=256, BK=64, WM=1, WN=4, STAGES=3, GROUP=8, XCD=1, RSP=8, TAIL=1)),
]

# the tail part of the TAIL rows: BM, BN, BK, WM, WN, STAGES of k_gemm_ilv8, then SW and MINKT of
# its split-K (0, 0: no split).  TAIL = 1: a quarter-size tile, and a row whose grid does not
# split runs plain; TAIL = 2: the same tiles with split-K, and the row fits only where N splits.
ILV8_TAIL = {1: (128, 128, 128, 1, 4, 2, 0, 0), 2: (128, 128, 128, 1, 4, 2, 256, 2)}


def tail_split(M, N, BM=256, BN=256, cus=256):
    """Columns the whole rounds of a TAIL row take (0: the row runs plain, one dispatch; else the
    rest of N runs as a second launch on the ILV8_TAIL tiles) -- ilv8_tail_cols of launch.h."""
    nm, nn = -(-M // BM), N // BN
    tiles = nm * nn
    whole = tiles // cus * cus
    if whole == 0 or whole % nm or whole // nm == nn or 4 * (tiles - whole) > cus:
        return 0
    return whole // nm * BN

STREAM_K_STEP = 64
STREAM_N_ROWS = 16
LINE_K_STEP = 128   # k per step of the line kernel (one 128-byte line of an int8 row)
LINE_K_MAX = 65536  # the line kernel's LDS holds one wave's metadata (fmt 2): bounded k
LINE_CUS = 256      # CUs of the part: one round of workgroups of the line kernel's tail grid
LINE_LDS = 160 * 1024


def _line_lds(p, fmt, K, sn, rr=None):
    """LDS of one workgroup of the line kernel with one k chunk, as StreamLine::lds(1, K/128)
    declares it: sn weight rings of rr row groups each (their own activation slots too when
    sn = 1), the fmt 2 metadata of K/128 groups per wave, and (sn > 1) the shared activation
    ring of D + 1 slots.  rr defaults to R (2R: a fused gate/up wave carrying both halves)."""
    rr = p["R"] if rr is None else rr
    wslot, aslot = rr * 2048, (p["MB"] * 16 * 256 if p["MB"] else 256)
    meta = -(-(rr * 16 * (K // LINE_K_STEP) * 3) // 16) * 16 if fmt == 2 else 0
    wave = -(-(p["D"] * (wslot + (aslot if sn == 1 else 0)) + meta) // 1024) * 1024
    act = -(-((p["D"] + 1) * aslot) // 1024) * 1024 if sn > 1 else 0
    return sn * wave + act


def line_mt_fits(p, K, fmt):
    """A row-tiled line row (MT = 1, launch.h line_mt_config): some count of waves, at most S,
    each taking an equal count of whole 128-k steps, whose rings (+ fmt 2 metadata of those
    steps) fit the LDS; with more than one wave the k chunks' partial sums ([S][R][MB] x 1 KiB)
    reuse the rings' bytes."""
    steps = K // LINE_K_STEP
    for s in range(min(p["S"], steps), 0, -1):
        per = -(-steps // s)
        s2 = -(-steps // per)
        rings = s2 * _line_lds(p, fmt, per * LINE_K_STEP, 1)
        if (max(rings, s2 * p["R"] * p["MB"] * 1024) if s2 > 1 else rings) <= LINE_LDS:
            return True
    return False


def line_tail_fits(p, N, K, fmt, epi=0):
    """The tail grid (TL = 1) of the line kernel (launch.h line_tail_grid): q >= 1 whole rounds of
    SN-slab-wave workgroups, at most one remaining output slab per CU, and a CU's q workgroups
    plus one tail resident together (LDS and 16 waves).  epi = 1 (fused gate/up): SN/2 output
    slabs per workgroup, and a tail workgroup is a gate, up pair of waves sharing an activation
    ring (one wave otherwise)."""
    sno = p["SN"] // 2 if epi else p["SN"]
    slabs, rnd = N // (STREAM_N_ROWS * p["R"]), LINE_CUS * sno
    q = slabs // rnd
    if q < 1 or slabs - q * rnd > LINE_CUS or K > LINE_K_MAX:
        return False
    lds = max(_line_lds(p, fmt, K, p["SN"]), _line_lds(p, fmt, K, 2 if epi else 1))
    return (q + 1) * lds <= LINE_LDS and (q + 1) * p["SN"] <= 16


def _fits_gate_up(kind, p, M, N, K, fmt=1):
    # N is the output width; the slab waves of the shared kernel and of the line kernel with
    # SN >= 2 pair up (SN/2 output slabs per workgroup)
    if kind == "phase":  # a workgroup's N / 256 output columns (a multiple of 4) take 2 N / 256
        # rows -- phase_gu_fits of launch.h
        return (N % LINE_CUS == 0 and (N // LINE_CUS) % 4 == 0
                and phase_fits(p, M, 2 * N, K, fmt) and K < p.get("KMAX", 1 << 30))
    if kind == "line" and p.get("TL"):  # tail grid of paired workgroups
        return (N % (STREAM_N_ROWS * p["R"]) == 0 and K % LINE_K_STEP == 0
                and line_tail_fits(p, N, K, fmt, epi=1))
    if kind == "line" and p.get("SN", 1) >= 2:
        return (N % (STREAM_N_ROWS * p["R"] * p["SN"] // 2) == 0 and K % LINE_K_STEP == 0
                and K <= LINE_K_MAX)
    if kind == "shared":
        return (p["SN"] % 2 == 0 and N % (STREAM_N_ROWS * p["R"] * p["SN"] // 2) == 0
                and K % (STREAM_K_STEP * p["U"]) == 0)
    if kind == "ilv8":  # a tile covers BN/2 output columns; a scale group is two k-tiles
        return N % (p["BN"] // 2) == 0 and K % 128 == 0 and K <= ilv_ld_max(p)
    return _fits(kind, p, M, N, K, fmt)


PHASE_WAVES = 8  # k_stream_phase: waves (k chunks) per workgroup


def phase_lds(p, K, fmt):
    """LDS of k_stream_phase (StreamPhase::lds of the kernel): the weight rings, the activation
    staging (after the loop: the chunk partial sums), the output image (whole K only), the
    metadata (k slices: the slice's groups, 4 bytes apart)."""
    mb, ns, d, ks = p["MB"], p["NS"], p["D"], p.get("KS", 1)
    mbe = max(1, mb)
    G, S = K // 128, K // (128 * ks)
    stg = 4 * mb * 1024 if mb else -(-S // PHASE_WAVES) * 256  # M = 1: every phase's slice
    kib = lambda b: -(-b // 1024) * 1024  # noqa: E731
    meta = ((kib(ns * 16 * 4 * S) * 2 if ks > 1 else kib(ns * 16 * G) + kib(ns * 32 * G))
            if fmt == 2 else kib(ns * 32))
    return (PHASE_WAVES * d * 2048 + max(PHASE_WAVES * stg, 2 * PHASE_WAVES * mbe * 1024)
            + (0 if ks > 1 else kib(mbe * 16 * ns * 16 * 2)) + meta)


def phase_fits(p, M, N, K, fmt):
    """k_stream_phase's fit -- phase_layout of launch.h (pointer alignment aside): one workgroup
    per CU over N / 256 rows (a multiple of 4; NS slabs of 16, the last 4 .. 16), K / 8 k per
    wave in steps of 128, a ring no deeper than a phase where activations ride it (M > 1), and
    the LDS."""
    mb, ks = p["MB"], p.get("KS", 1)
    if M > 16 * max(1, mb) or (mb == 0 and M != 1):
        return False
    groups = LINE_CUS // ks  # KS > 1: k slices across the workgroups (phase_ks_layout)
    if N % groups or K % (ks * LINE_K_STEP) or K // (ks * LINE_K_STEP) < PHASE_WAVES:
        return False
    if ks == 1 and K % (PHASE_WAVES * LINE_K_STEP):
        return False
    rwg = N // groups
    if rwg % 4 or -(-rwg // 16) != p["NS"] or (mb > 0 and p["NS"] < p["D"]):
        return False
    return phase_lds(p, K, fmt) <= LINE_LDS


def fill_fits(M, N, BM, BN, cus=LINE_CUS):
    """A FILL row: its BM x BN grid is one round of the part and holds more tiles than the grid
    of 256 x BN tiles would -- ilv8_fill_fits of launch.h."""
    nm = -(-M // BM)
    return nm * (N // BN) <= cus and nm > -(-M // 256)


def ilv_ld_max(p):
    """Largest leading dimension the interleaved int8 kernel takes: its copies address a 256-row
    panel with 31-bit byte offsets (A rows are fp16)."""
    return (2 ** 31 - 1) // (2 * max(p["BM"], p["BN"]))


def _fits(kind, p, M, N, K, fmt=1):
    if kind == "ilv8":  # a scale group of 128 k is two k-tiles; NMAX / KMIN / KMAX (optional)
        return (N % p["BN"] == 0 and K % 128 == 0 and K <= ilv_ld_max(p)
                and N < p.get("NMAX", 1 << 30) and K >= p.get("KMIN", 0)
                and K < p.get("KMAX", 1 << 30)
                and (p.get("TAIL") != 2 or tail_split(M, N, p["BM"], p["BN"]) > 0)
                and (not p.get("FILL") or fill_fits(M, N, p["BM"], p["BN"])))
    if kind == "line" and p.get("TL"):  # tail grid: whole slabs, one k chunk
        return (N % (STREAM_N_ROWS * p["R"]) == 0 and K % LINE_K_STEP == 0
                and line_tail_fits(p, N, K, fmt))
    if kind == "phase":  # NMAX / KMIN / KMAX (optional): narrower N / longer / shorter K only
        return (phase_fits(p, M, N, K, fmt) and N < p.get("NMAX", 1 << 30)
                and K >= p.get("KMIN", 0) and K < p.get("KMAX", 1 << 30))
    if kind == "line" and p.get("MT"):  # row tiles: whole slabs, whole k per workgroup
        return (N % (STREAM_N_ROWS * p["R"]) == 0 and K % LINE_K_STEP == 0 and K <= LINE_K_MAX
                and N < p.get("NMAX", 1 << 30) and line_mt_fits(p, K, fmt))
    if kind == "line":  # NMAX / KMIN (optional): the row holds narrower N / longer K only
        return (N % (STREAM_N_ROWS * p["R"] * p.get("SN", 1)) == 0 and K % LINE_K_STEP == 0
                and K <= LINE_K_MAX and N < p.get("NMAX", 1 << 30) and K >= p.get("KMIN", 0))
    if kind == "stream":
        return N % (STREAM_N_ROWS * p["R"]) == 0 and K % (STREAM_K_STEP * p["U"]) == 0
    if kind == "shared":
        return (N % (STREAM_N_ROWS * p["R"] * p["SN"]) == 0
                and K % (STREAM_K_STEP * p["U"]) == 0)
    # mfma: NMAX (optional) as for the line rows
    return N % p["BN"] == 0 and K % p["BK"] == 0 and N < p.get("NMAX", 1 << 30)


def select(op, M, N, K, fmt=1, group=128, dtype_a="fp16", dtype_c="fp16", arch=ARCH):
    if op != "gemm_w8a16" or arch != ARCH:
        return None
    if (dtype_a, dtype_c) != ("fp16", "fp16") or fmt not in FORMATS:
        return None
    if M <= 0 or N <= 0 or K <= 0 or N % 8 or K % 8:
        return None
    if fmt == 2 and (group != 128 or K % group):
        return None
    return _first(LADDER, M, N, K, fmt)


def _first(ladder, M, N, K, fmt, fits=_fits):
    for m_max, n_min, tag, kind, p in ladder:
        if fmt not in p.get("fmts", FORMATS):
            continue
        if M <= m_max and N >= n_min and fits(kind, p, M, N, K, fmt):
            q = {k: v for k, v in p.items() if k != "fmts"}
            return dict(tag=tag, kind=kind, fmt=fmt, **q)
    return None


def select_gate_up(op, M, N, K, fmt=1, group=128, dtype_a="fp16", dtype_c="fp16", arch=ARCH):
    """The fused gate/up row for output width N (the weights have 2N rows), or None."""
    if op != "gemm_w8a16_gate_up" or arch != ARCH:
        return None
    if (dtype_a, dtype_c) != ("fp16", "fp16") or fmt not in FORMATS:
        return None
    if M <= 0 or N <= 0 or K <= 0 or N % 8 or K % 8:
        return None
    if fmt == 2 and (group != 128 or K % group):
        return None
    return _first(LADDER_GATE_UP, M, N, K, fmt, _fits_gate_up)
