"""Shipped dispatcher for gemm_fp16 on gfx950: (op, M, N, K, dtypes, arch) -> kernel id or None.

None means "caller's own path" (the fallback).  Same contract as the reference's
kernels/shipped/gemm_fp16/sm_70/select.py:23-58; this file is the ONE source of the M-band
ladder -- dispatch.inc is generated from it by gen_dispatch.py and a test checks they agree.

Bands (M is the only runtime-varying extent in serving):
  * M <= 32   stream: the weight-streaming decode kernel (HBM-bound; one pass over B).
  * M >  32   mfma / dma: LDS-tiled MFMA kernels (dma = LDS-DMA copies), tile chosen by M.
"""

ARCH = "gfx950"

# (M_max, tag, kind, template params).  First matching row wins.
LADDER = [
    (16, "s16r1u4", "stream", dict(MB=1, R=1, U=4)),
    (32, "s32r1u4", "stream", dict(MB=2, R=1, U=4)),
    (256, "m128x128k64", "mfma",
     dict(BM=128, BN=128, BK=64, WM=2, WN=2, MS=32, SWZ=1, GROUP=8, XCD=1)),
    (1 << 30, "d256x256k64s2", "dma",
     dict(BM=256, BN=256, BK=64, WM=2, WN=2, STAGES=2, SWZ=2, GROUP=8, XCD=1)),
]

# Divisibility each kind needs (checked at run time by dispatch.inc, mirrored here).
STREAM_K_STEP = 64  # k per pipeline step of the stream kernel
STREAM_N_ROWS = 16  # weight rows per MFMA row group (times R)


def _fits(kind, p, M, N, K):
    if kind == "stream":
        return N % (STREAM_N_ROWS * p["R"]) == 0 and K % (STREAM_K_STEP * p["U"]) == 0
    return N % p["BN"] == 0 and K % p["BK"] == 0


def select(op, M, N, K, dtype_a="fp16", dtype_b="fp16", dtype_c="fp16", arch=ARCH):
    if op != "gemm" or arch != ARCH:
        return None
    if (dtype_a, dtype_b, dtype_c) != ("fp16", "fp16", "fp16"):
        return None
    if M <= 0 or N <= 0 or K <= 0 or N % 8 or K % 8:
        return None
    for m_max, tag, kind, p in LADDER:
        if M <= m_max:
            if not _fits(kind, p, M, N, K):
                return None  # the band's kernel does not cover this shape: fallback
            return dict(tag=tag, kind=kind, **p)
    return None
