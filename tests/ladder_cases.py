"""GPU parity cases that reach every row of the shipped ladders, named by the row they must take.

One list per ladder (plain and fused gate/up, per weight format).  Each case is
(row tag, M, N, K); for the gate/up ladders N is the output width (the weight has 2N rows).
tests/test_ladder_coverage.py checks on the CPU, with the deliveries' own select.py, that every
case routes to the row it names and that every row of every ladder (per format) is named by some
case; tests/test_gpu_ladder_rows.py runs every case on the GPU against the oracle and checks the
compiled dispatcher's route as well.  Shapes are the BASELINE configs where a config reaches the
row, else the smallest realistic shape that does (K > 65536 is past the line kernel's rows).

The pattern is the reference's dispatch consistency gate
(kernels/shipped/gemm_fp16/sm_70/test_gate.py:102-146) and its ship probe
(kernels/shipped/gemm_fp16/sm_70/ship_probe.cu:41-79), extended to run every row.
"""

FP16 = [
    ("l0r1d2", 1, 3840, 15360),
    ("l0r1d2w", 1, 15360, 3840),
    ("s1a_r1u4", 1, 512, 65792),
    ("l1r1n4d4", 8, 15360, 3840),
    ("l1r1n4d4", 16, 15360, 3840),          # the C2 point M = 16: the row's whole 16-row M tile
    ("l1r1n4d4k8", 16, 3840, 15360),        # 60 workgroups x 8 k slices
    ("l1r1n4d4k8", 8, 3840, 15360),         # the C2 point M = 8, N = 3840
    ("l1r1n4d4k8", 5, 3840, 12288),         # ragged M, 12 steps per slice
    ("l1r1n4d4k8", 16, 3840, 12416),        # 97 steps (prime): no slices (no workspace)
    ("l1r1d4", 16, 3840, 3840),
    ("s16r1u4", 16, 512, 65792),
    ("d32x64k256s3", 24, 15360, 3840),
    ("d32x64k256s3", 32, 12288, 4096),
    ("d32x64k256s3", 17, 12352, 512),       # ragged M, N = 193 x 64, two k-stages
    ("l2r1n4d4", 24, 15360, 3968),          # K % 256 != 0: past the 256-k tiles
    ("l2r1n4d4k8", 32, 3840, 15360),
    ("l2r1n4d4k8", 20, 3840, 12288),
    ("l2r1d4", 32, 3840, 3840),
    ("s32r1u4", 32, 512, 65792),
    ("d64x64k128s3", 64, 15360, 3840),
    ("d64x64k128s3", 40, 12352, 640),
    ("i64x128k64s4w256", 64, 3840, 15360),  # the C2 decode-sweep point M = 64, N = 3840
    ("i64x128k64s4w256", 40, 1920, 4096),   # ragged M, few k-tiles per split
    ("l4r1d3", 64, 6144, 3840),             # N at the interleaved row's NMAX
    ("d128x64k128s3", 128, 15360, 3840),
    ("d128x64k128s3", 100, 12288, 4096),
    ("d128x64k64s4", 128, 15360, 3904),     # K % 128 == 64: past the 128-k tiles
    ("d128x64k64s4", 200, 8192, 3840),
    ("i128x128k64s3w256", 128, 3840, 15360),
    ("i128x128k64s3w256", 100, 3840, 3840),
    ("d64x64k64s4", 128, 8192, 3840),       # N >= 6144: past the split-K row's band
    ("d64x64k64s4", 256, 3904, 3840),       # N % 256 != 0
    ("i128x256k64s3w256", 256, 3840, 15360),
    ("i128x256k64s3w256", 130, 2048, 7680),
    ("l8r1n2d3", 100, 3872, 3840),          # 64 < M <= 128 with N % 64 == 32
    ("d128x128k64s4", 256, 15360, 3840),
    ("i256x256k64w4r8", 512, 4096, 3840),
    ("i256x256k64w4r8", 2049, 3840, 15360),
]

# Strided operands and an 8-byte-aligned C (its rows take the 8-byte store path): (row, M, N, K,
# extra elements per row of A, B, C)
# W8A16 rows on views into wider buffers: (tag, M, N, K, lda - K, ldw - K, ldc - N); ldw keeps
# 16-byte weight rows, ldc = N + 4 leaves C rows 8-byte aligned only
W8_STRIDED = {
    1: [
        ("p1n9d4", 16, 34816, 5120, 8, 16, 4),
        ("p0n2d2", 1, 5120, 5120, 8, 16, 4),
        ("l0r1d2w", 1, 34816, 5120, 8, 16, 4),
        ("i8x128x128w1x4k128s2w256", 128, 7168, 5120, 8, 16, 4),
    ],
    2: [
        ("p0n9d3", 1, 34816, 5120, 8, 16, 4),
        ("p1n9d4", 9, 34816, 5120, 16, 32, 8),
        ("p2n9d4", 32, 34816, 5120, 8, 16, 4),
        ("l2r1n8d2t", 32, 34816, 3840, 8, 16, 4),
    ],
}
W8_GATE_UP_STRIDED = {
    1: [("gp1n9d4", 16, 17408, 5120, 8, 16, 4)],
    2: [("gp0n9d4", 1, 17408, 5120, 8, 16, 4), ("gp2n9d4", 32, 17408, 5120, 8, 16, 4)],
}

FP16_STRIDED = [
    ("l1r1d4", 16, 3840, 3840, 8, 16, 4),
    ("i64x128k64s4w256", 64, 3840, 3840, 8, 8, 4),
    ("i128x128k64s3w256", 128, 3840, 3840, 8, 8, 4),
    ("d64x64k64s4", 128, 8192, 3840, 8, 8, 4),
    ("d128x128k64s4", 256, 15360, 3840, 16, 8, 4),
    ("i256x256k64w4r8", 300, 4096, 3840, 8, 16, 4),
    ("i256x256k64w4r8", 512, 4096, 3840, 64, 64, 64),
]

FP16_GATE_UP = [
    ("gl0r1n2d3", 1, 17408, 5120),
    ("gl1r1n4d3", 16, 17408, 5120),
    ("gl1r1d3", 16, 7680, 3840),
    ("gl2r1n4d3", 32, 17408, 5120),
    ("gl2r1d3", 32, 7680, 3840),
    ("gh1r1u2n2", 1, 512, 65664),
    ("gh16r1u4n2", 16, 512, 65792),
    ("gh32r1u4n4", 32, 512, 65792),
    ("g32r1u4", 32, 496, 65792),
    ("gi128x256k64s3", 64, 17408, 5120),
    ("gi128x256k64s3", 100, 7680, 3840),    # ragged M
    ("gi256x256k64w4r8t", 300, 7680, 3840),
    ("gi256x256k64w4r8t", 512, 4096, 5120),
    ("gi256x256k64w4r8t", 512, 17408, 1024),   # output columns in two parts
]

W8 = {
    1: [
        ("l0r1d2k8", 1, 5120, 17408),     # 320 slabs x 4 k slices
        ("l0r1d2k8", 1, 4096, 16384),     # 256 slabs: no slices (no workspace)
        ("p0n2d2", 1, 5120, 6144),        # 20 rows per CU: a slab of 16 and one of 4
        ("p0n2d2", 1, 6144, 2048),        # 24 rows per CU
        ("l0r1n2d2", 1, 5120, 3840),      # K % 1024 != 0: past the phase-ordered row
        ("l0r1d2", 1, 1024, 5120),
        ("l0r1d2w", 1, 7168, 5120),
        ("l0r1d2w", 1, 34816, 5120),      # the C3/C4 decode point M = 1, N = 34816
        ("p1n9d4", 16, 34816, 5120),      # the C3/C4 decode point M = 16: 136 rows per CU
        ("p1n9d4", 9, 36864, 1024),       # ragged M; 144 rows per CU (a whole last slab), one phase
        ("p1n9d4", 2, 34816, 3072),
        ("l1r1n4d2t", 16, 34816, 3840),   # K % 1024 != 0: past the phase-ordered row
        ("l1r1n4d2t", 16, 16400, 256),    # one remaining slab
        ("l1r1n4d2t", 9, 16384, 384),     # whole rounds, no tail
        ("l1r1n4d3", 16, 15360, 5120),    # too few slabs for a round of the tail grid
        ("l1r1n4d2k8", 16, 5120, 17408),
        ("l1r1n4d2k8", 3, 5120, 12288),   # ragged M
        ("l1r1d2k8", 16, 1024, 5120),
        ("l1r1d2k8", 7, 1024, 1024),      # 8 steps: no slices (no workspace)
        ("l1r1n2d2", 16, 5120, 6144),
        ("l1r1n2d2", 16, 7168, 5120),
        ("l2r1n8d2t", 32, 34816, 5120),
        ("l2r1n8d2t", 17, 32784, 256),    # one remaining slab
        ("l2r1n8d2t", 32, 36864, 128),    # one slab per CU remaining, a single k step
        ("l2r1n4d4", 32, 15360, 5120),
        ("l2r1n8d3k8", 32, 5120, 17408),
        ("l2r1n8d3k8", 25, 5120, 12288),
        ("l2r1d2k8", 32, 1024, 5120),
        ("l2r1n4d2k8", 32, 5120, 6144),
        ("l2r1n4d2k8", 30, 7168, 6144),
        ("l2r1n2d4", 32, 5152, 5120),     # N % 64 == 32
        ("s1a_r1u8", 1, 512, 66048),
        ("s1a_r1u4", 1, 512, 65792),
        ("s8r2u4", 8, 512, 65792),
        ("h16r1u4n2", 16, 512, 65792),
        ("s16r1u4", 16, 2064, 5120),      # N % 32 == 16, past the narrow-N row
        ("h32r1u4n2", 32, 512, 65792),
        ("l4r1n4d3", 64, 34816, 5120),
        ("i8x128x256k128s2w256", 64, 5120, 17408),
        ("i8x128x128w1x4k128s2w256", 64, 5120, 6144),
        ("i8x128x128w1x4k128s2w256", 40, 7168, 5120),
        ("l4r1n2d3", 64, 5152, 5120),     # N % 128 == 32: no 128-column tiles
        ("i8x128x128w1x4k128s2w256", 128, 5120, 17408),
        ("i8x128x256s3w256", 128, 34816, 5120),
        ("i8x128x256s3w256", 128, 15360, 5120),
        ("i8x128x128w1x4k128s2w256", 100, 7168, 5120),
        ("i8x128x128w1x4k128s2w256", 128, 5120, 5120),
        ("i8x128x128w1x4k128s2w256", 100, 2048, 5120),
        ("l2r1d2m4", 128, 1024, 5120),
        ("l2r1d2m4", 100, 1024, 5120),    # last row tile of 4 rows
        ("l2r1d2m4", 72, 1040, 1536),     # 3 row tiles, 65 slab groups (not whole XCD rounds)
        ("l8r1n2d3", 128, 5152, 5120),
        ("m128x128k64", 256, 5120, 5120),
        ("i8x128x128w1x4k128s2w256", 2048, 1024, 5120),
        ("i8x128x128w1x4k128s2w256", 2049, 1024, 5120),
        ("m128x128k64s16", 2048, 1152, 5184),
        ("i8x192x256w1x4k64s3f", 2048, 5120, 1024),   # 11 x 20 tiles, the last tile row 128 rows
        ("i8x192x256w1x4k64s3f", 500, 5120, 640),     # 3 tile rows, the last 116 rows
        ("i8x256w1x4k64s3t", 2048, 7168, 5120),
        ("i8x256w1x4k64s3t", 512, 34816, 1024),   # N in two parts: 256 tiles, then 16 in 128 x 128
        ("i8x256w1x4k64s3t", 500, 34816, 1024),
        ("m256x256k64", 512, 2048, 5184),
    ],
    2: [
        ("p0n2d3", 1, 5120, 17408),       # 17 phases: 3 or 2 per wave
        ("p0n2d3", 1, 6144, 13312),       # 24 rows per CU, 13 phases
        ("l0r1d2k8", 1, 3840, 17408),     # N < 4096: past the whole-K phase row
        ("l0r1d2k8", 1, 4096, 12288),     # K < 13312
        ("p0n2d2", 1, 5120, 5120),
        ("p0n2d2", 1, 6144, 1024),        # 24 rows per CU, one phase
        ("l0r1n2d2", 1, 5120, 3840),
        ("l0r1d2", 1, 1024, 5120),
        ("l0r1d2w", 1, 7168, 5120),
        ("p0n9d3", 1, 34816, 5120),       # the C3/C4 decode point M = 1, N = 34816
        ("p0n9d3", 1, 36864, 1024),       # a whole last slab, one phase
        ("l0r1d2w", 1, 34816, 3840),      # K % 1024 != 0: past the phase-ordered row
        ("p1n9d4", 16, 34816, 5120),      # the C3/C4 decode point M = 16
        ("p1n9d4", 11, 36864, 2048),
        ("l1r1n4d2t", 16, 34816, 3840),
        ("l1r1n4d2t", 16, 16400, 256),    # one remaining slab
        ("l1r1n4d2t", 9, 16384, 384),     # whole rounds, no tail
        ("l1r1n4d3", 16, 15360, 5120),    # too few slabs for a round of the tail grid
        ("p1n10d4k8", 16, 5120, 17408),   # 8 k slices x 32 row groups of 160 rows
        ("p1n10d4k8", 3, 5120, 12288),    # ragged M; 12 steps per slice
        ("l1r1n4d2k8", 16, 5120, 12416),  # K % 1024 != 0: past the phase-ordered row
        ("l1r1d2k8", 16, 1024, 5120),
        ("l1r1d2k8", 7, 1024, 1024),      # 8 steps: no slices (no workspace)
        ("l1r1n2d2", 16, 5120, 6144),
        ("l1r1n2d2", 16, 7168, 5120),
        ("p2n9d4", 32, 34816, 5120),      # the C3/C4 decode point M = 32
        ("p2n9d4", 20, 36864, 3072),
        ("l2r1n8d2t", 32, 34816, 3840),
        ("l2r1n8d2t", 17, 32784, 256),    # one remaining slab
        ("l2r1n8d2t", 32, 36864, 128),    # one slab per CU remaining, a single k step
        ("l2r1n4d4", 32, 15360, 5120),
        ("p2n10d4k8", 32, 5120, 17408),
        ("p2n10d4k8", 25, 5120, 12288),
        ("l2r1n8d2k8", 32, 5120, 12416),
        ("l2r1d2k8", 32, 1024, 5120),
        ("l2r1n4d2k8", 32, 5120, 6144),
        ("l2r1n4d2k8", 30, 7168, 6144),
        ("l2r1n2d4", 32, 5152, 5120),     # N % 64 == 32
        ("s1a_r1u8", 1, 512, 66048),
        ("s1a_r1u4", 1, 512, 65792),
        ("s8r2u4", 8, 512, 65792),
        ("h16r1u4n2", 16, 512, 65792),
        ("s16r1u4", 16, 2064, 5120),      # N % 32 == 16, past the narrow-N row
        ("h32r1u4n2", 32, 512, 65792),
        ("l4r1n4d3", 64, 34816, 5120),
        ("i8x128x256k128s2w256", 64, 5120, 17408),
        ("i8x128x128w1x4k128s2w256", 64, 5120, 6144),
        ("i8x128x128w1x4k128s2w256", 40, 7168, 5120),
        ("l4r1n2d3", 64, 5152, 5120),     # N % 128 == 32: no 128-column tiles
        ("i8x128x256k128s2w256", 128, 5120, 17408),
        ("i8x128x256k128s2w256", 77, 5120, 12288),
        ("i8x128x128w1x4k128s3t2", 128, 34816, 5120),   # one round of 128 x 128, then 16 split
        ("i8x128x128w1x4k128s3t2", 100, 34816, 1024),
        ("i8x128x256s3w256", 128, 15360, 5120),     # 120 tiles of 128 x 128: no whole round
        ("i8x128x128w1x4k128s2w256", 100, 7168, 5120),
        ("i8x128x128w1x4k128s2w256", 128, 5120, 5120),
        ("i8x128x128w1x4k128s2w256", 100, 2048, 5120),
        ("l2r1d2m4", 128, 1024, 5120),
        ("l2r1d2m4", 100, 1024, 5120),    # last row tile of 4 rows
        ("l2r1d2m4", 72, 1040, 1536),     # 3 row tiles, 65 slab groups (not whole XCD rounds)
        ("l8r1n2d3", 128, 5152, 5120),
        ("m128x128k64", 256, 5120, 5120),
        ("i8x128x128w1x4k128s2w256", 2048, 1024, 5120),
        ("i8x128x128w1x4k128s2w256", 2049, 1024, 5120),
        ("i8x128x128w1x4k128s2w256", 2048, 1152, 5120),
        ("i8x192x256w1x4k64s3f", 2048, 5120, 1024),
        ("i8x192x256w1x4k64s3f", 700, 5120, 1024),    # 4 tile rows, the last 124 rows
        ("i8x256w1x4k64s3t", 2048, 7168, 5120),
        ("i8x256w1x4k64s3t", 512, 34816, 1024),   # N in two parts
        ("i8x256w1x4k64s3t", 300, 34816, 1024),
    ],
}

W8_GATE_UP = {
    1: [
        ("gl0r1n2d2", 1, 17408, 5120),
        ("gp1n9d4", 16, 17408, 5120),      # 68 output columns (136 rows) per CU
        ("gp1n9d4", 7, 18432, 1024),       # 72 columns per CU, one phase
        ("gl1r1n4d2t", 16, 17408, 3840),   # tail grid: 2 rounds of paired workgroups, 64 tail pairs
        ("gl1r1n4d2t", 9, 12288, 5120),    # ragged M; whole rounds and a full tail round
        ("gl1r1n4d3", 16, 13312, 5120),    # 320 remaining slabs: past the tail grid
        ("gl1r1n2d4", 8, 7680, 3840),
        ("gl2r1n8d2t", 32, 17408, 5120),
        ("gl2r1n4d2", 32, 12288, 5120),    # fewer slabs than one round of 8-wave workgroups
        ("gl2r1n2d4", 32, 7680, 3840),
        ("g1a_r1u2", 1, 512, 65664),
        ("gh16r1u2n2", 16, 512, 65664),
        ("gh32r1u2n4", 32, 512, 65664),
        ("g32r1u4", 32, 496, 65792),
        ("gi8x128x256k128s2", 64, 17408, 5120),
        ("gi8x128x256k128s2", 100, 7680, 3840),
        ("gi8x256w1x4k64s3t", 300, 7680, 3840),
        ("gi8x256w1x4k64s3t", 512, 17408, 1024),   # output columns in two parts
    ],
    2: [
        ("gp0n9d4", 1, 17408, 5120),
        ("gl0r1n2d2", 1, 17408, 3840),
        ("gp1n9d4", 16, 17408, 5120),
        ("gp1n9d4", 12, 17408, 2048),
        ("gl1r1n4d2t", 16, 17408, 3840),   # tail grid: 2 rounds of paired workgroups, 64 tail pairs
        ("gl1r1n4d2t", 9, 12288, 5120),    # ragged M; whole rounds and a full tail round
        ("gl1r1n4d3", 16, 13312, 5120),    # 320 remaining slabs: past the tail grid
        ("gl1r1n2d4", 8, 7680, 3840),
        ("gp2n9d4", 32, 17408, 5120),
        ("gp2n9d4", 20, 17408, 5120),      # ragged M
        ("gl2r1n8d2t", 32, 17408, 3840),
        ("gl2r1n4d2", 32, 12288, 5120),
        ("gl2r1n2d4", 32, 7680, 3840),
        ("g1a_r1u8", 1, 512, 66048),
        ("g1a_r1u4", 1, 512, 65792),
        ("gh16r1u4n2", 16, 512, 65792),
        ("gh32r1u4n4", 32, 512, 65792),
        ("g32r1u4", 32, 496, 65792),
        ("gi8x128x256k128s2", 64, 17408, 5120),
        ("gi8x128x256k128s2", 100, 7680, 3840),
        ("gi8x256w1x4k64s3t", 300, 7680, 3840),
        ("gi8x256w1x4k64s3t", 512, 17408, 1024),   # output columns in two parts
    ],
}


def case_id(case) -> str:
    tag, M, N, K = case[:4]
    return "%s-m%d-n%d-k%d" % (tag, M, N, K)
