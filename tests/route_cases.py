"""GPU test shapes whose kernel route is the point of the test, with the route each takes on a
256-CU MI355X.

The GPU tests (test_gpu_norm_fold.py, test_gpu_mlp.py) parametrize over these lists, and
tests/test_plans.py checks every label against the built planners on the CPU, so a planner retune
that moves a case off its route fails there instead of silently dropping the coverage.

Routes of the residual add + RMS norm folded into the projection (qmm4_add_rms_norm_qmm_bf16):
  "fold KS=1"     one row-split launch over whole K, x normalised as it is staged;
  "fold KS=2"     the same with K in 2 slices (each slice stages its own part of the normalised
                  row; the slices' sums meet through the arrival counters);
  "two launches"  the norm kernel, then the projection on its n (more than 4 rows, K above the
                  folded 8192, or a row-split plan that cannot normalise while staging).
Routes of 65-128 rows (qmm4_affine_bf16, dispatch_qmm):
  "row-phase"  the row-phase kernel with 80-128-row x blocks and K split over the CUs: up to 112
               rows, or 128 over at most 2048 columns, when K % 512 == 0 and N leaves the kernel's
               plan narrow; a wide plan (N >= 32768 on 256 CUs, every workgroup its own blocks
               over all of K) up to 96 rows when it needs at most one range per CU;
  "gemm"       the GEMM (stream-K over 128 x 128 tiles at these rows).
Row-phase variants of wide plans (qmm4_affine_bf16 at 17-64 rows over N >= 32768): "opt" is a
variant whose waves without a block in the last slot skip that slot's arithmetic (9 or 17 blocks
per workgroup leave most waves a block short); "full" computes every slot in every wave.
Routes of the gate+up SiLU·mul projection (qmm4_gate_up_silu_bf16):
  "fused"            one row-split launch with the epilogue fused;
  "row-phase fused"  otherwise, from 5 to 96 rows where the projection takes the row-phase kernel
                     (K % 512 == 0; no row-split plan up to 16 rows): its ranges hold the same
                     blocks of the gate and up halves and the epilogue is fused, in the kernel for
                     a wide plan (at most one range per CU past 64 rows; ranges no larger than the
                     projection's, or 17 rows or more with M x K <= 2^19), in the reduce kernel for
                     the projection's own K-split plan;
  "two-pass"         the projection into the library's scratch, then the SiLU·mul pass.
"""

CUS = 256

# (M, N, K, silu_mul, route)
FOLD_CASES = [
    (1, 34816, 5120, True, "fold KS=1"),    # decode gate+up (the decode MLP's first projection)
    (2, 34816, 5120, True, "fold KS=1"),
    (4, 34816, 5120, True, "fold KS=1"),
    (1, 17408, 5120, False, "fold KS=1"),   # plain
    (3, 5120, 5120, False, "fold KS=1"),    # one or two 16-row blocks per CU
    (4, 5120, 512, False, "fold KS=1"),     # one unit per block
    (2, 20480, 640, False, "fold KS=1"),    # units of 5 super-steps
    (2, 12288, 8192, False, "fold KS=1"),   # the largest folded K (4 chunks per thread)
    (1, 94240, 8192, True, "fold KS=2"),    # gate+up: whole-K unit slots exceed LDS
    (1, 176160, 6400, False, "fold KS=2"),  # plain, units of 5 super-steps (no paired form)
    (5, 5120, 5120, False, "two launches"),  # 5 rows: norm kernel + row-split (8-row fragments)
    (4, 5120, 10240, False, "two launches"),  # K > 8192
    (16, 8192, 1024, True, "two launches"),  # 16 rows: norm kernel + fused gate+up (K in 2 slices)
    (24, 34816, 5120, True, "two launches"),   # norm kernel + the fused row-phase gate+up
    (48, 33024, 2048, True, "two launches"),
    (64, 17408, 5120, False, "two launches"),  # norm kernel + row-phase (K split)
]

# (M, K, N, route): gate+up weights [N, K] stacked as [gate; up].
GATE_UP_CASES = [
    (1, 5120, 34816, "fused"),
    (2, 5120, 34816, "fused"),
    (4, 5120, 34816, "fused"),
    (3, 4096, 34848, "fused"),    # 17424 = 242 x 72: a partial last range
    (4, 17408, 10240, "fused"),
    (9, 5120, 34816, "fused"),    # 9-16 rows: 16-row fragments, K in slices
    (12, 5120, 34816, "fused"),
    (16, 5120, 34816, "fused"),
    (16, 5120, 20480, "fused"),
    (1, 512, 256, "fused"),       # one block per workgroup
    (5, 2048, 4096, "fused"),
    (16, 1024, 2048, "fused"),
    (1, 81920, 32, "two-pass"),   # x slices too large for LDS at every K split
    (3, 81920, 256, "two-pass"),
    (16, 20480, 1024, "row-phase fused"),  # the projection's K-split plan, the epilogue in its reduce
    (24, 5120, 34816, "row-phase fused"),   # 218 ranges of 5 + 5 blocks, the twin variant
    (48, 2048, 33024, "row-phase fused"),   # 1032 blocks per half: a partial last range
    (64, 4096, 32768, "row-phase fused"),   # one block per wave
    (80, 5120, 34816, "row-phase fused"),   # 80-row x blocks
    (96, 2048, 34816, "row-phase fused"),
    (17, 2048, 65536, "row-phase fused"),
    (12, 20480, 34816, "two-pass"),  # ranges of 10 blocks against the projection's 9, under 17 rows
    (12, 20480, 32768, "row-phase fused"),  # 5-16 rows with no row-split plan, ranges of 8 in both
    (64, 16384, 34816, "two-pass"),  # ranges of 10 against 9, M x K past 2^19
    (24, 16384, 32768, "row-phase fused"),  # long K, ranges of 8 blocks as the projection's
    (64, 5120, 1024, "row-phase fused"),  # K split over the CUs: the reduce kernel applies the epilogue
    (100, 512, 4096, "two-pass"),  # row-phase underneath (112-row x blocks)
    (136, 512, 4096, "two-pass"),  # GEMM underneath
]

# Seeded random (M, K, N) shapes (M 1-120, N a multiple of 32), reaching all three routes: one row-split
# launch (fused), the row-phase kernel with the epilogue fused (row-phase fused: wide plans, or the
# K-split plans' reduce kernel), and the two passes (K % 512 != 0, past 96 rows).
RANDOM_GATE_UP = [(8, 2560, 33056), (11, 512, 35488), (59, 2048, 35136), (89, 2048, 2272), (29, 512, 33568),
                  (9, 4096, 32768), (29, 2048, 33728), (5, 4608, 3232), (37, 1024, 11040), (64, 2048, 34080),
                  (23, 1024, 2912), (86, 384, 10656), (6, 512, 33504), (29, 1536, 33664), (32, 4096, 33024),
                  (60, 3072, 11712), (77, 512, 35040), (3, 1024, 34272), (7, 1024, 6784), (82, 1024, 33952),
                  (19, 2560, 36512), (34, 2048, 10144), (22, 4096, 36608), (91, 4608, 1728),
                  (40, 640, 8192), (70, 1152, 4096), (100, 2048, 4096), (120, 1024, 8192), (12, 2432, 6144),
                  (27, 4736, 2048)]

# (M, N, K, route)
MID_ROW_CASES = [
    (65, 17408, 5120, "row-phase"),   # up projection, one row past 64 (80-row x blocks)
    (65, 5120, 17408, "row-phase"),   # down projection
    (80, 5120, 17408, "row-phase"),
    (96, 8192, 2048, "row-phase"),    # 96-row blocks
    (112, 5120, 6144, "row-phase"),   # 112-row blocks
    (100, 2064, 1024, "row-phase"),   # one block per wave (few phases per workgroup)
    (128, 1024, 5120, "row-phase"),   # 128-row blocks over a small N
    (113, 5120, 17408, "gemm"),
    (128, 17408, 5120, "gemm"),
    (72, 34816, 5120, "row-phase"),   # a wide plan, 9 blocks per workgroup (the 80-row twin)
    (96, 34816, 5120, "row-phase"),   # the 96-row twin
    (112, 34816, 5120, "gemm"),       # a wide plan past 96 rows
    (72, 65984, 5120, "gemm"),        # a wide plan needing more ranges than CUs
    (96, 1024, 640, "gemm"),          # K % 512 != 0
]

# (M, N, K, variant form)
ROWPHASE_WIDE_CASES = [
    (24, 34816, 5120, "opt"),   # 9 blocks per workgroup, 2 slots per wave (phases of 512 k)
    (33, 32784, 2048, "opt"),   # 64-row x blocks, a partial last range
    (48, 33024, 3072, "opt"),
    (32, 65984, 2048, "opt"),   # 17 blocks, 3 slots per wave
    (64, 65984, 2048, "opt"),   # 64-row x blocks over the drafter's head
    (32, 131072, 2048, "full"),  # 32 blocks: every wave holds 4
]

# Shapes of the row-phase tests in test_gpu_parity.py, each of which dispatch_qmm must send to the
# row-phase kernel (checked in tests/test_plans.py against the built planners, in dispatch order).
# (M, K, N): wide and K-split plans, 9-16 rows where no row-split plan fits (x of 16 rows over
# K = 5120 leaves no LDS for a vocabulary head's unit slots), partial ranges and windows.
ROWPHASE_SHAPES = [(17, 5120, 4096), (33, 2048, 32784), (9, 5120, 65984), (48, 3072, 33024), (64, 1024, 2064),
                   (24, 17408, 1024), (16, 5120, 65984), (32, 2048, 65984), (16, 5120, 99984), (32, 2048, 131072),
                   (24, 5120, 17408), (12, 17408, 5120), (48, 6144, 5120), (32, 2048, 8192)]
# (N, M, K) of the one-hot exact-dequantization test.
ROWPHASE_ONE_HOT = [(32800, 32, 2048), (2064, 48, 2048), (65984, 16, 5120), (131072, 32, 2048), (4096, 80, 2048),
                    (2064, 112, 2048), (1024, 128, 2048), (33024, 48, 2048), (65984, 32, 2048), (65984, 64, 2048),
                    (34816, 72, 2048), (34816, 96, 2048)]
# (M, K, N) of the scale-window form switches.
ROWPHASE_WINDOW_CASES = [(12, 5120, 65552), (48, 3072, 33024), (64, 17408, 5120), (32, 5120, 65552),
                         (96, 17408, 5120)]

# (M, N, K, tiles) of GEMM stream-K launches in test_gpu_parity.py: "128x256" tiles past 128 rows,
# for K >= 8192, or at most 128 rows over enough columns that whole 256 x 256 tiles would otherwise
# run (8-group scale blocks and at least 2 units per CU), else "128x128".
GEMM_STREAM_K_CASES = [
    (128, 17408, 5120, "128x128"),   # the up projection at 128 rows
    (200, 784, 5120, "128x128"),     # too few units for the wide tiles
    (256, 17408, 5120, "128x256"),
    (320, 17408, 5120, "128x256"),   # a partial row tile
    (384, 5120, 17408, "128x256"),   # K >= 8192 at 257-384 rows: a half-empty last row of 256-row tiles
    (320, 5120, 12288, "128x256"),
    (120, 5120, 17408, "128x256"),   # K >= 8192 at 120 rows
    (136, 10256, 5120, "128x256"),   # partial row and column tiles
    (256, 8192, 4096, "128x256"),    # the one-hot exact-dequant case
    (72, 65984, 2048, "128x256"),    # at most 128 rows over many columns: instead of whole tiles
    (96, 65984, 5120, "128x256"),
]
