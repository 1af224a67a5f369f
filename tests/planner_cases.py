"""One shape per rule of the kernel planners, with the plan each should get.

Used by test_planner.py (the plan, on the CPU, for a 256-CU part) and by
test_gpu_parity.py (numerics of the same shapes on the GPU).  Each row is
(M, N, K, configuration name, tile_m, tile_n, K splits); the names are those
rf_w8a16_plan reports.
"""

# GEMV (forced), M <= 64.  tile_m = 16 x m-tiles per wavefront, tile_n = 16 x strips.
GEMV_POLICY = [
    # M<=2, >=640 strips: x staged in LDS by DMA
    (2, 10240, 512, "gemv 1x1 strips, 8 waves, x in LDS", 16, 16, 1),
    # same rule, x does not fit in LDS: plain 4-wave config
    (2, 10240, 16448, "gemv 1x1 strips, 4 waves", 16, 16, 1),
    # M 3..4, >=640 strips: two strips per 8-wave workgroup
    (3, 16384, 512, "gemv 1x2 strips, 8 waves", 16, 32, 1),
    (4, 10240, 8256, "gemv 1x2 strips, 8 waves", 16, 32, 1),  # the same at long K
    # M<=4, 257..639 strips, K <= 1024: two strips per 16-wave workgroup
    (1, 5000, 320, "gemv 1x2 strips, 16 waves", 16, 32, 1),
    # M<=4, 257..639 strips from K 1088 (int8): two strips per 8-wave workgroup
    (1, 8192, 5120, "gemv 1x2 strips, 8 waves", 16, 32, 1),
    (3, 6144, 2560, "gemv 1x2 strips, 8 waves", 16, 32, 1),
    (1, 5120, 16384, "gemv 1x2 strips, 8 waves", 16, 32, 1),   # very long K: no split
    # ... except M<=2 at K 8192..16383: x in LDS
    (1, 5120, 8192, "gemv 1x1 strips, 8 waves, x in LDS", 16, 16, 1),
    # M<=4, < 257 strips (int8): x in LDS, 8 wavefronts, at M 1..2
    (1, 512, 8192, "gemv 1x1 strips, 8 waves, x in LDS", 16, 16, 1),
    (2, 4096, 12288, "gemv 1x1 strips, 8 waves, x in LDS", 16, 16, 1),
    (1, 512, 2048, "gemv 1x1 strips, 8 waves, x in LDS", 16, 16, 1),
    # same, x copy ends mid-way through a 1 KB DMA chunk
    (1, 300, 3136, "gemv 1x1 strips, 8 waves, x in LDS", 16, 16, 1),
    # same, K % 64 != 0: x staged through registers, zero past K
    (1, 520, 3080, "gemv 1x1 strips, 8 waves, x in LDS", 16, 16, 1),
    # at M 3 below 256 strips and M 4 up to 128
    (3, 512, 8192, "gemv 1x1 strips, 8 waves, x in LDS", 16, 16, 1),
    (4, 2048, 6144, "gemv 1x1 strips, 8 waves, x in LDS", 16, 16, 1),
    # with a 2-way K split where only that fits in LDS (up to 128 strips)
    (3, 2048, 11008, "gemv 1x1 strips, 8 waves, x in LDS", 16, 16, 2),
    (4, 2000, 10000, "gemv 1x1 strips, 8 waves, x in LDS", 16, 16, 2),  # ragged N and K
    # M 3..4 otherwise: 16 wavefronts (long K included)
    (4, 2560, 4096, "gemv 1x1 strips, 16 waves", 16, 16, 1),
    (4, 4096, 12288, "gemv 1x1 strips, 16 waves", 16, 16, 1),
    (3, 4096, 2048, "gemv 1x1 strips, 16 waves", 16, 16, 1),
    # M 2..4 from K 16384 without room for x: two strips, about one workgroup per CU
    (2, 3584, 18944, "gemv 1x2 strips, 8 waves", 16, 32, 2),
    (4, 2048, 16384, "gemv 1x2 strips, 8 waves", 16, 32, 4),
    # M=1, K 4096..5119 on <= 64 strips: x in LDS, 16 wavefronts
    (1, 512, 4096, "gemv 1x1 strips, 16 waves, x in LDS", 16, 16, 1),
    # same, x copy ends mid-way through a 1 KB DMA chunk
    (1, 300, 4160, "gemv 1x1 strips, 16 waves, x in LDS", 16, 16, 1),
    # same, K % 64 != 0: x staged through registers, zero past K
    (1, 520, 4104, "gemv 1x1 strips, 16 waves, x in LDS", 16, 16, 1),
    # M<=4, K <= 1024: four wavefronts of four tiles
    (1, 3072, 1024, "gemv 1x1 strips, 4 waves", 16, 16, 1),
    (4, 512, 1000, "gemv 1x1 strips, 4 waves", 16, 16, 1),   # ragged K (16 blocks)
    # M=1, 80..127 K blocks: x in LDS, 8 wavefronts
    (1, 1024, 5120, "gemv 1x1 strips, 8 waves, x in LDS", 16, 16, 1),
    # M 9..16, >=2048 strips, K < 3072
    (12, 32768, 128, "gemv 1x4 strips, 4 waves", 16, 64, 1),
    # the same from K 3072 (int8): five strips per 8-wave workgroup
    (12, 32768, 3072, "gemv 1x5 strips, 8 waves", 16, 80, 1),
    # M 5..8, >=2048 strips from K 1088 (int8): three or five strips, the
    # fuller rounds of workgroups (2368 strips: five)
    (6, 37888, 1088, "gemv 1x5 strips, 8 waves", 16, 80, 1),
    (8, 34816, 1152, "gemv 1x3 strips, 8 waves", 16, 48, 1),     # 2176 strips: three
    # M 5..8, >=2048 strips: three strips per 8-wave workgroup
    (8, 32768, 128, "gemv 1x3 strips, 8 waves", 16, 48, 1),
    (5, 40016, 136, "gemv 1x3 strips, 8 waves", 16, 48, 1),    # ragged N (2501 strips), K tail
    # M 5..16, 1025..1792 strips (5 or 7 per CU): one workgroup per CU
    (16, 20480, 256, "gemv 1x5 strips, 8 waves", 16, 80, 1),
    (16, 28672, 128, "gemv 1x7 strips, 8 waves", 16, 112, 1),
    (9, 26000, 320, "gemv 1x7 strips, 8 waves", 16, 112, 1),    # 1625 strips
    # 6 per CU: three strips, two workgroups per CU
    (12, 24576, 512, "gemv 1x3 strips, 8 waves", 16, 48, 1),
    (16, 24576, 512, "gemv 1x3 strips, 8 waves", 16, 48, 1),
    (13, 24000, 200, "gemv 1x3 strips, 8 waves", 16, 48, 1),   # ragged N (1500 strips), K tail
    # M 3..4 at 1536 strips keeps two strips per workgroup
    (4, 24576, 256, "gemv 1x2 strips, 8 waves", 16, 32, 1),
    # M 5..16, >=1024 strips: two strips per 8-wave workgroup
    (16, 16384, 256, "gemv 1x2 strips, 8 waves", 16, 32, 1),
    # M 5..16, 769..1023 strips: 4 strips per workgroup
    (12, 14336, 256, "gemv 1x4 strips, 8 waves", 16, 64, 1),
    # M 5..16, 513..768 strips: three strips per workgroup
    (12, 10240, 256, "gemv 1x3 strips, 8 waves", 16, 48, 1),
    (16, 12288, 4096, "gemv 1x3 strips, 8 waves", 16, 48, 1),
    # M 5..16, 257..511 strips: two strips per 16-wave workgroup
    (10, 5000, 512, "gemv 1x2 strips, 16 waves", 16, 32, 1),
    # the same from K 5120: two strips per 8-wave workgroup
    (16, 5120, 5120, "gemv 1x2 strips, 8 waves", 16, 32, 1),
    # M 7..16, K 8192..16383, 129..256 strips: two strips per workgroup, 2-way K split
    (16, 4096, 12288, "gemv 1x2 strips, 8 waves", 16, 32, 2),
    (7, 2056, 8200, "gemv 1x2 strips, 8 waves", 16, 32, 2),     # ragged N and K
    # M 5..6 (int8): one strip per 16-wave workgroup, no split
    (5, 2056, 8200, "gemv 1x1 strips, 16 waves", 16, 16, 1),
    # from M 8 on <= 192 strips (int8): three strips split 4-way
    (8, 2560, 9728, "gemv 1x3 strips, 8 waves", 16, 48, 4),
    # M 5..16, K 8192..16383, up to 128 strips (int8): two strips, 4-way K split
    (16, 1024, 8192, "gemv 1x2 strips, 8 waves", 16, 32, 4),
    (8, 1536, 11008, "gemv 1x2 strips, 8 waves", 16, 32, 4),
    # ... up to M 6 (M 8 below K 10240): one strip per 8-wave workgroup, 2-way split
    (5, 2048, 11008, "gemv 1x1 strips, 8 waves", 16, 16, 2),
    (8, 2048, 8192, "gemv 1x1 strips, 8 waves", 16, 16, 2),
    # 257..511 strips at K 8192..16383 from M 8 (int8): three strips split
    # 2-way; five split 4-way from K 10240 and M 12 where one round holds them
    (16, 5120, 8192, "gemv 1x3 strips, 8 waves", 16, 48, 2),
    (8, 5120, 10240, "gemv 1x3 strips, 8 waves", 16, 48, 2),
    (12, 5120, 10240, "gemv 1x5 strips, 8 waves", 16, 80, 4),
    (12, 6144, 10240, "gemv 1x3 strips, 8 waves", 16, 48, 2),
    # M 13..16 on 65..128 strips at K 5120..8191 (int8): two strips per
    # 16-wave workgroup, 4-way split
    (16, 2048, 6144, "gemv 1x2 strips, 16 waves", 16, 32, 4),
    # M 5..16 from K 16384 (int8): 4-way K split with five strips per
    # workgroup on 257..511 strips, four on 129..256, two on fewer
    (16, 4112, 16456, "gemv 1x5 strips, 8 waves", 16, 80, 4),  # ragged N and K
    (8, 3584, 18944, "gemv 1x4 strips, 8 waves", 16, 64, 4),
    (5, 2048, 16384, "gemv 1x2 strips, 8 waves", 16, 32, 4),
    # M 5..16, <=64 strips (int8): one strip per 16-wave workgroup, no split
    (9, 1000, 1024, "gemv 1x1 strips, 16 waves", 16, 16, 1),
    (16, 1024, 2048, "gemv 1x1 strips, 16 waves", 16, 16, 1),
    # at M >= 8 from K 5120: one strip per 8-wave workgroup, 4-way K split
    (12, 1024, 5120, "gemv 1x1 strips, 8 waves", 16, 16, 4),
    # M 5..16, default
    (16, 2048, 1024, "gemv 1x1 strips, 16 waves", 16, 16, 1),
    # M <= 16, 512..639 strips, K >= 16384: 2 strips per workgroup, 8-way split
    (1, 8192, 16384, "gemv 1x2 strips, 8 waves", 16, 32, 8),
    # M 3..4, 257..639 strips, long K: 2 strips per workgroup
    (4, 5120, 8192, "gemv 1x2 strips, 8 waves", 16, 32, 1),
    # M 5..16, 512 strips (two per CU): 2 strips per workgroup
    (12, 8192, 512, "gemv 1x2 strips, 8 waves", 16, 32, 1),
    # M 17..32, >=1024 strips
    (20, 16384, 128, "gemv 2x4 strips, 4 waves", 32, 64, 1),
    # M 17..32, long K on 257..1023 strips: 4-way K split
    (32, 4112, 8192, "gemv 2x4 strips, 4 waves", 32, 64, 4),
    # ... on <= 256 strips (int8): two strips per 16-wave workgroup, 4-way
    # split up to 128 strips, 2-way above
    (32, 640, 8192, "gemv 2x2 strips, 16 waves", 32, 32, 4),
    (24, 2560, 9728, "gemv 2x2 strips, 16 waves", 32, 32, 2),
    # M 17..32, <=128 strips, K 4096..8191 (int8): two strips per 16-wave workgroup, 4-way split
    (24, 1024, 4096, "gemv 2x2 strips, 16 waves", 32, 32, 4),
    (32, 2040, 5128, "gemv 2x2 strips, 16 waves", 32, 32, 4),  # ragged N and K
    # 129..256 strips from K 3072 (int8): the same, 2-way split
    (17, 2064, 4096, "gemv 2x2 strips, 16 waves", 32, 32, 2),
    # below K 3072 (int8): one strip per 8-wave workgroup on 65..256 strips,
    # two per 16-wave workgroup on 257..639
    (24, 2048, 512, "gemv 2x1 strips, 8 waves", 32, 16, 1),
    (24, 2560, 2048, "gemv 2x1 strips, 8 waves", 32, 16, 1),
    (24, 6144, 1024, "gemv 2x2 strips, 16 waves", 32, 32, 1),
    # M 17..32, <=64 strips: 4-way K split; no split up to M 24 and K 2048 (int8)
    (32, 1024, 512, "gemv 2x1 strips, 8 waves", 32, 16, 4),
    (17, 1024, 512, "gemv 2x1 strips, 8 waves", 32, 16, 1),
    # M 17..32, default
    (24, 6144, 4096, "gemv 2x2 strips, 8 waves", 32, 32, 1),
    # M 33..64, >=512 strips
    (40, 8192, 256, "gemv 4x2 strips, 4 waves", 64, 32, 1),
    # M 33..64, default: 2-way K split
    (64, 1000, 640, "gemv 4x2 strips, 8 waves", 64, 32, 2),
]

# GEMV of packed int4 (forced), per-channel and group-wise scales: the rules
# that differ from int8 (K counted in 128-wide int4 tiles).  Rows are
# (M, N, K, group-wise, name, tile_m, tile_n, K splits); packed int4 needs
# N % 16 == 0 and K % 64 == 0.
GEMV_INT4_POLICY = [
    # M <= 4, < 257 strips, <= 8 tiles: four wavefronts per-channel, 16 group-wise
    (1, 3072, 1024, False, "gemv 1x1 strips, 4 waves", 16, 16, 1),
    (2, 3072, 1024, True, "gemv 1x1 strips, 16 waves", 16, 16, 1),
    # 9..16 tiles: x in LDS per-channel at M = 1, else 16 wavefronts
    (1, 2048, 2048, False, "gemv 1x1 strips, 8 waves, x in LDS", 16, 16, 1),
    (2, 2048, 2048, False, "gemv 1x1 strips, 16 waves", 16, 16, 1),
    (1, 2048, 2048, True, "gemv 1x1 strips, 16 waves", 16, 16, 1),
    # 17..63 tiles per-channel: x in LDS, 8 wavefronts, up to M = 4 (63 tiles)
    (4, 1008, 8064, False, "gemv 1x1 strips, 8 waves, x in LDS", 16, 16, 1),
    (1, 1008, 4160, False, "gemv 1x1 strips, 8 waves, x in LDS", 16, 16, 1),  # K % 128 = 64
    # 17..63 tiles group-wise: x in LDS at M = 1, and at M = 2 from 40 tiles
    (1, 1008, 4160, True, "gemv 1x1 strips, 16 waves, x in LDS", 16, 16, 1),
    (2, 1024, 5120, True, "gemv 1x1 strips, 16 waves, x in LDS", 16, 16, 1),
    (2, 1024, 4096, True, "gemv 1x1 strips, 16 waves", 16, 16, 1),
    # 64..127 tiles, M <= 3: x in LDS, 16 wavefronts, where the copy fits
    # (per-channel at M <= 2: 8 wavefronts)
    (2, 4096, 12288, False, "gemv 1x1 strips, 8 waves, x in LDS", 16, 16, 1),
    (3, 4096, 8192, False, "gemv 1x1 strips, 16 waves, x in LDS", 16, 16, 1),
    (2, 1008, 16256, True, "gemv 1x1 strips, 16 waves, x in LDS", 16, 16, 1),
    (3, 4096, 12288, True, "gemv 1x1 strips, 16 waves", 16, 16, 1),
    # M = 4 from 64 tiles: the int8 rule
    (4, 4096, 8192, False, "gemv 1x1 strips, 16 waves", 16, 16, 1),
    # M <= 4, 257..639 strips, >= 64 tiles: x in LDS at M = 1 and at M = 2
    # per-channel where it fits, else two strips per 16-wave workgroup
    (1, 5120, 8192, False, "gemv 1x1 strips, 8 waves, x in LDS", 16, 16, 1),
    (2, 6144, 12288, False, "gemv 1x1 strips, 8 waves, x in LDS", 16, 16, 1),
    (2, 6144, 12288, True, "gemv 1x2 strips, 16 waves", 16, 32, 1),
    # ... from 128 tiles on 257..511 strips: x in LDS split 2-way (4-way from
    # 192 tiles) at M <= 2, two strips per 8-wave workgroup split 4-way at M 3..4
    (2, 5120, 25600, False, "gemv 1x1 strips, 8 waves, x in LDS", 16, 16, 4),
    (1, 5120, 17408, True, "gemv 1x1 strips, 8 waves, x in LDS", 16, 16, 2),
    (4, 5120, 25600, True, "gemv 1x2 strips, 8 waves", 16, 32, 4),
    # M 3..4 on <= 128 strips from 64 tiles: two strips, 4-way split
    (4, 2048, 11008, False, "gemv 1x2 strips, 8 waves", 16, 32, 4),
    # M 3..4 on >= 1024 strips from 16 tiles: two strips per 8-wave workgroup
    (4, 32768, 2048, False, "gemv 1x2 strips, 8 waves", 16, 32, 1),
    # M 8..16 at five strips per CU: three strips per workgroup, six from M 12
    (8, 19456, 2560, False, "gemv 1x3 strips, 8 waves", 16, 48, 1),
    (16, 19456, 2560, True, "gemv 1x6 strips, 8 waves", 16, 96, 1),
    # M 3..4, >= 640 strips: x in LDS (int8 takes two strips per workgroup)
    (4, 12288, 4096, True, "gemv 1x1 strips, 8 waves, x in LDS", 16, 16, 1),
    # M 8..16, >= 2048 strips: four strips per 8-wave workgroup, or three /
    # seven where they fill the rounds of workgroups more than 5% better
    (8, 32768, 4096, False, "gemv 1x4 strips, 8 waves", 16, 64, 1),
    (16, 34816, 1024, True, "gemv 1x3 strips, 8 waves", 16, 48, 1),
    (12, 51200, 1024, False, "gemv 1x7 strips, 8 waves", 16, 112, 1),
    # ... and where none fills them to 85% (2368 strips), or at 1793..2047
    # strips: four strips per 4-wave workgroup; M 5..7 at 1025..1280 strips
    # keeps two
    (16, 37888, 1024, True, "gemv 1x4 strips, 4 waves", 16, 64, 1),
    (8, 31744, 1024, False, "gemv 1x4 strips, 4 waves", 16, 64, 1),
    (5, 20480, 4096, False, "gemv 1x2 strips, 8 waves", 16, 32, 1),
    # M 2..4 on >= 1024 strips from 24 tiles (M 1 below 40): two strips per
    # 8-wave workgroup
    (2, 24576, 4096, False, "gemv 1x2 strips, 8 waves", 16, 32, 1),
    (1, 24576, 4096, True, "gemv 1x2 strips, 8 waves", 16, 32, 1),
    # M 2..4 from 128 tiles below 257 strips: two strips, split to about one
    # workgroup per CU
    (4, 2048, 16384, False, "gemv 1x2 strips, 8 waves", 16, 32, 4),
    (2, 3584, 18944, True, "gemv 1x2 strips, 8 waves", 16, 32, 2),
    # M 8..16 on <= 128 strips from 64 tiles (48 from M 12): two strips,
    # 4-way K split
    (8, 2048, 11008, False, "gemv 1x2 strips, 8 waves", 16, 32, 4),
    (12, 2048, 6144, True, "gemv 1x2 strips, 8 waves", 16, 32, 4),
    # M 12..16 on 129..256 strips from 64 tiles: four strips, 4-way K split
    (16, 2560, 9728, False, "gemv 1x4 strips, 8 waves", 16, 64, 4),
    # M 8..16 on 257..511 strips from 128 tiles: three strips and a 2-way
    # split at M 8, six strips and a 4-way split above
    (8, 5120, 17408, False, "gemv 1x3 strips, 8 waves", 16, 48, 2),
    (16, 5120, 25600, True, "gemv 1x6 strips, 8 waves", 16, 96, 4),
    # M 9..16 on <= 64 strips below 32 tiles: one strip, no split
    (12, 1024, 2048, False, "gemv 1x1 strips, 16 waves", 16, 16, 1),
    # M 17..32 (int4 keeps the GEMV to M 64): four strips per 4-wave
    # workgroup from 640 strips; on 257..639 two per 8-wave workgroup, split
    # 4-way by 4 waves from 128 tiles
    (32, 10240, 5120, False, "gemv 2x4 strips, 4 waves", 32, 64, 1),
    (24, 6144, 4096, True, "gemv 2x2 strips, 8 waves", 32, 32, 1),
    # 65..256 strips: one strip per 8-wave workgroup below 24 tiles, else two
    # strips split 2-way (129..256, below 128 tiles) or 4-way
    (24, 2048, 2048, False, "gemv 2x1 strips, 8 waves", 32, 16, 1),
    (32, 2560, 9728, False, "gemv 2x2 strips, 8 waves", 32, 32, 2),
    (32, 2048, 16384, True, "gemv 2x2 strips, 8 waves", 32, 32, 4),
    (32, 3584, 18944, False, "gemv 2x4 strips, 4 waves", 32, 64, 4),
    # <= 64 strips: no split up to M 24 below 24 tiles, else 4-way
    (24, 1024, 2048, False, "gemv 2x1 strips, 8 waves", 32, 16, 1),
    (32, 1024, 2048, True, "gemv 2x1 strips, 8 waves", 32, 16, 4),
    # M 33..64: from 512 strips four strips per 4-wave workgroup (two per
    # 8-wave workgroup at <= 8 tiles), 2-way split on 512..767 strips from 32 tiles
    (48, 12288, 2048, False, "gemv 4x2 strips, 4 waves", 64, 32, 1),
    (40, 10240, 5120, True, "gemv 4x2 strips, 4 waves", 64, 32, 2),
    (48, 8192, 1024, False, "gemv 4x2 strips, 8 waves", 64, 32, 1),
    # 257..511 strips: no split, or 4-wave and 4-way from 128 tiles
    (48, 4096, 1024, False, "gemv 4x2 strips, 8 waves", 64, 32, 1),
    (48, 5120, 17408, False, "gemv 4x2 strips, 4 waves", 64, 32, 4),
    # below 257 strips: 4-way up to 128 strips, 2-way above (none at <= 8 tiles)
    (64, 1024, 2048, False, "gemv 4x2 strips, 8 waves", 64, 32, 4),
    (48, 4096, 4096, True, "gemv 4x2 strips, 8 waves", 64, 32, 2),
    (33, 2560, 1024, False, "gemv 4x2 strips, 8 waves", 64, 32, 1),
    # M 5..16, 3 / 6 / 7 strips per CU: that many strips per 8-wave
    # workgroup (three at 6 per CU below M 12)
    (5, 12288, 4096, True, "gemv 1x3 strips, 8 waves", 16, 48, 1),
    (16, 10000, 2048, False, "gemv 1x3 strips, 8 waves", 16, 48, 1),   # 625 strips
    (16, 24576, 4096, True, "gemv 1x6 strips, 8 waves", 16, 96, 1),
    (8, 24576, 4096, False, "gemv 1x3 strips, 8 waves", 16, 48, 1),
    (8, 25600, 5120, False, "gemv 1x7 strips, 8 waves", 16, 112, 1),
    (12, 27008, 4224, True, "gemv 1x7 strips, 8 waves", 16, 112, 1),  # 1688 strips, K % 128 = 0
    # M 5..16, 257..511 strips, >= 128 tiles: four strips, 2-way K split
    (5, 5120, 25600, True, "gemv 1x4 strips, 8 waves", 16, 64, 2),
    # the same strips at 64..127 tiles: two strips per 8-wave workgroup from M 8
    (8, 5120, 8192, True, "gemv 1x2 strips, 8 waves", 16, 32, 1),
    (5, 5120, 8192, True, "gemv 1x2 strips, 16 waves", 16, 32, 1),
    # M 5..11, >= 64 tiles on 129..256 strips: two strips per workgroup, 2-way K split
    (8, 4096, 12288, True, "gemv 1x2 strips, 8 waves", 16, 32, 2),
    # M 5..8, <= 64 strips: no K split (int8 splits 4 ways); from M 9 the split
    (8, 1024, 4096, False, "gemv 1x1 strips, 16 waves", 16, 16, 1),
    (12, 1024, 4096, False, "gemv 1x2 strips, 16 waves", 16, 32, 4),
]

# GEMM (forced).
GEMM_POLICY = [
    # M < 128 beyond 128 tile columns of 128: 64x256 tiles
    (100, 16520, 1032, "gemm 64x256 3-stage", 64, 256, 1),
    # M >= 1024, 520 tiles of 128x128 (3 per CU) cost less than 264 of 128x256
    (1024, 8200, 264, "gemm 128x128 B-in-registers", 128, 128, 1),
    # 768 tiles of 128x128 (3 per CU): one round of 384 128x256 tiles; K tail
    (1024, 12288, 200, "gemm 128x256 B-in-registers", 128, 256, 1),
    # M >= 1024, 768 tiles of 128x256 tie with 1536 of 128x128: 128x256; K tail
    (1024, 24576, 136, "gemm 128x256 B-in-registers", 128, 256, 1),
    # M >= 1024, N < 8192: 128x128 tiles, 3 workgroups/CU
    (1100, 1000, 520, "gemm 128x128 B-in-registers", 128, 128, 1),
    # the same with 341 tiles (1..2 per CU): interleaved schedule, ragged M/N/K
    (1300, 3900, 1032, "gemm 128x128 interleaved", 128, 128, 1),
    # M >= 1024, 8 x 64 = 512 tiles of 128x256 (two whole rounds)
    (1024, 16384, 128, "gemm 128x256 B-in-registers", 128, 256, 1),
    # the same rule on ragged M, N, K (9 x 256 = 2304 tiles)
    (1025, 65300, 72, "gemm 128x256 B-in-registers", 128, 256, 1),
    # 128 <= M < 1024: 258 tiles of 128x128 (1..2 per CU): interleaved schedule
    (200, 16400, 136, "gemm 128x128 interleaved", 128, 128, 1),
    # 128 <= M < 1024: 400 tiles of 128x256 tie with 800 of 128x128: 128x256
    (500, 25600, 136, "gemm 128x256 B-in-registers", 128, 256, 1),
    # 128 <= M < 1024, N < 16384: 128x128 tiles, 3 stages (M > 512: no K groups)
    (600, 384, 1024, "gemm 128x128 3-stage", 128, 128, 1),
    # 15 tiles, 64 K blocks: 4-way K split of 16 blocks
    (600, 384, 4096, "gemm 128x128 3-stage", 128, 128, 4),
    # 160 tiles, 17 K blocks: too short to split; K tail
    (640, 4096, 1032, "gemm 128x128 3-stage", 128, 128, 1),
    # 275 tiles (1..2 per CU): interleaved schedule
    (640, 7000, 520, "gemm 128x128 interleaved", 128, 128, 1),
    # 40 tiles, 33 K blocks: 2-way split, K tail in split 1
    (600, 1000, 2056, "gemm 128x128 3-stage", 128, 128, 2),
    # M 128..512, <= 128 tiles of 128x128: two K groups, tile and split by the
    # estimated time (one round, >= 16 K blocks per split)
    (300, 384, 1024, "gemm 64x64 two K groups", 64, 64, 1),      # 30 tiles, 16 K blocks
    (200, 1000, 2056, "gemm 64x64 two K groups", 64, 64, 1),     # ragged M/N, K tail
    (128, 2048, 4096, "gemm 64x64 two K groups", 64, 64, 4),     # 64 tiles, 4-way split
    (512, 4096, 4096, "gemm 64x128 two K groups", 64, 128, 1),   # 256 tiles, one per CU
    (512, 4096, 1032, "gemm 64x128 two K groups", 64, 128, 1),   # 17 K blocks, K tail
    (512, 1024, 5120, "gemm 64x128 two K groups", 64, 128, 4),   # Qwen3-VL-32B k at M = 512
    (256, 4096, 12288, "gemm 128x128 two K groups", 128, 128, 4),
    (384, 2048, 12288, "gemm 128x128 two K groups", 128, 128, 4),  # 48 tiles, 192 workgroups
    # 18 K blocks with a K tail: the tail block falls to the second K group
    (300, 384, 1096, "gemm 64x64 two K groups", 64, 64, 1),
    # 65 K blocks in 4 splits of 17: each split's last stage has one block (the
    # other group reloads it and skips it); K tail in the last split's group 2
    (128, 2048, 4104, "gemm 64x64 two K groups", 64, 64, 4),
    (129, 1040, 3016, "gemm 64x64 two K groups", 64, 64, 2),    # ragged M/N, K tail, 2 splits
    (512, 2056, 2120, "gemm 64x128 two K groups", 64, 128, 1),  # ragged N, 34 K blocks, K tail
    # ... and at 129..256 tiles (one round) with K <= 5120: the 128x128 tile
    # with two K groups, unsplit
    (384, 5504, 4096, "gemm 128x128 two K groups", 128, 128, 1),  # 129 tiles
    (512, 8192, 5120, "gemm 128x128 two K groups", 128, 128, 1),  # Qwen3-VL-32B q at M = 512
    (128, 24576, 4096, "gemm 128x128 two K groups", 128, 128, 1),  # 192 tiles
    (300, 10000, 4104, "gemm 128x128 two K groups", 128, 128, 1),  # ragged M/N, K tail
    # ... but not at K >= 8192 with >= 96 tiles, beyond 128 tiles otherwise,
    # or below 16 K blocks
    (256, 6144, 8192, "gemm 128x128 B-in-registers", 128, 128, 5),
    (136, 8192, 8200, "gemm 128x128 B-in-registers", 128, 128, 4),
    (512, 8256, 5120, "gemm 128x128 interleaved", 128, 128, 1),  # 260 tiles
    (512, 8192, 5184, "gemm 128x128 3-stage", 128, 128, 1),  # 81 K blocks
    (130, 520, 264, "gemm 128x128 3-stage", 128, 128, 1),
    # M < 128, 130 tile columns at K >= 8192: 64x256, 3-way K split
    (100, 16520, 8192, "gemm 64x256 3-stage", 64, 256, 3),
    # M 33..64, <= 64 tiles of 64x64, K >= 4096: 64x64 two K groups, 4 splits
    (48, 1024, 4096, "gemm 64x64 two K groups", 64, 64, 4),
    (33, 1000, 4104, "gemm 64x64 two K groups", 64, 64, 4),  # ragged N and K
    (64, 4096, 8192, "gemm 64x64 two K groups", 64, 64, 4),
    (48, 5120, 4096, "gemm 64x64 4-stage", 64, 64, 8),  # 80 tiles: more than 64
    (64, 2048, 2048, "gemm 64x64 4-stage", 64, 64, 4),  # K < 4096
    # M 65..127 with few tiles: two K groups
    (100, 520, 1032, "gemm 64x64 two K groups", 64, 64, 1),
    (80, 1024, 4096, "gemm 64x64 two K groups", 64, 64, 4),
    (112, 4096, 8192, "gemm 64x128 two K groups", 64, 128, 4),
    (65, 2056, 4104, "gemm 64x128 two K groups", 64, 128, 4),  # one row in the second m-tile
    # M 513..2048, K <= 5120, few tiles and >= 0.75 workgroups per CU: two K groups
    (1024, 1024, 4096, "gemm 64x64 two K groups", 64, 64, 1),
    (1500, 1000, 4104, "gemm 64x128 two K groups", 64, 128, 1),  # ragged M, N and K
    (1024, 512, 4096, "gemm 64x64 two K groups", 64, 64, 2),
    (2048, 1024, 5120, "gemm 64x128 two K groups", 64, 128, 1),
    (640, 1024, 4096, "gemm 128x128 3-stage", 128, 128, 4),  # 160 workgroups: fewer than 0.75 per CU
    (2048, 1024, 5128, "gemm 128x128 B-in-registers", 128, 128, 3),  # K > 5120
    # M >= 1024: 128 tiles of 128x128, 5-way K split (>= 24 blocks each)
    (1024, 2048, 8192, "gemm 128x128 B-in-registers", 128, 128, 5),
    # 160 tiles, 3-way split (two per CU): 128x128 with B in registers; K tail
    (500, 5000, 8200, "gemm 128x128 B-in-registers", 128, 128, 3),
    # 256 tiles (one per CU), K >= 12288, beyond M 2048: 2-way K split
    (4096, 1024, 12288, "gemm 128x128 B-in-registers", 128, 128, 2),
    # M 512..2048, K >= 8192: about one round of 128x256 tiles as two K groups
    # with B in registers, the fewest splits (<= 3, >= 96 K blocks each) that
    # reach 0.75 workgroups per CU
    (2048, 4096, 12288, "gemm 128x256 two K groups, B-in-registers", 128, 256, 1),  # cfg3 down
    (1024, 4096, 12288, "gemm 128x256 two K groups, B-in-registers", 128, 256, 2),
    (512, 5120, 25600, "gemm 128x256 two K groups, B-in-registers", 128, 256, 3),  # VL down
    (1500, 4000, 12296, "gemm 128x256 two K groups, B-in-registers", 128, 256, 1),  # ragged, K tail
    (600, 5000, 24584, "gemm 128x256 two K groups, B-in-registers", 128, 256, 2),  # ragged, K tail
    # ... but not where no split count fits one round, or below 96 K blocks per split
    (1024, 5120, 25600, "gemm 128x128 B-in-registers", 128, 128, 2),  # 160 tiles
    (520, 4096, 12288, "gemm 128x128 3-stage", 128, 128, 3),  # 3 splits of 64 K blocks
    # M <= 32: 32x64 tiles, 4-way K split (16 K blocks each)
    (20, 4096, 4096, "gemm 32x64 3-stage", 32, 64, 4),
    # M <= 32, K >= 192 blocks: 8-way split
    (32, 4096, 12288, "gemm 32x64 3-stage", 32, 64, 8),
    # M <= 32, 200 tiles of 32x128 (>= 192), 100 of 32x256: 32x128, no split
    (32, 25600, 320, "gemm 32x128 4-stage", 32, 128, 1),
    # M <= 32, 193 tiles of 32x256 (>= 192): 32x256, no split; ragged N, K tail
    (24, 49408, 136, "gemm 32x256 3-stage", 32, 256, 1),
    # M <= 32, 33 tiles, 25 K blocks: 2-way split (4 would leave < 8 blocks), K tail in split 1
    (17, 2056, 1544, "gemm 32x64 3-stage", 32, 64, 2),
    # M = 1 forced to the GEMM: 16 tiles of 32x64, 4-way split
    (1, 1024, 4096, "gemm 32x64 3-stage", 32, 64, 4),
    # M 33..64: 64x64 tiles, split to ~3 workgroups per CU
    (48, 5120, 8192, "gemm 64x64 4-stage", 64, 64, 8),     # 80 tiles, 8-way split
    # M 33..64, 100 tiles of 64x256 (>= 96): 64x256 with a 2-way K split
    (40, 25600, 5120, "gemm 64x256 3-stage", 64, 256, 2),
    # M 33..64, 193 tiles of 64x256 (>= 192): 64x256, no split; ragged N, K tail
    (40, 49408, 136, "gemm 64x256 3-stage", 64, 256, 1),
    (64, 1000, 200, "gemm 64x64 4-stage", 64, 64, 1),      # ragged N, 4 K blocks: no split
    (33, 4104, 520, "gemm 64x64 4-stage", 64, 64, 1),      # ragged M and N, K tail (9 K blocks)
]

# Launches of several projections sharing x where the GEMV planner gives a
# workgroup three to seven strips (513..1792 strips at M 5..16, from 2048 at
# M <= 8): (M, N per projection, K, the plan's name on a 256-CU part).  They
# mix ragged projections, so a workgroup's strips run past its projection's
# last strip, and K tails.
STRIP_GROUP_LAUNCHES = [
    (16, [4000, 4000, 1032], 1032, "gemv 1x3 strips, 8 waves"),
    (16, [10000, 10480], 512, "gemv 1x5 strips, 8 waves"),
    (13, [12000, 12008, 264], 256, "gemv 1x3 strips, 8 waves"),
    (9, [12000, 12000], 456, "gemv 1x3 strips, 8 waves"),
    (16, [9000, 9000, 9000], 320, "gemv 1x7 strips, 8 waves"),
    (6, [20000, 20000, 40], 192, "gemv 1x3 strips, 8 waves"),
]


