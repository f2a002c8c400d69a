"""Host-side choices that must be pure functions of the shape (so a given model and input
give the same bits in every process): the projection path and the lollm_gemm grid."""

from lollm_amd.qwen3_5.blocks import gemm_grid, gemm_path


def test_gemm_path_is_a_function_of_rows():
    assert gemm_path(12352, 4096, 0, 64) == "gemm"
    assert gemm_path(12352, 4096, 0, 16) == "gemm"
    assert gemm_path(12352, 4096, 0, 65) == "blas"          # the prefill
    assert gemm_path(4096, 4096, 0, 64, tiled=False) == "blas"


def test_gemm_grid_whole_groups_only_when_they_fill_the_device():
    # the GDN in_proj of the 4096-hidden model: 193 groups of 64 columns on 256 CUs
    assert gemm_grid(12352, 256) == 193
    # 4 groups per 3 CUs or more, or fewer than 3/4 of the CUs: one workgroup per CU
    for N in (4096, 8192, 24576, 151936):
        assert gemm_grid(N, 256) == 256
    # else one workgroup per 96-column group when those fill 3/4 of the CUs or more
    # (attention q|gate|k|v 18432 = 192 x 96; gate|up 24576 = 256 x 96, one per CU either
    # way), for any number of rows
    for rows in (64, 33, 32, 16, 1):
        assert gemm_grid(18432, 256, rows) == 192
        assert gemm_grid(24576, 256, rows) == 256
    assert gemm_grid(191 * 96, 256, 64) == 256
    assert gemm_grid(192 * 64, 256) == 192
    assert gemm_grid(191 * 64, 256) == 256
    assert gemm_grid(256 * 64, 256) == 256
    assert gemm_grid(257 * 64, 256) == 256
