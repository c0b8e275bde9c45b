"""The prefill GEMM planner (host code of libcujev_ops.so, no GPU needed):
every engine shape gets a tile the kernel is built for and a legal split."""
import pytest

from cujev import ops as o

TILES = {(2, 8), (2, 12), (3, 8), (3, 12), (4, 6), (4, 8), (4, 10), (4, 12), (6, 4), (6, 6),
         (6, 8), (8, 4), (8, 6)}


def test_plan_covers_engine_shapes():
    o.load()
    for N in (1, 97, 530, 1024, 8192):
        for M, K, gated, ms in [(10240, 2560, 0, 1), (12352, 2560, 0, 1), (18432, 2560, 1, 1),
                                (2560, 4096, 0, 8), (2560, 9216, 0, 8), (12288, 4096, 0, 1),
                                (24576, 4096, 1, 1), (4096, 12288, 0, 8)]:
            rg, ng, s = o.gemm_wide_plan(N, M, K, gated, ms)
            assert (rg, ng) in TILES and 1 <= s <= ms and (K // 128) % s == 0
            if gated:
                assert rg % 2 == 0


def test_plan_rejects_unsupported_shapes():
    o.load()
    for N, M, K, gated in [(10, 100, 256, 0), (10, 256, 200, 0), (10, 272, 256, 1), (0, 256, 256, 0)]:
        with pytest.raises(o.OpsError):
            o.gemm_wide_plan(N, M, K, gated)
