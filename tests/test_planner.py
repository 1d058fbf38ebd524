"""CPU checks of the GEMM planner (gemm_plan through the volta_hip_gemm_plan
hook, which makes no device call): the tile family, K split and K groups it
picks for the benchmark configurations' products on a 256-CU MI355X, and the
environment knobs that change them."""
import ctypes as C
import os

import pytest

from volta_amd import HIP_LIB, load_hip

pytestmark = pytest.mark.skipif(not os.path.exists(HIP_LIB), reason="libvolta_hip.so not built")

NN, NT, TN = 0, 1, 2
TILE_64, TILE_128, TILE_SMALLM, TILE_DW_SMALLK, TILE_BIG, TILE_BIG128, TILE_NARROW_TN = 0, 1, 3, 4, 5, 6, 7
CUS = 256


def plan(layout, M, N, K, vec=True, small_m=True, env=None):
    """(tile, splits, k_per_split, kgroups, waves) with `env` set meanwhile."""
    env = env or {}
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        out = (C.c_int32 * 6)()
        lib = load_hip()
        assert lib.lib.volta_hip_gemm_plan(layout, M, N, K, int(vec), CUS, int(small_m), out) == 0
        return tuple(out[:5])
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def test_big_tile_for_full_grids_of_256_multiples():
    """C5's 4096-wide products: 256x256 tiles, one per CU, whole K."""
    assert plan(NN, 4096, 4096, 4096) == (TILE_BIG, 1, 4096, 1, 0)
    assert plan(NT, 4096, 4096, 1024)[:2] == (TILE_BIG, 1)
    assert plan(NN, 4096, 4096, 4096, env={"VOLTA_BIG_TILE": "0"})[0] == TILE_128


def test_big128_tile_for_full_grids_of_128_multiples():
    """C5's 4096x1024 and 1024x4096 products (256 tiles of 128x128, 64 of
    256x256): the 128x128 direct-to-LDS tile, one per CU, whole K; not for
    a K that is below 1024 or no multiple of 128, a grid of fewer tiles
    than CUs, or with VOLTA_BIG128=0."""
    assert plan(NN, 4096, 1024, 4096) == (TILE_BIG128, 1, 4096, 1, 0)
    assert plan(TN, 1024, 4096, 4096) == (TILE_BIG128, 1, 4096, 1, 0)
    assert plan(TN, 4096, 1024, 4096)[:2] == (TILE_BIG128, 1)
    assert plan(NT, 4096, 1024, 1024)[:2] == (TILE_BIG128, 1)
    assert plan(NN, 4096, 1024, 4160)[0] == TILE_128  # K % 128 != 0
    assert plan(NN, 4096, 1024, 512)[0] == TILE_128  # K < 1024
    assert plan(NN, 2048, 1024, 4096)[0] != TILE_BIG128  # 128 tiles
    assert plan(NN, 4096, 1024, 4096, vec=False)[0] != TILE_BIG128
    assert plan(NN, 4096, 4096, 4096)[0] == TILE_BIG  # the 256x256 grid has a tile per CU


def test_128_tiles_from_a_tile_per_cu():
    """Without the direct-to-LDS tile (VOLTA_BIG128=0), 128x128 tiles where
    their grid has a tile per CU (M*N >= 4M outputs, K > 256), split in two
    to two workgroups per CU: C5's 4096x1024 products.  Below that (C4
    B=1024's 1024x1024 products) 64x64 tiles."""
    off = {"VOLTA_BIG128": "0"}
    assert plan(NN, 4096, 1024, 4096, env=off) == (TILE_128, 2, 2048, 1, 0)
    assert plan(TN, 1024, 4096, 4096, env=off)[:2] == (TILE_128, 2)
    assert plan(NN, 1024, 1024, 1024)[0] == TILE_64
    assert plan(NN, 4096, 1024, 256)[0] == TILE_64  # short K
    # the knob restores 128x128 tiles from 2^20 outputs: 64 tiles, split 8 ways
    assert plan(NN, 1024, 1024, 1024, env={"VOLTA_TILE128_MIN_MN": str(1 << 20)})[:4] == (TILE_128, 8, 128, 1)


def test_k_groups_for_full_64_grids_split_in_two():
    """A forward product, or a dX with K >= 1024, on 64x64 tiles split in two
    with a tile per CU runs both slices in one workgroup (kgroups 2, no
    split launches); dW products, short-K dX products and grids of fewer
    tiles than CUs keep the split launches; VOLTA_KGROUPS=0 / 1 turn K
    groups off / on wherever they apply."""
    assert plan(NN, 1024, 1024, 1024) == (TILE_64, 1, 512, 2, 0)
    assert plan(NN, 1024, 1024, 512) == (TILE_64, 1, 256, 2, 0)
    assert plan(NT, 1024, 1024, 1024) == (TILE_64, 1, 512, 2, 0)
    assert plan(NT, 1024, 1024, 512)[:4] == (TILE_64, 2, 256, 1)
    assert plan(TN, 1024, 1024, 1024)[:4] == (TILE_64, 2, 512, 1)
    assert plan(NN, 1024, 512, 1024)[:4] == (TILE_64, 4, 256, 1)  # 128 tiles
    assert plan(NN, 1024, 1024, 1024, env={"VOLTA_KGROUPS": "0"})[:4] == (TILE_64, 2, 512, 1)
    assert plan(NN, 1024, 512, 1024, env={"VOLTA_KGROUPS": "1"})[:4] == (TILE_64, 1, 256, 4)
    assert plan(TN, 1024, 1024, 1024, env={"VOLTA_KGROUPS": "1"})[:4] == (TILE_64, 1, 512, 2)
    # never for the loss-head product (small_m false)
    assert plan(NN, 1024, 1024, 1024, small_m=False)[:4] == (TILE_64, 2, 512, 1)


def test_small_batch_tiles():
    """B <= 256: forward and dX products on the small-M tile (16 waves for
    grids up to one workgroup per CU, dX planned at 4), a dX with K >= 1024
    and M*K >= 2^17 on split-K 64x64 tiles (C3's dX_1), dW on the small-K
    tile."""
    assert plan(NN, 64, 1024, 1024)[:2] == (TILE_SMALLM, 1)
    assert plan(NN, 64, 1024, 1024)[4] == 16
    assert plan(NN, 256, 1024, 512)[4] == 4  # 512 workgroups
    assert plan(NT, 64, 1024, 1024)[:2] == (TILE_SMALLM, 1)  # M*K = 2^16
    assert plan(NT, 64, 2048, 2048)[0] == TILE_64  # M*K = 2^17
    assert plan(NT, 64, 2048, 2048, env={"VOLTA_NT_SPLIT_MIN": "0"})[0] == TILE_SMALLM
    assert plan(TN, 512, 1024, 64)[:2] == (TILE_DW_SMALLK, 1)
    assert plan(TN, 512, 1024, 64, env={"VOLTA_DW_SMALLK_MAX_K": "0"})[0] == TILE_64


def test_planner_rejects_bad_arguments():
    out = (C.c_int32 * 6)()
    lib = load_hip()
    assert lib.lib.volta_hip_gemm_plan(7, 64, 64, 64, 1, CUS, 1, out) == -1
    assert lib.lib.volta_hip_gemm_plan(NN, 0, 64, 64, 1, CUS, 1, out) == -1
    assert "volta_hip_gemm_plan" in lib.last_error()


def test_narrow_tn_for_long_k():
    """The output layer's dW at a large batch (N <= 16, K > 256): 64 rows of
    the product per workgroup over K slices of at most 128, halved down to
    32 until the grid has two workgroups per CU: C5's dW_3 (1024 x 10 x 4096)
    in 32 slices of 128, C4 B=1024's dW_4 (256 x 1 x 1024) in 32 of 32; a
    short K keeps the other tiles, and VOLTA_NARROW_TN=0 the 64x64 ones."""
    assert plan(TN, 1024, 10, 4096) == (TILE_NARROW_TN, 32, 128, 1, 0)
    assert plan(TN, 256, 1, 1024) == (TILE_NARROW_TN, 32, 32, 1, 0)
    assert plan(TN, 64, 1, 256)[0] == TILE_64
    assert plan(TN, 1024, 10, 4096, env={"VOLTA_NARROW_TN": "0"})[0] == TILE_64
    assert plan(TN, 1024, 17, 4096)[0] != TILE_NARROW_TN


def test_split_k_smallest_slice():
    """K slices of at least 128 k, except for forward products of at most 256
    rows (64: a split plan is what sends them to the small-M tile): C4
    B=1024's fwd3 (1024 x 256, K = 512) splits in four, not eight;
    VOLTA_SPLITK_MIN_K=64 restores eight; a 19-row forward product with
    K = 130 still takes the small-M tile."""
    assert plan(NN, 1024, 256, 512)[:3] == (TILE_64, 4, 128)
    assert plan(NN, 1024, 256, 512, env={"VOLTA_SPLITK_MIN_K": "64"})[:3] == (TILE_64, 8, 64)
    assert plan(NN, 19, 66, 130)[0] == TILE_SMALLM
