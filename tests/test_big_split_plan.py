"""A host replay of the FP16 256x256 kernel's K split (gemm_fp16.hip
big_split_plan, f16_dma_gemm.hpp gemm_f16_big_split) over the shapes the tests
run and a sweep of tile counts and K.

For each plan the replay recomputes what every workgroup touches and checks:
every (tile, K tile) pair is computed exactly once; each workgroup's tile, K
range, partial slab and counter lie inside the tile grid, the K tiles, the
scratch the host acquires and the counters; the partial tiles stay within
64 MiB (the allocation-free entry point's array holds them and its counters).
"""
import numpy as np
import pytest

CUS = 256
BM = BN = 256
BK = 64
SLAB = 8 * 8 * 256 * 16  # FM x FN chunks of 16 bytes x 256 threads


def cdiv(a, b):
    return -(-a // b)


def plan(tiles, batch, KT, cus=CUS):
    # gemm_fp16.hip big_split_plan
    if batch != 1 or 2 * tiles > cus or KT < 128:
        return None
    ktps = cdiv(KT, 2)
    return dict(nsplit=cdiv(KT, ktps), ktps=ktps)


def tile_rc(tile, tiles_m, tiles_n):
    # f16_dma_gemm.hpp tile_rc
    GM = 8
    group = tile // (GM * tiles_n)
    first_m = group * GM
    gm = min(tiles_m - first_m, GM)
    in_group = tile - group * GM * tiles_n
    return first_m + in_group % gm, in_group // gm


def replay(M, N, K, cus=CUS):
    tiles_m, tiles_n = cdiv(M, BM), cdiv(N, BN)
    tiles = tiles_m * tiles_n
    KT = K // BK
    if 2 * tiles < cus:
        return None  # below cus / 2 tiles the 256x256 kernel is not chosen
    p = plan(tiles, 1, KT, cus)
    if p is None:
        return None
    part_bytes = tiles * p["nsplit"] * SLAB
    assert part_bytes <= 64 << 20
    assert tiles <= 16384  # counters of a bound workspace
    done = np.zeros((tiles, KT), np.int32)
    for r in range(tiles * p["nsplit"]):
        rtile, split = divmod(r, p["nsplit"])
        assert 0 <= rtile < tiles
        tm, tn = tile_rc(rtile, tiles_m, tiles_n)
        assert 0 <= tm < tiles_m and 0 <= tn < tiles_n
        kbeg = split * p["ktps"]
        kend = min(KT, kbeg + p["ktps"])
        assert 0 <= kbeg < kend <= KT
        slab = (rtile * p["nsplit"] + split) * SLAB
        assert 0 <= slab and slab + SLAB <= part_bytes
        done[tm * tiles_n + tn, kbeg:kend] += 1
    assert np.all(done == 1)
    return p


SHAPES = [(2048, 4096, 8192), (2048, 4096, 11008), (1900, 4000, 8256), (4096, 2048, 11008), (1024, 8192, 16384)]


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_split_plans_cover_every_tile_once(M, N, K):
    assert replay(M, N, K) is not None


def test_plans_of_the_tested_shapes():
    assert replay(2048, 4096, 8192) == dict(nsplit=2, ktps=64)
    assert replay(1900, 4000, 8256) == dict(nsplit=2, ktps=65)
    # more tiles, or K below 8192: no split; the headline shape keeps its one launch
    assert replay(4096, 4096, 4096) is None
    assert replay(2048, 11008, 4096) is None
    assert replay(2048, 4096, 4096) is None


def test_sweep_of_tile_counts():
    for tiles in range(1, 3 * CUS + 1):
        for KT in (1, 16, 64, 127, 128, 129, 172, 256):
            p = plan(tiles, 1, KT)
            if p is None:
                continue
            assert 2 * tiles <= CUS and p["nsplit"] == 2
            assert tiles * p["nsplit"] * SLAB <= 64 << 20
            cover = np.zeros(KT, np.int32)
            for s in range(p["nsplit"]):
                kb = s * p["ktps"]
                cover[kb:min(KT, kb + p["ktps"])] += 1
            assert np.all(cover == 1), (tiles, KT)


def test_replay_catches_a_planted_overlap():
    # a K range one tile too long would compute a K tile twice
    p = plan(128, 1, 129)
    cover = np.zeros(129, np.int32)
    for s in range(p["nsplit"]):
        kb = s * p["ktps"]
        cover[kb:min(129, kb + p["ktps"] + 1)] += 1
    assert not np.all(cover == 1)
