"""A host replay of the INT4 int8-MFMA kernel's index math (i4i4_gemm.hpp,
i4i4_gemm.hip) over every plan the tests and the config shapes launch.

For each workgroup, wave, lane and stage the replay recomputes the kernel's
DMA offsets and checks:
  * every weight / zA / sA / Bt / sBf / junk load against its buffer: a lane
    whose voffset is inside the buffer's range reads only bytes of the buffer
    with the soffset added, and a lane past it has voffset at or past the
    range (the bounds check then returns zeros: rows past M);
  * the LDS bytes every DMA writes against its stage region, the regions
    against each other and the LDS size;
  * the ring: the slot a stage is issued into is not the one being read,
    and each wave's vmcnt wait leaves exactly the later stages in flight;
  * the partials (P) store index and the epilogue staging bounds.
Constants are read from the kernel header so the replay follows the source.
"""
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HDR = os.path.join(ROOT, "clove_compute_amd", "csrc", "i4i4_gemm.hpp")
CUS = 256


def _consts():
    src = open(HDR).read()
    names = ["NW", "NT", "BR", "BC", "NB", "LA", "LB", "DA", "DB", "PREP_COLS"]
    c = {}
    for n in names:
        m = re.search(r"\b%s\s*=\s*(\d+)" % n, src)
        assert m, n
        c[n] = int(m.group(1))
    c["ZA_OFF"] = c["BR"] * 128
    c["SA_OFF"] = c["ZA_OFF"] + c["BR"] * 4
    c["AST"] = c["SA_OFF"] + c["BR"] * 4
    c["SB_OFF"] = 2 * c["BC"] * 128
    c["BST"] = c["SB_OFF"] + 2 * c["BC"] * 4
    c["BT0"] = c["LA"] * c["AST"]
    c["JUNK"] = c["BT0"] + c["LB"] * c["BST"]
    c["LDS"] = c["JUNK"] + 1024
    # the header's own derivations must match the ones above
    for expr, key in [(r"ZA_OFF = BR \* 128", "ZA_OFF"), (r"SA_OFF = ZA_OFF \+ BR \* 4", "SA_OFF"),
                      (r"AST = SA_OFF \+ BR \* 4", "AST"), (r"SB_OFF = 2 \* BC \* 128", "SB_OFF"),
                      (r"BST = SB_OFF \+ 2 \* BC \* 4", "BST"), (r"BT0 = LA \* AST", "BT0"),
                      (r"JUNK = BT0 \+ LB \* BST", "JUNK"), (r"LDS = JUNK \+ 1024", "LDS")]:
        assert re.search(expr, src), key
    return c


C = _consts()


def cdiv(a, b):
    return -(-a // b)


def plan_for(M, tiles_n, G, cus=CUS):
    # i4i4_gemm.hip plan_for
    tiles_m = cdiv(M, C["BR"])
    tiles = tiles_m * tiles_n
    ns = 1 if tiles >= cus else cus // tiles
    ns = max(1, min(ns, G // 2))
    gps = 2 * cdiv(cdiv(G, ns), 2)
    return tiles_m, cdiv(G, gps), gps


def swz(r):
    return (r >> 1) & 7


def check_load(name, voff, soff, size, nrec):
    """voff: lane offsets (int64 array), soff: scalar.  In-range lanes read
    inside the buffer with soffset added; the rest are past the range."""
    voff = np.asarray(voff, np.int64)
    inr = voff + size <= nrec
    assert np.all((voff[inr] + soff + size) <= nrec) and np.all(voff[inr] + soff >= 0), \
        f"{name}: an in-range lane reads past the buffer with soffset {soff}"
    assert np.all(voff[~inr] >= nrec), f"{name}: a lane straddles the end of the buffer"
    return inr


def replay(M, N, K, part):
    BR, BC, NB, LA, LB, DA, DB = (C[k] for k in ("BR", "BC", "NB", "LA", "LB", "DA", "DB"))
    G = K // 128
    Npad = cdiv(N, BC) * BC
    tiles_n = Npad // BC
    tiles_m, nsplit, gps = plan_for(M, tiles_n, G)
    KB = K // 2
    n_a, n_za, n_bt, n_sb = M * KB, M * G * 2, G * Npad * 128, G * Npad * 4
    lane = np.arange(64)
    # LDS regions: [weight stages][Bt stages][junk][row-scale slots]
    regions = {"a": (0, C["BT0"]), "b": (C["BT0"], C["JUNK"]), "junk": (C["JUNK"], C["LDS"])}
    assert C["LDS"] <= 160 * 1024
    rows_loaded = {}
    for split in range(nsplit):
        gbeg = split * gps
        gend = min(G, gbeg + gps)
        assert (gend - gbeg) % 2 == 0
        nst = (gend - gbeg) >> 1
        assert nst >= 1
        for tile in range(tiles_m * tiles_n):
            tn, tm = tile % tiles_n, tile // tiles_n
            m0, n0 = tm * BR, tn * BC
            for t in range(nst):
                gs = gbeg + 2 * t
                ast = (t % LA) * C["AST"]
                bst = C["BT0"] + (t % LB) * C["BST"]
                # weight waves 0-3: two 1 KB blocks of 8 rows each, then zA / sA / junk
                for wave in range(4):
                    for i in range(2):
                        r = 8 * (2 * wave + i) + (lane >> 3)
                        chunk = (lane & 7) ^ swz(r)
                        voff = (m0 + r) * KB + 16 * chunk
                        inr = check_load("A", voff, gs * 64, 16, n_a)
                        assert np.array_equal(inr, m0 + r < M)
                        lo = ast + (2 * wave + i) * 1024
                        assert regions["a"][0] <= lo and lo + 1024 <= ast + C["ZA_OFF"]
                        # LDS slot lane & 7 of row r holds global chunk (lane & 7) ^ swz(r)
                        dst = lo + 16 * lane
                        assert np.array_equal(dst, ast + r * 128 + 16 * (lane & 7))
                        for l in np.nonzero(inr)[0]:
                            rows_loaded[(split, tile, t, int(m0 + r[l]), int(chunk[l]))] = True
                    if wave < 2:
                        offm = 2 * ((m0 + lane) * G)
                        inr = check_load("zA" if wave == 0 else "sA", offm, gs * 2, 4, n_za)
                        assert np.array_equal(inr, m0 + lane < M)
                        lo = ast + (C["ZA_OFF"] if wave == 0 else C["SA_OFF"])
                        assert lo + 256 <= ast + C["AST"]
                    else:
                        check_load("junk sA", np.zeros(64, np.int64), 0, 4, n_za)
                        lo = C["JUNK"] + 256 * (wave - 2)
                        assert regions["junk"][0] <= lo and lo + 256 <= regions["junk"][1]
                # Bt waves 4-7: eight 1 KB blocks, then sBf / junk
                for wave in range(4, 8):
                    soff = (gs + ((wave - 4) >> 1)) * Npad * 128
                    for i in range(8):
                        j = 8 * (wave - 4) + i
                        n = 8 * (j & 15) + (lane >> 3)
                        voff = (n0 + n) * 128 + 16 * ((lane & 7) ^ swz(n))
                        inr = check_load("Bt", voff, soff, 16, n_bt)
                        assert inr.all()
                        lo = bst + j * 1024
                        assert lo + 1024 <= bst + C["SB_OFF"]
                        # block j: group j >> 4, columns 8 (j & 15) ..: LDS column n of that group
                        assert lo == bst + (j >> 4) * BC * 128 + 8 * (j & 15) * 128
                    if wave == 4:
                        offm = 4 * ((lane >> 5) * Npad + n0 + 4 * (lane & 31))
                        inr = check_load("sBf", offm, gs * Npad * 4, 16, n_sb)
                        assert inr.all()
                        assert bst + C["SB_OFF"] + 1024 <= bst + C["BST"]
                    else:
                        check_load("junk sBf", np.zeros(64, np.int64), 0, 16, n_sb)
                        assert C["JUNK"] + 1024 <= regions["junk"][1]
            # the ring: at step t the wave waits with min(nst - 1 - t, L - 2)
            # stages of D loads outstanding; exactly the stages after t have
            # been issued past it (prologue L - 1 stages, one per step after its barrier)
            for L, D in ((LA, DA), (LB, DB)):
                for t in range(nst):
                    issued = min(nst, L - 1 + t)
                    assert min(nst - 1 - t, L - 2) == issued - (t + 1)
                    assert (L - 2) * D <= 63
                    # the slot refilled in step t is the one read in step t - 1
                    if t + L - 1 < nst:
                        assert (t + L - 1) % L == (t - 1) % L and (t + L - 1) % L != t % L
        # every valid weight byte of every tile and stage was loaded exactly where expected
    for split in range(nsplit):
        gbeg = split * gps
        nst = (min(G, gbeg + gps) - gbeg) >> 1
        for tile in range(tiles_m * tiles_n):
            m0 = (tile // tiles_n) * BR
            for t in range(nst):
                for r in range(m0, min(M, m0 + BR)):
                    for c in range(8):
                        assert (split, tile, t, r, c) in rows_loaded
    # epilogue staging (fp16 tile, pitch BC + 8 halves) and the set-1 hand-off
    assert BR * (BC + 8) * 2 <= C["BT0"] + C["LB"] * C["BST"]
    assert 4 * 64 * NB * 16 * 4 <= C["BT0"] + C["LB"] * C["BST"]
    # partials store: P[(row * N + col) * G + g] for row < M, col < N, g < G
    if part:
        for split in range(nsplit):
            gbeg = split * gps
            nst = (min(G, gbeg + gps) - gbeg) >> 1
            gmax = gbeg + 2 * (nst - 1) + 1
            assert gmax < G
        rowmax = M - 1
        colmax = N - 1
        assert ((rowmax * N + colmax) * G + (G - 1)) < M * N * G
    return tiles_m, nsplit, gps


HOOK_SHAPES = [(130, 64, 512), (64, 1, 256), (257, 200, 1024), (1000, 128, 11008), (70, 90, 512)]
PRODUCT_SHAPES = [(130, 64, 512), (257, 136, 1024), (1, 64, 256), (192, 128, 512), (4096, 128, 11008),
                  (600, 100, 2816), (1000, 320, 1024), (11008, 128, 4096), (8192, 512, 512),
                  (4096, 128, 11008), (11008, 128, 4096)]


@pytest.mark.parametrize("M,N,K", HOOK_SHAPES)
def test_partials_plan_in_bounds(M, N, K):
    replay(M, N, K, part=True)


@pytest.mark.parametrize("M,N,K", PRODUCT_SHAPES)
def test_product_plan_in_bounds(M, N, K):
    replay(M, N, K, part=False)


def test_failing_case_plan():
    # the case that read weight rows 128-129 as zeros: three 64-row tiles, two
    # splits of one two-group stage each; its index math is in bounds, so the
    # zeros came from the load itself (a stale resource word, test_hazards.py)
    assert replay(130, 64, 512, part=True) == (3, 2, 2)


def test_replay_catches_a_planted_straddle():
    # a lane in range by voffset that reads past the buffer once soffset is added
    with pytest.raises(AssertionError):
        check_load("A", np.array([100]), 16, 16, 120)
    with pytest.raises(AssertionError):
        check_load("A", np.array([110]), 0, 16, 120)
