"""Index-level emulation (CPU) of the backward's workspace and of the split dK/dV partition.

Restates, for the host and the kernels in nanonemo_amd/csrc/flash_attn.hip, only the index arithmetic:
carve() (where -D, -lse/scale and the split partials sit in the workspace), dkdv_split(), the dK/dV kernel's
block -> (split, unit pair) mapping, each split's iteration range [s n / S, (s + 1) n / S) of a unit, the
chunk-owner reduction's part[] stores, and the sum kernel's part[] reads. It proves, per shape:
  * every part element the sum kernel reads is stored by exactly one block of the same split in the dK/dV
    launch (so no element is read before it is written in stream order, and none is written twice);
  * every (query head, query tile) iteration of every unit is taken by exactly one (split, wave);
  * the three workspace regions are disjoint, 256-byte aligned, inside the size the library reports.
The kernels exchange data only through these buffers and only across kernel boundaries (dQ writes -D and
-lse/scale, dK/dV reads them and writes part, the sum kernel reads part); no block reads what another block
of the same launch writes. The shape (B=2, H=12, KVH=1, T=1024, D=64, 16 splits) is the one whose first HIP
graph replay once differed from the eager result.
"""

from __future__ import annotations

import numpy as np
import pytest

from nanonemo_amd.kernels.hip import lib


def round256(n):
    return (n + 255) & ~255


def dkdv_split(B, H, KVH, T):
    nkb = (T + 63) // 64
    base = B * KVH * ((nkb + 1) // 2)
    if base >= 256 or (H // KVH) * nkb * 16 >= 2**31:
        return 1
    return max(1, min(16, -(-256 // base), (H // KVH) * (nkb + 1) // 8))


def carve(B, H, KVH, T, D):
    vec = round256(4 * B * H * T)
    S = dkdv_split(B, H, KVH, T)
    regions = {"nD": (0, 4 * B * H * T), "nL": (vec, vec + 4 * B * H * T)}
    if S > 1:
        regions["part"] = (2 * vec, 2 * vec + S * 2 * 4 * B * KVH * T * D)
    total = 2 * vec + (round256(S * 2 * 4 * B * KVH * T * D) if S > 1 else 0)
    return S, regions, total


def emulate_split(B, H, KVH, T, D):
    """Returns (store count per part element, iteration owner count per (bk, unit, iteration))."""
    S = dkdv_split(B, H, KVH, T)
    nkb = nqt = (T + 63) // 64
    npairs = (nkb + 1) // 2
    BKV, group, WPP, NW = B * KVH, H // KVH, 4, 4  # a split launch always runs 4 waves per pair
    ND = D // 32
    nbk = BKV  # PPB = 1
    nbase = nbk * npairs
    stores = np.zeros((S, 2, BKV, T, D), dtype=np.int32)
    owners = {}
    for block in range(nbk * npairs * S):
        sidx, bid = divmod(block, nbase)
        bgrp, pj = bid % nbk, bid // nbk
        bk = bgrp
        units = [pj] if nkb - 1 - pj == pj else [pj, nkb - 1 - pj]
        for unit in units:
            n = group * (nqt - unit)
            first, end = sidx * n // S, (sidx + 1) * n // S
            for wp in range(WPP):
                for itn in range(first + wp, end, WPP):
                    owners[(bk, unit, itn)] = owners.get((bk, unit, itn), 0) + 1
            kb0 = unit * 64
            for which in range(2):  # dK, then dV: every chunk c (its owner wave c % 4) stores 4 columns per lane
                for c in range(2 * ND * 4):
                    for lane in range(64):
                        l32, hh = lane & 31, lane >> 5
                        key = kb0 + 32 * (c // (4 * ND)) + l32
                        col = 32 * (c // 4 % ND) + 8 * (c % 4) + 4 * hh
                        if key < T:
                            stores[sidx, which, bk, key, col:col + 4] += 1
    return S, stores, owners, nkb, nqt, group, BKV


SHAPES = [(2, 12, 1, 1024, 64), (8, 12, 1, 1024, 64), (1, 12, 4, 1024, 64), (1, 12, 4, 400, 32), (2, 6, 2, 333, 64)]


def iteration(itn, unit, first_unit, group, nqt):
    """Restates the dK/dV kernel's iter_head / iter_tile: iteration itn of unit ``unit`` of a pair whose first unit
    is ``first_unit`` -> (query head of the group, query tile), head-minor; the first unit's tiles descend from the
    last, the second unit's ascend from its own."""
    t = nqt - 1 - itn // group if unit == first_unit else unit + itn // group
    return itn % group, t


@pytest.mark.parametrize("group, nqt", [(3, 16), (1, 16), (12, 16), (3, 128), (4, 7), (2, 1), (3, 15)])
def test_pairs_cover_their_iterations_once_and_walk_the_tiles_in_step(group, nqt):
    nkb = nqt
    for pj in range((nkb + 1) // 2):
        units = [pj] if nkb - 1 - pj == pj else [pj, nkb - 1 - pj]
        walk = []
        for unit in units:
            n = group * (nqt - unit)
            got = [iteration(i, unit, pj, group, nqt) for i in range(n)]
            assert sorted(got) == sorted((h, t) for h in range(group) for t in range(unit, nqt))
            walk += got
        # at the pair's i-th iteration every pair of the (batch, KV head) is on tile nqt - 1 - i // group (first
        # unit) or i // group - 1 (second unit), whichever pair it is
        for i, (h, t) in enumerate(walk):
            assert h == i % group and t == (nqt - 1 - i // group if i < group * (nqt - pj) else i // group - 1)


@pytest.mark.parametrize("shape", SHAPES)
def test_split_partials_are_each_stored_once_and_every_iteration_is_taken_once(shape):
    B, H, KVH, T, D = shape
    S, stores, owners, nkb, nqt, group, BKV = emulate_split(B, H, KVH, T, D)
    assert S > 1, "the shapes here all split"
    # the sum kernel reads part[s][which][bk][key][col] for every s < S, key < T, col < D: each stored exactly once
    assert stores.min() == 1 and stores.max() == 1
    want = {(bk, u, i) for bk in range(BKV) for u in range(nkb) for i in range(group * (nqt - u))}
    assert set(owners) == want and all(v == 1 for v in owners.values())


@pytest.mark.parametrize("shape", SHAPES + [(8, 12, 4, 1024, 64), (32, 12, 4, 1024, 64), (1, 1, 1, 1, 32)])
def test_workspace_regions_are_disjoint_aligned_and_sized_as_the_library_says(shape):
    B, H, KVH, T, D = shape
    S, regions, total = carve(B, H, KVH, T, D)
    assert lib().nn_fa_bwd_workspace_size(B, H, KVH, T, D) == total
    spans = sorted(regions.values())
    for (a0, a1), (b0, b1) in zip(spans, spans[1:]):
        assert a1 <= b0, regions
    assert all(lo % 256 == 0 and hi <= total for lo, hi in spans)


def test_the_replay_shape_splits_sixteen_ways():
    S, regions, total = carve(2, 12, 1, 1024, 64)
    assert S == 16 and set(regions) == {"nD", "nL", "part"}
    assert regions["part"][1] - regions["part"][0] == 16 * 2 * 4 * 2 * 1 * 1024 * 64


# ---- forward / dQ grid: block -> (batch * H + head, query block) ---------------------------------


def qblock_of(bid, BH, group, nqb):
    """Restates qblock_of() of nanonemo_amd/csrc/flash_attn.hip: heaviest query blocks first; when the B*KVH head
    groups divide evenly over the 8 XCDs, every query head of group g goes to XCD g % 8 (block i runs on XCD i % 8)."""
    G = BH // group
    if G % 8 == 0:
        x, slot = bid & 7, bid >> 3
        per = (G >> 3) * group
        qi, r = divmod(slot, per)
        gi, hq = divmod(r, group)
        return (gi * 8 + x) * group + hq, nqb - 1 - qi
    return bid % BH, nqb - 1 - bid // BH


@pytest.mark.parametrize(
    "B, H, KVH, T",
    [(8, 12, 4, 1024), (32, 12, 4, 1024), (2, 12, 4, 8192), (1, 12, 4, 256), (8, 12, 12, 1024), (8, 12, 1, 1024),
     (3, 8, 2, 65), (2, 4, 4, 37), (16, 16, 8, 512), (4, 6, 2, 300), (1, 1, 1, 1), (5, 12, 3, 130)],
)
def test_qblock_of_covers_every_block_once_heaviest_first_per_xcd(B, H, KVH, T):
    BH, group, nqb = B * H, H // KVH, (T + 127) // 128
    seen = {}
    for bid in range(nqb * BH):
        bh, qb = qblock_of(bid, BH, group, nqb)
        assert 0 <= bh < BH and 0 <= qb < nqb
        assert (bh, qb) not in seen, f"block {bid} repeats {(bh, qb)} of block {seen[(bh, qb)]}"
        seen[(bh, qb)] = bid
    assert len(seen) == nqb * BH
    # Dispatch order within each XCD (block i on XCD i % 8): the causal work (qb + 1 key tiles) never grows.
    for x in range(8):
        qbs = [qblock_of(bid, BH, group, nqb)[1] for bid in range(x, nqb * BH, 8)]
        assert all(a >= b for a, b in zip(qbs, qbs[1:])), f"XCD {x}: query blocks {qbs[:12]}..."
    if (BH // group) % 8 == 0:  # every query head of one (batch, KV head) group shares one XCD
        for (bh, _), bid in seen.items():
            assert (bh // group) % 8 == bid % 8


# ---- dK/dV grid: block -> (split, waves' (batch, KV head), unit pair or single unit) -------------------


def dkdv_waves_per_pair(B, H, KVH, T):
    """Restates dkdv_waves_per_pair() of nanonemo_amd/csrc/flash_attn.hip."""
    nkb = (T + 63) // 64
    pairs = B * KVH * ((nkb + 1) // 2)
    if (H // KVH) * (nkb + 1) > 300:
        return 4
    return 1 if pairs >= 3 * 256 else (2 if pairs >= 2 * 256 else 4)


def dkdv_mode(B, H, KVH, T):
    """Restates dkdv_mode(): (paired, waves per pair or unit). Unsplit four-wave problems take single units when
    they fit in one block per CU (four waves each) or in two (two waves each) while a wave's share of the heaviest
    unit stays below a pair wave's share plus a unit change (3 iterations)."""
    wpp = dkdv_waves_per_pair(B, H, KVH, T)
    if dkdv_split(B, H, KVH, T) != 1 or wpp != 4:
        return True, wpp
    nkb = (T + 63) // 64
    units, g = B * KVH * nkb, H // KVH
    if units <= 256:
        return False, 4
    if units <= 512 and (g * nkb + 1) // 2 < (g * (nkb + 1) + 3) // 4 + 3:
        return False, 2
    return True, 4


def dkdv_owners(B, H, KVH, T):
    """Every (batch * KV head, unit, iteration) the dK/dV launch's waves take, with its count: the kernel's block ->
    (split, (batch, KV head) of each wave, first unit) mapping, its unit list and each wave's iterations
    ifirst + wp + WPP j of the split's range."""
    S = dkdv_split(B, H, KVH, T)
    paired, wpp = dkdv_mode(B, H, KVH, T)
    nkb = nqt = (T + 63) // 64
    BKV, group, NW = B * KVH, H // KVH, 4
    ppb = NW // wpp
    nbk = (BKV + ppb - 1) // ppb
    nbase = nbk * ((nkb + 1) // 2 if paired else nkb)
    owners = {}
    for block in range(nbase * S):
        sidx, bid = divmod(block, nbase)
        bgrp, pj = bid % nbk, bid // nbk
        units = [pj] if (not paired or nkb - 1 - pj == pj) else [pj, nkb - 1 - pj]
        for wave in range(NW):
            wp = wave % wpp
            bk = bgrp if wpp == NW else bgrp * ppb + wave // wpp
            if bk >= BKV:
                continue  # the last block's idle waves
            for unit in units:
                n = group * (nqt - unit)
                first, end = sidx * n // S, (sidx + 1) * n // S
                for itn in range(first + wp, end, wpp):
                    owners[(bk, unit, itn)] = owners.get((bk, unit, itn), 0) + 1
    return owners, (S, wpp, paired, nbase * S)


@pytest.mark.parametrize(
    "B, H, KVH, T",
    [(1, 12, 4, 256), (4, 12, 4, 256), (16, 12, 4, 256), (32, 12, 4, 256), (8, 12, 4, 1024), (32, 12, 4, 1024),
     (64, 12, 4, 128), (24, 12, 4, 256), (8, 12, 12, 256), (33, 3, 3, 256), (16, 12, 4, 512),
     (16, 12, 4, 1024), (1, 12, 4, 1024), (2, 12, 4, 8192), (8, 12, 12, 1024), (8, 12, 1, 1024), (1, 4, 4, 65),
     (3, 6, 2, 333), (1, 1, 1, 1), (2, 8, 8, 100)],
)
def test_dkdv_blocks_take_every_iteration_once(B, H, KVH, T):
    owners, (S, wpp, paired, blocks) = dkdv_owners(B, H, KVH, T)
    nkb = nqt = (T + 63) // 64
    want = {(bk, u, i) for bk in range(B * KVH) for u in range(nkb) for i in range((H // KVH) * (nqt - u))}
    assert set(owners) == want and all(c == 1 for c in owners.values()), (S, wpp, paired)
    if not paired:
        assert S == 1 and blocks <= 256 and (wpp == 4 or wpp == 2)


def test_single_units_only_for_small_unsplit_problems():
    assert dkdv_mode(1, 12, 4, 256) == (False, 4)  # BASELINE config 1's shape: 16 blocks of one unit, not 8 pairs
    assert dkdv_mode(16, 12, 4, 256) == (False, 4)  # 256 units, one per CU
    assert dkdv_mode(32, 12, 4, 256) == (False, 2)  # 512 units, two per block (the ladder's T=256 point)
    assert dkdv_mode(64, 12, 4, 128) == (False, 2)
    assert dkdv_mode(16, 12, 4, 512) == (True, 4)  # 512 units, but a wave's share of unit 0 (12) is too long
    assert dkdv_mode(8, 12, 4, 1024) == (True, 4)  # config 2
    assert dkdv_mode(1, 12, 4, 1024)[0]  # split work keeps pairs


@pytest.mark.parametrize(
    "B, H, KVH, T",
    [(1, 12, 4, 256), (16, 12, 4, 256), (32, 12, 4, 256), (64, 12, 4, 128), (16, 12, 4, 512), (8, 12, 4, 1024),
     (32, 12, 4, 1024), (2, 12, 4, 8192), (1, 12, 4, 16384), (16, 12, 4, 1024), (65, 4, 2, 700), (91, 2, 1, 700),
     (2, 12, 1, 1024), (1, 12, 2, 700), (33, 3, 3, 256), (8, 12, 12, 256), (1, 1, 1, 1), (0, 12, 4, 256), (4, 8, 8, 0)],
)
def test_library_plan_matches_the_mirrors(B, H, KVH, T):
    # The library's own launch decisions (nn_fa_bwd_plan, computed on the host) are what the emulations above
    # restate: the same splits, waves, pairing and grid.
    import ctypes

    n, w, p, g = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int64()
    assert lib().nn_fa_bwd_plan(B, H, KVH, T, ctypes.byref(n), ctypes.byref(w), ctypes.byref(p), ctypes.byref(g)) == 0
    if B == 0 or T == 0:
        assert g.value == 0
        return
    paired, wpp = dkdv_mode(B, H, KVH, T)
    assert (n.value, w.value, bool(p.value)) == (dkdv_split(B, H, KVH, T), wpp, paired)
    nkb, ppb = (T + 63) // 64, 4 // wpp
    assert g.value == -(-B * KVH // ppb) * ((nkb + 1) // 2 if paired else nkb) * n.value
    if B * KVH * T <= 1 << 16:  # and the grid the block-mapping emulation walks
        assert g.value == dkdv_owners(B, H, KVH, T)[1][3]


def test_library_plan_rejects_bad_sizes():
    import ctypes

    n, w, p, g = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int64()
    assert lib().nn_fa_bwd_plan(1, 12, 5, 64, ctypes.byref(n), ctypes.byref(w), ctypes.byref(p), ctypes.byref(g)) != 0
    assert b"group evenly" in lib().nn_fa_last_error()
    assert lib().nn_fa_bwd_plan(1, 12, 4, 64, None, ctypes.byref(w), ctypes.byref(p), ctypes.byref(g)) != 0
