"""LDS layout and workgroup->tile order, through the built library (no GPU).

The kernel's LDS tile rows are 128 bytes (eight 16-byte slots).  hipgemm_lds_slot
(plain K order) and hipgemm_lds_slot_kpair (the MFMA's own K order) expose the
slot of (row, K-chunk); these tests check the properties the kernels rely on
rather than restating the formula:
  * each row's chunk->slot map is a permutation (DMA lands every chunk once);
  * MFMA operand fetches hit 16 distinct 16-byte bank groups per 256 bytes
    in each 16-lane group (a necessary condition);
  * the instruction-order fetch (lane group g: chunks g and g + 4) reads
    exactly the addresses of the plain fetch of chunks 2g and 2g + 1 -- the
    pattern measured conflict-free on gfx950 (SQ_LDS_BANK_CONFLICT), where
    reading chunks g and g + 4 from the plain layout measured 4 conflict
    cycles per ds_read_b128;
  * the tile order visits every tile exactly once for any grid size.
"""
import itertools

import numpy as np
import pytest

import hipgemm_amd as hg


ROW = 128  # bytes per LDS tile row
SLOTS = 8


def slot(r, c):
    s = hg.lds_slot(r, c)
    assert 0 <= s < SLOTS
    return s


def test_slot_is_permutation_per_row():
    for r in range(512):
        assert sorted(slot(r, c) for c in range(SLOTS)) == list(range(SLOTS)), r
    assert hg.lds_slot(-1, 0) == -1 and hg.lds_slot(0, SLOTS) == -1


def test_slot_depends_on_row_mod_16_only():
    for r in range(256):
        for c in range(SLOTS):
            assert slot(r, c) == slot(r % 16, c)


@pytest.mark.parametrize("base", [0, 32, 64, 96, 128, 160, 192, 224])
def test_operand_fetch_bank_conflict_free(base):
    # lane l of an MFMA fragment fetch reads row base + l%32 at chunk
    # 4*kh + 2*(l//32) + t (K-half kh, sub-chunk t); hardware serves 16 (or 8)
    # lanes at a time.
    for kh, t in ((0, 0), (0, 1), (1, 0), (1, 1)):
        addrs = [(base + l % 32) * ROW +
                 slot(base + l % 32, 4 * kh + 2 * (l // 32) + t) * 16
                 for l in range(64)]
        for g0 in range(0, 64, 16):
            grp = addrs[g0:g0 + 16]
            assert len({(a % 256) // 16 for a in grp}) == 16, (base, kh, t, g0)
        for g0 in range(0, 64, 8):
            grp = addrs[g0:g0 + 8]
            assert len({(a % 128) // 16 for a in grp}) == 8, (base, kh, t, g0)


def test_kpair_slot_is_permutation_per_row():
    for r in range(64):
        assert sorted(hg.lds_slot_kpair(r, c) for c in range(SLOTS)) == \
            list(range(SLOTS)), r
    assert hg.lds_slot_kpair(-1, 0) == -1 and hg.lds_slot_kpair(0, SLOTS) == -1


@pytest.mark.parametrize("base", [0, 16, 48, 112])
def test_kpair_fetch_equals_plain_pair_fetch(base):
    # 16x16x128 fetch: lane l reads row base + l%16; lane group g = l//16
    # needs K-chunks g (first read) and g + 4 (second).  Plain order reads
    # chunks 2g and 2g + 1 at the same lanes: the same addresses, read for
    # read.
    for first in (True, False):
        kp = [(base + l % 16) * ROW +
              hg.lds_slot_kpair(base + l % 16, (l // 16) + (0 if first else 4)) * 16
              for l in range(64)]
        plain = [(base + l % 16) * ROW +
                 slot(base + l % 16, 2 * (l // 16) + (0 if first else 1)) * 16
                 for l in range(64)]
        assert kp == plain, (base, first)
        for g0 in range(0, 64, 16):
            assert len({(a % 256) // 16 for a in kp[g0:g0 + 16]}) == 16


def test_kpair_dma_fill_covers_every_chunk_once():
    # DMA lane l fetches the chunk stored at slot l%8 of row R0 + l//8.
    for R0 in (0, 8, 16, 248):
        seen = set()
        for l in range(64):
            r, s = R0 + l // 8, l % 8
            c = [c for c in range(SLOTS) if hg.lds_slot_kpair(r, c) == s]
            assert len(c) == 1
            seen.add((r, c[0]))
        assert len(seen) == 64


def test_dma_fill_covers_every_chunk_once():
    # DMA lane l of the instruction for rows [R0, R0+8) fetches chunk
    # (l%8) ^ xor(row) into slot l%8 of row R0 + l//8; i.e. slot s of row r
    # holds chunk c with lds_slot(r, c) == s.  Every (row, chunk) lands once.
    for R0 in (0, 8, 16, 248):
        seen = set()
        for l in range(64):
            r, s = R0 + l // 8, l % 8
            c = [c for c in range(SLOTS) if slot(r, c) == s]
            assert len(c) == 1
            seen.add((r, c[0]))
        assert len(seen) == 64


GRIDS = [(1, 1, 1), (4, 2, 2), (305, 16, 20), (320, 16, 20), (256, 16, 20),
         (1024, 32, 32), (3584, 32, 112), (7, 3, 5), (9, 3, 3), (64, 4, 4),
         (13, 1, 40), (100, 40, 1), (255, 17, 15)]


@pytest.mark.parametrize("grid,tm,tn", GRIDS)
def test_tile_order_bijective(grid, tm, tn):
    for gm in (0, 1, 3, 4, 8):
        ms, ns = hg.tile_order(grid, tm, tn, gm)
        assert len(ms) == tm * tn
        pairs = set(zip(ms, ns))
        assert pairs == set(itertools.product(range(tm), range(tn))), (grid, gm)


def test_tile_order_xcd_blocks_are_compact():
    # 8192^3: 32 x 32 tiles, one tile per workgroup.  Workgroup b runs on XCD
    # b % 8; the 32 workgroups an XCD holds at once (one per CU) should form a
    # compact block of tiles (few distinct A row-panels and B column-panels).
    grid = 1024
    ms, ns = hg.tile_order(grid, 32, 32)
    first = {}
    for b in range(grid):
        first[b] = (ms[b], ns[b])
    for x in range(8):
        wave0 = [first[b] for b in range(x, grid, 8)][:32]
        assert len({m for m, _ in wave0}) <= 4
        assert len({n for _, n in wave0}) <= 8


# ---- the 4-wave schedule's epilogue stage (hipgemm_lds_stage_slot) -------
# 64 rows x 128 bytes per wave.  Measured on gfx950 with a probe kernel that
# replays one access pattern under SQ_LDS_BANK_CONFLICT (per instruction,
# block write / read-back): slot x ^ (r mod 16): 0 / 2 cycles;
# x ^ ((r & 14) | ((r >> 1) & 1)): 4 / 0; the layout used: 0 / 0.  The two
# conditions below are the ones those results fit.

def test_stage_slot_is_permutation_per_row():
    for r in range(64):
        assert sorted(hg.lds_stage_slot(r, x) for x in range(16)) == list(range(16))
        assert [hg.lds_stage_slot(r, x) for x in range(16)] == \
            [hg.lds_stage_slot(r % 16, x) for x in range(16)]
    assert hg.lds_stage_slot(-1, 0) == -1 and hg.lds_stage_slot(0, 16) == -1


def test_stage_block_writes_take_16_slots():
    """A block write (ds_write_b64): lane l writes piece 4 bj + l / 16 of row
    16 bi + l % 16; the 16 lanes of one piece index take 16 distinct slots."""
    for x in range(16):
        assert sorted(hg.lds_stage_slot(r, x) for r in range(16)) == list(range(16))


def test_stage_readback_rows_two_apart_disjoint():
    """A read-back (ds_read_b64): lane l reads piece 2 (l % 8) + h of row
    8 p + l / 8; rows r and r + 2 (256 bytes apart) read disjoint slot
    sets, i.e. opposite slot parities."""
    for r in range(64):
        for h in range(2):
            a = {hg.lds_stage_slot(r, 2 * c + h) for c in range(8)}
            b = {hg.lds_stage_slot(r + 2, 2 * c + h) for c in range(8)}
            assert not a & b, (r, h)
