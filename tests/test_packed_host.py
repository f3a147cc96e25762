"""Packed one-member tiles (blockgrid_hip.build_packed) on the CPU.

The kernel's reading of a tile row is restated here from its description: tile
row r of (A, qa0, na, B, qb0) is query qa0 + r of window A below na rows and
query qb0 + (r - na) of window B from there; a two-window tile walks the KV
cuboid of A's frames and rows over the union of the two column ranges, and the
lane masks the columns outside its own window.  These tests check that every
query of every window lands in exactly one tile row and that the keys such a
row sees are exactly its window's KV cuboid (the planner's visibility rule),
by enumerating them.
"""
import pytest

from sr_dit import attention as att
from sr_dit import blockgrid_hip as bgh


def _shipped(streaming=True, h=45, w=80, f_cur=3, f_kv=12):
    return att._BlockGridSpec(f_cur=f_cur, f_kv=f_kv, h=h, w=w, block_t=3, bh=4, bw=4, rh=3,
                              rw=3, rt=f_kv // 3 - 1, streaming=streaming)


def _rows_of_tile(p, tile):
    """(window row, query index) of each of the tile's 64 rows (None: padding)."""
    ra, qa0, na, rb, qb0 = tile
    out = []
    for r in range(64):
        if r < na:
            lq = p[ra][1] * p[ra][4] * p[ra][5]
            out.append((ra, qa0 + r) if qa0 + r < lq else None)
        elif rb >= 0:
            lq = p[rb][1] * p[rb][4] * p[rb][5]
            q = qb0 + r - na
            out.append((rb, q) if q < lq else None)
        else:
            out.append(None)
    return out


def _cuboid(row):
    """The KV tokens (frame, row, column) of a plain params row."""
    t0, tl, h0, hl, w0, wl = row[6], row[7], row[8], row[9], row[10], row[11]
    return {(t, y, x) for t in range(t0, t0 + tl) for y in range(h0, h0 + hl)
            for x in range(w0, w0 + wl)}


@pytest.mark.parametrize("h,w", [(45, 80), (24, 40), (20, 36)])
def test_every_query_in_one_tile_row(h, w):
    plan = bgh.build_plan(_shipped(h=h, w=w))
    tiles = bgh.build_packed(plan)
    assert tiles is not None and tiles.shape[1] == 5
    p = plan["params"].tolist()
    seen = {}
    for tile in tiles.tolist():
        assert 0 < tile[2] <= 64
        for slot in _rows_of_tile(p, tile):
            if slot is not None:
                seen[slot] = seen.get(slot, 0) + 1
    want = {(r, q) for r, row in enumerate(p) for q in range(row[1] * row[4] * row[5])}
    assert set(seen) == want
    assert all(c == 1 for c in seen.values())


def test_two_window_tiles_see_exactly_their_windows_keys():
    plan = bgh.build_plan(_shipped())
    tiles = bgh.build_packed(plan).tolist()
    p = plan["params"].tolist()
    pairs = [t for t in tiles if t[3] >= 0]
    assert len(pairs) > len(tiles) // 3
    for ra, qa0, na, rb, qb0 in pairs:
        a, b = p[ra], p[rb]
        assert a[6:10] == b[6:10] and a[0:2] == b[0:2]  # frames and rows shared
        u0 = min(a[10], b[10])
        u1 = max(a[10] + a[11], b[10] + b[11])
        assert u1 - u0 == bgh.PACK_WIDTH
        union = {(t, y, x) for t in range(a[6], a[6] + a[7]) for y in range(a[8], a[8] + a[9])
                 for x in range(u0, u1)}
        for row in (a, b):
            lo = row[10] - u0
            hi = lo + row[11]
            seen = {(t, y, x) for (t, y, x) in union if lo <= x - u0 < hi}
            assert seen == _cuboid(row)
        # a 32-key step of the union is one token row: key k is column u0 + k
        assert (u1 - u0) % 32 == 0


def test_no_tile_holds_more_than_two_windows_and_work_drops():
    plan = bgh.build_plan(_shipped())
    tiles = bgh.build_packed(plan)
    singles = bgh.build_singles(plan)
    p = plan["params"].tolist()
    for tile in tiles.tolist():
        wins = {s[0] for s in _rows_of_tile(p, tile) if s is not None}
        assert 1 <= len(wins) <= 2
    # the shipped 45x80 geometry: 240 windows of 48 (or 12) queries
    assert tiles.shape[0] < singles.shape[0]

    def keys(row):
        return row[7] * row[9] * row[11]
    work_singles = sum(keys(p[r]) for r, *_ in singles.tolist())
    work_packed = sum(p[a][7] * p[a][9] * bgh.PACK_WIDTH if b >= 0 else keys(p[a])
                      for a, _, _, b, _ in tiles.tolist())
    assert work_packed < 0.95 * work_singles


def test_greedy_cut_packs_40_query_windows():
    # c3: 8x8 blocks of radius 1; the ragged last block row has 40-query windows
    # whose interior neighbours span 32 columns: three windows in two tiles
    from sr_dit import workloads as wl
    plan = bgh.build_plan(wl.window_spec("c3"))
    tiles = bgh.build_packed(plan)
    p = plan["params"].tolist()
    pairs = [t for t in tiles.tolist() if t[3] >= 0]
    assert pairs and all(p[a][1] * p[a][4] * p[a][5] == 40 for a, *_ in pairs)
    assert tiles.shape[0] < bgh.build_singles(plan).shape[0]


def test_plans_that_do_not_pack():
    # c1: 16x16 frames of 8x8 blocks, every window spans the same 16 columns
    from sr_dit import workloads as wl
    assert bgh.build_packed(bgh.build_plan(wl.window_spec("c1"))) is None
    # a 28-token-wide frame: every window spans all 28 columns, no union is 32 wide
    assert bgh.build_packed(bgh.build_plan(_shipped(h=16, w=28))) is None
    # an anchored plan is never packed
    spec = _shipped()
    assert bgh.build_packed(bgh.build_plan(spec, anchor_mode="frame")) is None


def test_auto_packs_only_where_tiles_drop():
    """kernel="auto" takes packed tiles only when they remove PACKED_MIN_SAVING of
    the one-window tiles: the shipped geometry at every cache length, not c1-c4."""
    from sr_dit import workloads as wl
    for f_kv in (3, 6, 9, 12):
        assert bgh.packed_saving(bgh.build_plan(_shipped(f_kv=f_kv))) >= bgh.PACKED_MIN_SAVING
    for cfg in ("c1", "c2", "c3", "c4"):
        assert bgh.packed_saving(bgh.build_plan(wl.window_spec(cfg))) < bgh.PACKED_MIN_SAVING
