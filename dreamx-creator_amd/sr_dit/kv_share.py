"""Shared-fetch schedules for the block-grid window kernel on gfx950.

Neighbouring windows of the block grid read overlapping KV cuboids: under the
8x8-block, radius-1, +-1-frame rule a window's 3x3x3 blocks overlap its
spatial neighbour's in 2x3x3 of them.  The shared-fetch kernel
(``srdit_window_attn_shared_fwd``) runs four 64-query *members* per workgroup
(eight wavefronts) and fetches every KV *unit* once for all the members that
read it in the same step.

A unit is 32 keys: 4 token rows x 8 token columns of one KV frame, on a grid
aligned to row multiples of 4 and column multiples of 8.  A window's KV cuboid
(fields ``kv_t0 kv_tL kh0 khL kw0 kwL`` of a plain params row,
blockgrid_triton.py:77-80) is a union of whole units when its row extent starts
on a multiple of 4, its column extent on a multiple of 8, and both end on such
a multiple or at the grid edge; units cut by the grid edge carry their valid
row and column counts and the kernel masks the rest.  Plans that do not meet
this (the shipped 4x4-block geometry, anchored rows) run on the other kernels.

The host builds, per workgroup:

* the members: up to four (row, m-tile) pairs whose windows have the same
  number of units (so every member is busy in every step) and overlap as much
  as possible (chosen among the nearest candidates);
* the steps: in each step every member with units left consumes one; the unit
  read by the most members is picked first, so the shared middle of a group's
  windows is fetched once per step for all its readers;
* the fills: a unit's K and V each take one 8 KB slot from a pool of
  ``5 * members`` slots, from the iteration its fill is issued until its last
  read has retired.

The kernel reads K of step ``s`` at iteration ``s - 1`` (the S MFMAs run one
step ahead of the softmax) and V at iteration ``s``.  The fill list of record
``r`` (the units of step ``r``) is issued at iteration ``r - 2`` (records 0
and 1 before the first iteration).  Every iteration starts with a full wait
for the wavefront's fills and a barrier, so a fill lands before the next
iteration and may overwrite a slot whose last read was at iteration ``i - 1``
or earlier.  With five slots per member a step's K and V always fit (K of
two steps and V of three are live).  :func:`check_schedule` replays these
rules on the CPU.
"""
from __future__ import annotations

import itertools

import torch

#: Keys per unit and its token shape.
UNIT_KEYS = 32
UNIT_ROWS = 4
UNIT_COLS = 8
#: Largest number of members per workgroup (two wavefronts each).
MEMBERS = 4


def n_slots(members):
    """LDS slots of the kernel, shared by K and V tiles (8 KB each: 32 keys x
    128 dims x 2 bytes): 160 KB for four members, 80 KB for two."""
    return 5 * members


#: Iterations between a fill's issue and the V read of its step.
LOOKAHEAD = 2
#: Fill units per record.
FILLS_PER_RECORD = 4
#: Record flag: this record's fills must land by the next iteration's barrier.
FLAG_LAND_NEXT = 1
#: int32 words per step record.
STEP_WORDS = 16
#: Query rows per member.
MEMBER_Q = 64
#: Candidate partners examined per group seed.
NEIGHBOURS = 10


def _row_units(row, H, W):
    """Units of a plain params row's KV cuboid, or None if it is not a union of units."""
    kv_t0, kv_tl, kh0, khl, kw0, kwl = row[6], row[7], row[8], row[9], row[10], row[11]
    if row[12] != 0 or kv_tl <= 0 or khl <= 0 or kwl <= 0:
        return None
    if kh0 % UNIT_ROWS or kw0 % UNIT_COLS:
        return None
    if khl % UNIT_ROWS and kh0 + khl != H:
        return None
    if kwl % UNIT_COLS and kw0 + kwl != W:
        return None
    urs = range(kh0 // UNIT_ROWS, -(-(kh0 + khl) // UNIT_ROWS))
    ucs = range(kw0 // UNIT_COLS, -(-(kw0 + kwl) // UNIT_COLS))
    return frozenset((f, ur, uc) for f in range(kv_t0, kv_t0 + kv_tl) for ur in urs for uc in ucs)


def share_supported(plan, H, W, head_dim) -> bool:
    """True when the shared-fetch kernel can run ``plan`` on an H x W token grid:
    plain 19-field rows without an anchor prefix, head_dim 128, every KV cuboid
    a union of 4x8 units, at most 255 KV frames."""
    if plan["p_stride"] != 19 or head_dim != 128:
        return False
    p = plan["params"].tolist()
    if not p:
        return False
    for row in p:
        if row[6] + row[7] > 255 or _row_units(row, H, W) is None:
            return False
    return True


def _members(plan):
    """(row, m-tile, q_t0, q_h0, q_w0) for every 64-query tile of every window."""
    out = []
    for r, row in enumerate(plan["params"].tolist()):
        lq = row[1] * row[4] * row[5]
        for mt in range(-(-lq // MEMBER_Q) if lq > 0 else 0):
            out.append((r, mt, row[0], row[2], row[3]))
    return out


def _form_groups(members, units, size):
    """Groups of up to ``size`` member indices.

    Seeds are taken in raster order (query frame, row, column); a seed's
    partners are drawn from the NEIGHBOURS members with the same unit count
    that overlap it most (ties: the same query frame, then the nearest in the
    frame), choosing the largest group whose union of units is smallest.
    Groups within one query frame keep a group's KV to the frame's own
    neighbourhood, so workgroups running together share more of the L2.
    """
    order = sorted(range(len(members)), key=lambda i: (members[i][2], members[i][3],
                                                        members[i][4], members[i][0],
                                                        members[i][1]))
    left = set(order)
    by_size: dict = {}
    for i in order:
        by_size.setdefault(len(units[i]), []).append(i)
    groups = []
    for seed in order:
        if seed not in left:
            continue
        left.discard(seed)
        su = units[seed]
        ms = members[seed]
        cands = [i for i in by_size[len(su)] if i in left and units[i] & su]
        cands.sort(key=lambda i: (-len(units[i] & su), abs(members[i][2] - ms[2]),
                                  abs(members[i][3] - ms[3]) + abs(members[i][4] - ms[4]), i))
        cands = cands[:NEIGHBOURS]
        best = None
        for k in range(min(size - 1, len(cands)), -1, -1):
            for combo in itertools.combinations(cands, k):
                n_union = len(su.union(*(units[c] for c in combo)))
                if best is None or n_union < best[0]:
                    best = (n_union, combo)
            if best is not None:
                break
        for c in best[1]:
            left.discard(c)
        groups.append([seed, *best[1]])
    return groups


def _steps(sets):
    """Per step, {member slot: unit}: every member with units left takes one, the
    unit wanted by the most remaining members first (ties: frame, row, column)."""
    rem = [set(s) for s in sets]
    steps = []
    while any(rem):
        assigned = {}
        free = [m for m in range(len(rem)) if rem[m]]
        while free:
            count: dict = {}
            for m in free:
                for u in rem[m]:
                    count[u] = count.get(u, 0) + 1
            unit = min(count, key=lambda u: (-count[u], u))
            takers = [m for m in free if unit in rem[m]]
            for m in takers:
                assigned[m] = unit
                rem[m].discard(unit)
            free = [m for m in free if m not in takers]
        steps.append(assigned)
    return steps


def _allocate(steps, members):
    """LDS slots of every unit of a group's steps.

    Returns ``(slots, fills, flags)``: per step ``{unit: (k_slot, v_slot)}``,
    per record ``r`` the units issued at iteration ``r - LOOKAHEAD`` (the
    units of step ``r``; record n is empty) and the record flags (none).  A
    unit of step s is held from its fill (iteration s-2) to its K read (s-1)
    and V read (s); a slot frees for fills of the iteration after its last read.
    """
    n = len(steps)
    nsl = n_slots(members)
    busy = [[] for _ in range(nsl)]  # per slot: (first, last) iterations it is held

    def free(slot, lo, hi):
        return all(hi < a or lo > b for a, b in busy[slot])

    fills = [[] for _ in range(n + 1)]
    flags = [0] * (n + 1)
    slots = []
    for s, assigned in enumerate(steps):
        here = {}
        first = s - LOOKAHEAD
        for unit in sorted(set(assigned.values())):
            ks = next((k for k in range(nsl) if free(k, first, s - 1)), None)
            vs = next((v for v in range(nsl) if v != ks and free(v, first, s)), None)
            if ks is None or vs is None or len(fills[s]) >= FILLS_PER_RECORD:
                raise RuntimeError("kv_share: a step needs more LDS slots or fill entries than "
                                   "the kernel has")
            busy[ks].append((first, s - 1))
            busy[vs].append((first, s))
            fills[s].append((unit, ks, vs))
            here[unit] = (ks, vs)
        slots.append(here)
    return slots, fills, flags


def _member_word(ks, vs, nrows, ncols):
    return ks | (vs << 5) | (nrows << 10) | (ncols << 13)


def build_share_schedule(plan, H, W, members=MEMBERS):
    """The shared-fetch launch tables for ``plan`` on an H x W token grid, with
    ``members`` (2 or 4) members per workgroup.

    Returns ``{"groups": int32 [G, 8] ((row, m-tile) x 4, row -1 = none),
    "step_off": int32 [G + 1], "steps": int32 [S, 16], "n_groups": G,
    "members", "fetched_units", "member_units"}``.  Record ``r`` words 0-7: up
    to four fill units issued at iteration ``r - 3``, (frame << 24 | token
    offset of the unit in its frame, k_slot | v_slot << 8) or (-1, 0); words
    8-11: per member its unit of step ``r``, k_slot | v_slot << 5 | valid rows
    << 10 | valid columns << 13 (0: idle this step); word 12: the number of
    fill units; word 13: flags (1: the fills must land by the next barrier).
    A workgroup of n steps has n + 1 records (the last carries fills only).
    """
    if members not in (2, 4):
        raise ValueError(f"build_share_schedule: members must be 2 or 4, got {members}")
    size = members
    p = plan["params"].tolist()
    members = _members(plan)
    units = [_row_units(p[m[0]], H, W) for m in members]
    if any(u is None for u in units):
        raise ValueError("build_share_schedule: plan rows are not unions of 4x8 KV units")
    groups = _form_groups(members, units, size)
    # heaviest first within a query frame, groups of one frame together
    groups.sort(key=lambda g: (members[g[0]][2], -max(len(units[i]) for i in g),
                               members[g[0]][3], members[g[0]][4]))
    gtab, offs, recs = [], [0], []
    fetched = used = 0
    for g in groups:
        row = []
        for slot in range(MEMBERS):
            if slot < len(g):
                row += [members[g[slot]][0], members[g[slot]][1]]
            else:
                row += [-1, 0]
        gtab.append(row)
        steps = _steps([units[i] for i in g])
        slots, fills, flags = _allocate(steps, size)
        for r in range(len(steps) + 1):
            assigned, here = (steps[r], slots[r]) if r < len(steps) else ({}, {})
            rec = [-1, 0] * 4 + [0] * 8
            for u_i, (unit, ks, vs) in enumerate(fills[r]):
                f, ur, uc = unit
                rec[2 * u_i] = (f << 24) | (ur * UNIT_ROWS * W + uc * UNIT_COLS)
                rec[2 * u_i + 1] = ks | (vs << 8)
            rec[12] = len(fills[r])
            rec[13] = flags[r]
            for m, unit in assigned.items():
                f, ur, uc = unit
                ks, vs = here[unit]
                nrows = min(UNIT_ROWS, H - ur * UNIT_ROWS)
                ncols = min(UNIT_COLS, W - uc * UNIT_COLS)
                rec[8 + m] = _member_word(ks, vs, nrows, ncols)
            recs.append(rec)
            fetched += len(here)
            used += len(assigned)
        offs.append(len(recs))
    return {"groups": torch.tensor(gtab, dtype=torch.int32).reshape(-1, 2 * MEMBERS).contiguous(),
            "step_off": torch.tensor(offs, dtype=torch.int32),
            "steps": torch.tensor(recs, dtype=torch.int32).reshape(-1, STEP_WORDS).contiguous(),
            "n_groups": len(groups), "members": size, "fetched_units": fetched,
            "member_units": used}


def check_schedule(plan, H, W, sched) -> None:
    """Replay a schedule on the CPU; raise AssertionError on any violation.

    Checks that every member consumes exactly its window's units, each once,
    with its active steps first, and that every K read (iteration s-1) and V
    read (iteration s) of a member's step-s unit finds that unit's tile in the
    slot, written by the latest fill into that slot before the read (issued
    in an earlier iteration, so a barrier waited for it), and not raced by a
    fill into the same slot issued in the reading iteration.
    """
    p = plan["params"].tolist()
    gt = sched["groups"].tolist()
    offs = sched["step_off"].tolist()
    recs = sched["steps"].tolist()
    nsl = n_slots(sched["members"])
    seen = set()
    for gi, g in enumerate(gt):
        mem = [(g[2 * m], g[2 * m + 1]) for m in range(MEMBERS)]
        assert all(r < 0 for r, _ in mem[sched["members"]:]), "member past the group size"
        want = []
        for r, mt in mem:
            want.append(set(_row_units(p[r], H, W)) if r >= 0 else set())
            if r >= 0:
                assert (r, mt) not in seen, ("member twice", r, mt)
                seen.add((r, mt))
        grecs = recs[offs[gi]:offs[gi + 1]]
        n = len(grecs) - 1  # compute steps; the last record carries fills only
        assert n >= 0 and all(w == 0 for w in grecs[n][8:12]), "last record computes"
        # fills per slot: (issue iteration, unit, kind, flagged)
        writes = [[] for _ in range(nsl)]
        for r, rec in enumerate(grecs):
            it = r - LOOKAHEAD
            nf = rec[12]
            assert 0 <= nf <= FILLS_PER_RECORD
            for u_i in range(4):
                a, b = rec[2 * u_i], rec[2 * u_i + 1]
                if u_i >= nf:
                    assert a == -1, "fill word past the count"
                    continue
                f, off = a >> 24, a & 0xFFFFFF
                unit = (f, off // W // UNIT_ROWS, (off % W) // UNIT_COLS)
                assert off == unit[1] * UNIT_ROWS * W + unit[2] * UNIT_COLS
                ks, vs = b & 0xFF, b >> 8
                assert 0 <= ks < nsl and 0 <= vs < nsl and ks != vs
                flagged = bool(rec[13] & FLAG_LAND_NEXT)
                writes[ks].append((it, unit, "K", flagged))
                writes[vs].append((it, unit, "V", flagged))
        got = [set() for _ in range(MEMBERS)]
        idle = [False] * MEMBERS

        def tile_at(slot, i):
            """The fill an iteration-i read of `slot` sees; asserts it has landed."""
            if i < 0:  # prologue read, after the full wait on every prologue fill
                before = [w for w in writes[slot] if w[0] < 0]
            else:
                assert not any(w[0] == i for w in writes[slot]), (
                    f"slot {slot} filled in iteration {i}, which reads it")
                before = [w for w in writes[slot] if w[0] < i]
            assert before, f"read of slot {slot} at iteration {i} before any fill"
            it, unit, kind, flagged = max(before, key=lambda w: w[0])
            # every barrier waits for all earlier fills
            assert it < 0 or it <= i - 1, (
                f"slot {slot} read at iteration {i}, fill issued at {it} not yet landed")
            return unit, kind

        for s, rec in enumerate(grecs[:n]):
            for m in range(MEMBERS):
                w = rec[8 + m]
                nrows = (w >> 10) & 7
                if nrows == 0:
                    idle[m] = True
                    continue
                assert not idle[m], "a member's active steps must be a prefix of the steps"
                ks, vs, ncols = w & 31, (w >> 5) & 31, (w >> 13) & 15
                assert ks < nsl and vs < nsl
                uk, kk = tile_at(ks, s - 1)
                uv, kv = tile_at(vs, s)
                assert kk == "K" and kv == "V" and uk == uv, "K and V tiles of different units"
                assert uk not in got[m], "unit consumed twice"
                got[m].add(uk)
                assert nrows == min(UNIT_ROWS, H - uk[1] * UNIT_ROWS)
                assert ncols == min(UNIT_COLS, W - uk[2] * UNIT_COLS)
        assert got == want, f"group {gi}: members' units differ from their windows"
    n_members = sum(1 for _ in _members(plan))
    assert len(seen) == n_members, "not every member is scheduled"
