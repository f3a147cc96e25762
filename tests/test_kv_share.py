"""Shared-fetch schedules (sr_dit/kv_share.py) on the CPU.

Every schedule is replayed by ``check_schedule``: each member consumes exactly
its window's 4x8-token units, once each, from slots filled in its step, and no
fill overwrites a slot before its last read retires.  The unit sets are
checked against a per-token brute force of the params rows, and a corrupted
schedule must fail the replay.
"""
import itertools

import pytest
import torch

from sr_dit import attention as att
from sr_dit import blockgrid_hip as bgh
from sr_dit import kv_share as ks
from sr_dit import workloads as wl


def _sym(f, h, w, bh=8, bw=8, rh=1, rw=1, rt=1):
    return att._BlockGridSpec(f_cur=f, f_kv=f, h=h, w=w, block_t=1, bh=bh, bw=bw, rh=rh, rw=rw,
                              sym_rt=rt)


CASES = [
    ("c1", wl.window_spec("c1")),
    ("c2", wl.window_spec("c2")),
    ("c3", wl.window_spec("c3")),
    ("c4", wl.window_spec("c4")),
    ("ragged_3x13x21", _sym(3, 13, 21)),
    ("one_frame_8x40", _sym(1, 8, 40)),
    ("radius2_4x24x32", _sym(4, 24, 32, rh=2, rw=2, rt=1)),
    ("block16x8_3x32x24", _sym(3, 32, 24, bh=16, bw=8)),
    ("stream_2of4_16x16", att._BlockGridSpec(f_cur=2, f_kv=4, h=16, w=16, block_t=3, bh=8, bw=8,
                                             rh=1, rw=1, rt=1, streaming=True)),
]


@pytest.mark.parametrize("name,spec", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("members", [2, 4])
def test_schedule_replays(name, spec, members):
    plan = bgh.build_plan(spec)
    assert ks.share_supported(plan, spec.h, spec.w, 128)
    sched = ks.build_share_schedule(plan, spec.h, spec.w, members)
    ks.check_schedule(plan, spec.h, spec.w, sched)
    assert sched["member_units"] >= sched["fetched_units"]


def test_units_match_token_brute_force():
    """The units of a row cover exactly the row's KV tokens (per frame, row, column)."""
    spec = _sym(3, 13, 21)
    plan = bgh.build_plan(spec)
    for row in plan["params"].tolist():
        toks = {(f, r, c) for f in range(row[6], row[6] + row[7])
                for r in range(row[8], row[8] + row[9]) for c in range(row[10], row[10] + row[11])}
        from_units = set()
        for f, ur, uc in ks._row_units(row, spec.h, spec.w):
            for r, c in itertools.product(range(4 * ur, 4 * ur + 4), range(8 * uc, 8 * uc + 8)):
                if r < spec.h and c < spec.w:
                    from_units.add((f, r, c))
        assert from_units == toks


def test_fetch_reduction_c3():
    """c3: each fetched unit serves more than two members on average, and every
    member is busy in more than 90% of its workgroup's steps."""
    spec = wl.window_spec("c3")
    sched = ks.build_share_schedule(bgh.build_plan(spec), spec.h, spec.w)
    assert sched["member_units"] / sched["fetched_units"] > 2.0
    assert sched["member_units"] / (4 * sched["steps"].shape[0]) > 0.9


def test_unsupported_geometries():
    prod = wl.window_spec("prod")       # 4x4 blocks: cuboids not made of 4x8 units
    assert not ks.share_supported(bgh.build_plan(prod), prod.h, prod.w, 128)
    c3 = wl.window_spec("c3")
    assert not ks.share_supported(bgh.build_plan(c3), c3.h, c3.w, 64)
    anc = att._BlockGridSpec(f_cur=2, f_kv=4, h=16, w=16, block_t=2, bh=8, bw=8, rh=1, rw=1, rt=1,
                             streaming=True)
    assert not ks.share_supported(bgh.build_plan(anc, anchor_mode="chunk"), 16, 16, 128)


def _corrupt(sched, fn):
    s = {k: (v.clone() if torch.is_tensor(v) else v) for k, v in sched.items()}
    fn(s)
    return s


def test_negative_controls():
    spec = _sym(3, 16, 24)
    plan = bgh.build_plan(spec)
    sched = ks.build_share_schedule(plan, spec.h, spec.w)
    ks.check_schedule(plan, spec.h, spec.w, sched)

    def drop_member_unit(s):       # a member skips one of its units
        st = s["steps"]
        i = int((st[:, 8] != 0).nonzero()[0])
        st[i, 8] = 0

    def reuse_k_slot_early(s):     # step 1 fills into the K slot step 0 still reads
        st = s["steps"]
        k0 = int(st[0, 1]) & 0xFF
        st[1, 1] = (int(st[1, 1]) & ~0xFF) | k0
        for m in range(4):
            w = int(st[1, 8 + m])
            if w:
                st[1, 8 + m] = (w & ~31) | k0

    def wrong_valid_rows(s):
        st = s["steps"]
        i = int((st[:, 8] != 0).nonzero()[0])
        st[i, 8] = (int(st[i, 8]) & ~(7 << 10)) | (2 << 10)

    for bad in (drop_member_unit, reuse_k_slot_early, wrong_valid_rows):
        with pytest.raises(AssertionError):
            ks.check_schedule(plan, spec.h, spec.w, _corrupt(sched, bad))
