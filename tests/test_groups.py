"""Grouped window kernel: host pairing of 64-query members and the slot schedule (CPU)."""
import itertools

import pytest
import torch

from sr_dit import blockgrid_hip as bgh
from sr_dit import workloads as wl


def _members(plan):
    out = set()
    for r, row in enumerate(plan["params"].tolist()):
        lq = row[1] * row[4] * row[5]
        out |= {(r, mt) for mt in range(-(-lq // 64))}
    return out


@pytest.mark.parametrize("cfg", ["c1", "c2", "c3", "c4"])
def test_groups_cover_every_member_once(cfg):
    plan = bgh.build_plan(wl.window_spec(cfg))
    g = bgh.build_groups(plan).tolist()
    seen = []
    p = plan["params"].tolist()
    for r0, m0, r1, m1 in g:
        seen.append((r0, m0))
        if r1 >= 0:
            seen.append((r1, m1))
            assert p[r0][8:12] == p[r1][8:12]                       # same spatial KV extent
            a0, la, a1, lb = p[r0][6], p[r0][7], p[r1][6], p[r1][7]
            assert min(a0 + la, a1 + lb) > max(a0, a1)              # overlapping frames
    assert len(seen) == len(set(seen)) and set(seen) == _members(plan)


def test_c3_pairs_neighbouring_query_frames():
    plan = bgh.build_plan(wl.window_spec("c3"))
    p = plan["params"].tolist()
    pairs = {(p[r0][0], p[r1][0]) for r0, _, r1, _ in bgh.build_groups(plan).tolist()}
    assert pairs == {(0, 1), (2, 3), (4, 5)}


def test_c4_pairs_the_two_m_tiles_of_each_window():
    plan = bgh.build_plan(wl.window_spec("c4"))
    g = bgh.build_groups(plan).tolist()
    assert all(r0 == r1 and (m0, m1) == (0, 1) for r0, m0, r1, m1 in g)
    assert len(g) == plan["n_w"]


def _schedule(a0, la, a1, lb):
    """Frame consumed by each member in each frame slot, as the kernel walks them:
    private slots first (each member its own frames, in order), then shared frames."""
    s_lo = max(a0, a1)
    nsh = max(0, min(a0 + la, a1 + lb) - s_lo) if lb > 0 else 0

    def priv(a, l):
        if nsh == 0:
            return list(range(a, a + l))
        return list(range(a, min(a + l, s_lo))) + list(range(max(a, s_lo + nsh), a + l))

    p0, p1 = priv(a0, la), priv(a1, lb) if lb > 0 else []
    P = max(len(p0), len(p1))
    slots = []
    for k in range(P):
        slots.append((p0[k] if k < len(p0) else None, p1[k] if k < len(p1) else None, 2))
    for k in range(nsh):
        slots.append((s_lo + k, s_lo + k, 1))
    return slots


def test_slot_schedule_consumes_each_frame_once():
    for a0, la, a1, lb in itertools.product(range(4), range(1, 5), range(4), range(0, 5)):
        slots = _schedule(a0, la, a1, lb)
        f0 = [s[0] for s in slots if s[0] is not None]
        f1 = [s[1] for s in slots if s[1] is not None]
        assert sorted(f0) == list(range(a0, a0 + la))
        assert sorted(f1) == list(range(a1, a1 + lb))
        # a shared slot fetches one block that both members consume
        assert all(s[0] == s[1] for s in slots if s[2] == 1)


def test_grouping_cuts_c3_fetches():
    """Blocks fetched per spatial step: c3's pairs fetch 10 frame blocks per window
    column where single windows would fetch 16."""
    plan = bgh.build_plan(wl.window_spec("c3"))
    p = plan["params"].tolist()
    single = sum(row[7] for row in p)
    grouped = 0
    for r0, _, r1, _ in bgh.build_groups(plan).tolist():
        slots = _schedule(p[r0][6], p[r0][7], p[r1][6], p[r1][7])
        grouped += sum((s[0] is not None) + (s[1] is not None) if s[2] == 2 else 1 for s in slots)
    assert grouped * 16 == single * 10


def test_unsupported_plans_and_kernel_switch():
    spec = wl.window_spec("c1")
    plan = bgh.build_plan(spec, anchor_mode="chunk")
    assert not bgh.groups_supported(plan)
    assert bgh.groups_supported(bgh.build_plan(spec))


@pytest.mark.parametrize("cfg", ["c1", "c2", "c3", "c4"])
def test_singles_cover_every_member_once(cfg):
    plan = bgh.build_plan(wl.window_spec(cfg))
    s = bgh.build_singles(plan).tolist()
    assert all(r1 == -1 for _, _, r1, _ in s)
    seen = [(r, m) for r, m, _, _ in s]
    assert len(seen) == len(set(seen)) and set(seen) == _members(plan)


def test_shared_fraction_separates_mtile_pairs_from_frame_pairs():
    """m-tile pairs (c4) share every KV frame; +-1-frame neighbour pairs (c3) share
    2 of 3 interior frames (2 of 2 / 3 at the clip edges): 0.75 overall."""
    c3 = bgh.build_plan(wl.window_spec("c3"))
    c4 = bgh.build_plan(wl.window_spec("c4"))
    assert bgh.shared_fraction(c4, bgh.build_groups(c4)) == 1.0
    assert bgh.shared_fraction(c3, bgh.build_groups(c3)) == 0.75
    assert bgh.shared_fraction(c3, bgh.build_singles(c3)) == 0.0


def test_grouped_form_pairs_identical_kv_members():
    """Two members per workgroup where pairs share all their KV: c4's m-tile pairs and
    the query tiles of dense attention over the text context qualify at any length;
    c3's neighbouring-frame pairs (0.75 shared) do not."""
    from sr_dit.model import CrossAttentionPlan
    c4 = bgh.build_plan(wl.window_spec("c4"))
    assert bgh.mean_kv_tokens(c4) >= bgh.GROUPED_MIN_KV
    cross = CrossAttentionPlan(21600, 512).plan
    assert bgh.mean_kv_tokens(cross) == 512.0 >= bgh.GROUPED_MIN_KV
    assert bgh.shared_fraction(cross, bgh.build_groups(cross)) == 1.0
    c3 = bgh.build_plan(wl.window_spec("c3"))
    assert bgh.shared_fraction(c3, bgh.build_groups(c3)) < 0.9


@pytest.mark.parametrize("cfg", ["c2", "c3", "c4", "prod", "prod_frame"])
def test_singles_order_heaviest_first_within_runs(cfg):
    """One-member launch table: every (row, m-tile) exactly once, query runs in plan
    order, and within a run the windows by non-increasing cost."""
    from sr_dit import attention as att
    if cfg.startswith("prod"):
        spec = att._BlockGridSpec(f_cur=3, f_kv=12, h=45, w=80, block_t=3, bh=4, bw=4, rh=3, rw=3,
                                  rt=3, streaming=True)
        plan = bgh.build_plan(spec, anchor_mode="frame" if cfg == "prod_frame" else None)
    else:
        plan = bgh.build_plan(wl.window_spec(cfg))
    s = bgh.build_singles(plan)
    p = plan["params"]
    want = {(r, mt) for r in range(p.shape[0])
            for mt in range(-(-bgh._row_lq(plan, p[r].tolist()) // bgh.HIP_BLOCK_M))}
    got = [tuple(x) for x in s[:, :2].tolist()]
    assert len(got) == len(want) and set(got) == want
    assert (s[:, 2] == -1).all()
    cost = bgh._window_cost(plan)[s[:, 0].long()]
    run = p[s[:, 0].long(), 0] if plan["p_stride"] == bgh.P_PLAIN else torch.zeros(len(s))
    assert (run[1:] >= run[:-1]).all()
    same = run[1:] == run[:-1]
    assert (cost[1:][same] <= cost[:-1][same]).all()


@pytest.mark.parametrize("cfg", ["c2", "c3", "c4"])
def test_groups_order_heaviest_first_within_runs(cfg):
    plan = bgh.build_plan(wl.window_spec(cfg))
    g = bgh.build_groups(plan)
    p = plan["params"]
    cost = bgh._window_cost(plan)
    w = cost[g[:, 0].long()] + torch.where(g[:, 2] >= 0, cost[g[:, 2].clamp(min=0).long()], 0)
    run = p[g[:, 0].long(), 0]
    assert (run[1:] >= run[:-1]).all()
    same = run[1:] == run[:-1]
    assert (w[1:][same] <= w[:-1][same]).all()
