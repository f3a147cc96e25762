"""Planner parity (CPU): product planner and oracle vs the reference's own tables.

The golden vectors in tests/golden/plans.json were written by the reference's
build_plan / _BlockGridSpec (tests/golden/make_golden.py).  The visibility a
table implies is further checked token by token against the oracle's
block-distance rule, a formulation independent of the interval arithmetic.
"""
import numpy as np
import pytest
import torch

from sr_dit import attention as att
from sr_dit import blockgrid_hip as bgh
from oracle import blockgrid as obg


def _spec(case):
    kw = dict(case["spec"])
    if "anchor_hw" in kw and kw["anchor_hw"] is not None:
        kw["anchor_hw"] = tuple(kw["anchor_hw"])
    return att._BlockGridSpec(**kw, sym_rt=case["sym_rt"])


def _geom(case):
    kw = dict(case["spec"])
    if kw.get("anchor_hw") is not None:
        kw["anchor_hw"] = tuple(kw["anchor_hw"])
    return obg.Geometry(**kw, sym_rt=case["sym_rt"])


def test_golden_cases_present(golden_plans):
    names = {c["name"] for c in golden_plans}
    for must in ("c1_3x16x16", "c2_6x34x60", "c3_6x45x80", "c4_ar_2of6x45x80",
                 "prod_anchor_frame_fkv12_45x80", "prod_anchor_chunk_fkv12_45x80"):
        assert must in names


@pytest.mark.parametrize("idx", range(21))
def test_product_plan_bit_exact(golden_plans, idx):
    case = golden_plans[idx]
    spec = _spec(case)
    assert [list(r) for r in spec.temporal_runs()] == case["temporal_runs"]
    plan = bgh.build_plan(spec, anchor_mode=case["anchor_mode"])
    assert plan["params"].dtype == torch.int32
    assert plan["params"].tolist() == case["params"]
    for key in ("n_w", "block_m", "m_tiles", "block_n", "hr_base", "p_stride"):
        assert plan[key] == case[key], key


@pytest.mark.parametrize("idx", range(21))
def test_oracle_plan_bit_exact(golden_plans, idx):
    case = golden_plans[idx]
    g = _geom(case)
    assert [list(r) for r in obg.temporal_runs(g)] == case["temporal_runs"]
    rows, block_m, m_tiles, hr_base, p_stride = obg.params_rows(g, case["anchor_mode"])
    assert rows == case["params"]
    assert (block_m, m_tiles, hr_base, p_stride) == (
        case["block_m"], case["m_tiles"], case["hr_base"], case["p_stride"])


TINY = ["c1_3x16x16", "tiny_sym_4x13x11", "tiny_sym_r2_3x9x10", "tiny_anchor_frame_2of4x8x12",
        "tiny_anchor_chunk_2of4x8x12", "tiny_cache_sym_2of4x9x9", "legacy_parallel_6f_13x11",
        "hist_parallel_6f_20x24", "native_anchor_chunk_12x16"]


@pytest.mark.parametrize("name", TINY)
def test_table_visibility_matches_token_rule(golden_plans, name):
    """Union of the table's window cuboids == the per-token block-distance rule."""
    case = next(c for c in golden_plans if c["name"] == name)
    g = _geom(case)
    dense = obg.dense_mask(g, case["anchor_mode"])
    from_rows = obg.rows_mask(case["params"], g, case["anchor_mode"], kv_total=dense.shape[1])
    assert from_rows.shape == dense.shape
    assert np.array_equal(from_rows, dense)
    # the oracle's gather windows give the same set
    gm = np.zeros_like(dense)
    seen = np.zeros(dense.shape[0], dtype=int)
    for q_idx, kv_idx in obg.windows(g, case["anchor_mode"]):
        gm[np.ix_(q_idx, kv_idx)] = True
        seen[q_idx] += 1
    assert np.array_equal(gm, dense)
    # query windows partition the tokens (each exactly once; frame-aligned
    # anchors split a window into one pass per frame, still once per token)
    assert (seen == 1).all()


def test_temporal_rule_negative_control(golden_plans):
    """A plausible mistake (one frame too many on the left) must break the match."""
    case = next(c for c in golden_plans if c["name"] == "tiny_sym_4x13x11")
    g = _geom(case)
    dense = obg.dense_mask(g)
    bad = [list(r) for r in case["params"]]
    for r in bad:                                   # widen kv span by one frame
        if r[6] > 0:
            r[6] -= 1
            r[7] += 1
    assert not np.array_equal(obg.rows_mask(bad, g, kv_total=dense.shape[1]), dense)


def test_partition_check_raises():
    spec = att._BlockGridSpec(f_cur=5, f_kv=5, h=8, w=8, block_t=3, bh=4, bw=4, rh=1, rw=1, rt=1)
    with pytest.raises(ValueError):
        spec.temporal_runs()


def test_anchor_stride_contract():
    with pytest.raises(ValueError):
        att._anchor_grid_stride(45, 80, 4, 4, (15, 40))      # stride 3 does not divide bh
    with pytest.raises(ValueError):
        att._anchor_grid_stride(45, 80, 4, 4, (7, 40))       # does not divide h
    assert att._anchor_grid_stride(44, 80, 4, 4, (22, 40)) == (2, 2)


def test_plan_cache_and_keys():
    bgh.clear_plan_cache()
    spec = att._BlockGridSpec(f_cur=3, f_kv=3, h=16, w=16, block_t=1, bh=8, bw=8, rh=1, rw=1,
                              sym_rt=1)
    p1 = bgh.cached_plan(spec)
    p2 = bgh.cached_plan(spec)
    assert p1 is p2
    assert bgh.hip_kernel_keys(p1, d=128) == {("plain", 64, 128)}
    assert bgh.kernel_m_tiles(p1) == 1


def test_kernel_m_tiles_cover_largest_window(golden_plans):
    for case in golden_plans:
        plan = bgh.build_plan(_spec(case), anchor_mode=case["anchor_mode"])
        rows = np.array(case["params"])
        if case["p_stride"] == 17:
            lq = rows[:, 10] * rows[:, 2] * rows[:, 3]
        else:
            lq = rows[:, 1] * rows[:, 4] * rows[:, 5]
        assert bgh.kernel_m_tiles(plan) * bgh.HIP_BLOCK_M >= lq.max()


def test_launch_orders_are_permutations(golden_plans):
    case = next(c for c in golden_plans if c["name"] == "c3_6x45x80")
    plan = bgh.build_plan(_spec(case))
    order = bgh.launch_order(plan).tolist()
    assert order == list(range(plan["n_w"]))
    lpt = bgh.longest_first_order(plan).tolist()
    assert sorted(lpt) == list(range(plan["n_w"]))
    cost = bgh._window_cost(plan)
    costs = [int(cost[i]) for i in lpt]
    assert costs == sorted(costs, reverse=True)


def test_useful_flops_factorise():
    """Sum over windows of Lq*Lkv factorises over the three axes (no anchor)."""
    for (f, h, w) in ((6, 45, 80), (6, 34, 60), (3, 16, 16)):
        g = obg.Geometry(f_cur=f, f_kv=f, h=h, w=w, block_t=1, bh=8, bw=8, rh=1, rw=1, sym_rt=1)
        st = sum((q1 - q0) * (k1 - k0) for (q0, q1, k0, k1) in obg.temporal_runs(g))
        sh = sum(qL * kL for (_, qL, _, kL) in obg.axis_blocks(h, 8, 1))
        sw = sum(qL * kL for (_, qL, _, kL) in obg.axis_blocks(w, 8, 1))
        assert obg.useful_flops(g) == 4 * 128 * 24 * st * sh * sw
    g = obg.Geometry(f_cur=6, f_kv=6, h=45, w=80, block_t=1, bh=8, bw=8, rh=1, rw=1, sym_rt=1)
    assert abs(obg.useful_flops(g) / 330.13e9 - 1) < 1e-4


def test_op_needs_block_t_or_chunk_frames():
    """attention.py:1575 takes int(None) when neither is given: a TypeError."""
    import torch
    from sr_dit import attention as att
    q = torch.zeros(1, 768, 2, 128, dtype=torch.bfloat16)
    grid = torch.tensor([[3, 16, 16]])
    with pytest.raises(TypeError):
        att.mask_free_window_attention(q, q, q, grid, block_hw=(8, 8), block_radius_hw=(1, 1))
