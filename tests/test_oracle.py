"""Oracle self-checks (CPU): pin the attention oracle before trusting it.

* the window oracle equals brute-force dense masked attention (float64) on tiny
  grids, anchors included, where the mask comes from the per-token rule;
* a single window covering the whole grid is plain softmax attention;
* the torch gather restatement (the CPU baseline) equals the numpy oracle;
* negative controls: an all-zero output and a uniform-average-of-V output PASS
  the bare max/mean-abs tolerance at the benchmark distribution but FAIL the
  strengthened suite; a mask error (one extra frame) fails it too.
"""
import numpy as np
import pytest
import torch

from oracle import blockgrid as obg
from oracle import gather_torch as ogt

from parity import metrics, passes_attention, passes_abs_bounds_only


def _rand(shape, seed, scale=1.0):
    g = torch.Generator("cpu").manual_seed(seed)
    return (torch.randn(*shape, generator=g, dtype=torch.float32) * scale).numpy()


def _inputs(g, anchor_mode, n=2, d=16, seed=0, scale=None):
    scale = d ** -0.5 if scale is None else scale
    L = g.h * g.w
    a_h, a_w = g.anchor_grid
    n_a = g.f_cur * a_h * a_w if anchor_mode else 0
    q = _rand((g.f_cur * L, n, d), seed, scale)
    k = _rand((n_a + g.f_kv * L, n, d), seed + 1, scale)
    v = _rand((n_a + g.f_kv * L, n, d), seed + 2, scale)
    return q, k, v


GEOMS = [
    (obg.Geometry(f_cur=3, f_kv=3, h=8, w=8, block_t=1, bh=4, bw=4, rh=1, rw=1, sym_rt=1), None),
    (obg.Geometry(f_cur=4, f_kv=4, h=13, w=11, block_t=1, bh=4, bw=4, rh=1, rw=1, sym_rt=1), None),
    (obg.Geometry(f_cur=2, f_kv=4, h=9, w=9, block_t=1, bh=4, bw=4, rh=1, rw=1, streaming=True,
                  sym_rt=1), None),
    (obg.Geometry(f_cur=2, f_kv=6, h=10, w=12, block_t=3, bh=4, bw=4, rh=1, rw=1, rt=1,
                  streaming=True), None),
    (obg.Geometry(f_cur=6, f_kv=6, h=13, w=11, block_t=3, bh=4, bw=4, rh=1, rw=1, rt=1), None),
    (obg.Geometry(f_cur=2, f_kv=4, h=8, w=12, block_t=2, bh=4, bw=4, rh=1, rw=1, rt=1,
                  streaming=True), "frame"),
    (obg.Geometry(f_cur=2, f_kv=4, h=8, w=12, block_t=2, bh=4, bw=4, rh=1, rw=1, rt=1,
                  streaming=True), "chunk"),
    (obg.Geometry(f_cur=2, f_kv=4, h=12, w=16, block_t=2, bh=4, bw=4, rh=1, rw=2, rt=1,
                  streaming=True, anchor_hw=(6, 8)), "frame"),
]


@pytest.mark.parametrize("gi", range(len(GEOMS)))
@pytest.mark.parametrize("temp", [1.0, 8.0])
def test_window_oracle_equals_dense_masked(gi, temp):
    g, mode = GEOMS[gi]
    q, k, v = _inputs(g, mode, scale=16 ** -0.5 * temp)
    out = obg.window_attention(q, k, v, g, mode)
    ref = obg.dense_attention(q, k, v, obg.dense_mask(g, mode))
    np.testing.assert_allclose(out, ref, rtol=1e-10, atol=1e-12)


def test_single_window_is_plain_attention():
    """One window covering the whole grid (radius >= block count) == softmax(QK^T)V."""
    g = obg.Geometry(f_cur=2, f_kv=2, h=8, w=8, block_t=1, bh=8, bw=8, rh=1, rw=1, sym_rt=5)
    q, k, v = _inputs(g, None, d=16, scale=0.5)
    out = obg.window_attention(q, k, v, g)
    s = np.einsum("qnd,knd->nqk", q.astype(np.float64), k.astype(np.float64)) / 4.0
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    ref = np.einsum("nqk,knd->qnd", p, v.astype(np.float64))
    np.testing.assert_allclose(out, ref, rtol=1e-10, atol=1e-12)
    tq = torch.from_numpy(q).transpose(0, 1)[None].double()
    tk = torch.from_numpy(k).transpose(0, 1)[None].double()
    tv = torch.from_numpy(v).transpose(0, 1)[None].double()
    sdpa = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv)[0].transpose(0, 1).numpy()
    np.testing.assert_allclose(out, sdpa, rtol=1e-9, atol=1e-12)


@pytest.mark.parametrize("gi", [0, 3, 5, 6])
def test_gather_torch_equals_oracle(gi):
    g, mode = GEOMS[gi]
    q, k, v = _inputs(g, mode, scale=0.5)
    plan = ogt.GatherPlan(g, mode)
    out = ogt.gather_attend(plan, torch.from_numpy(q).double(), torch.from_numpy(k).double(),
                            torch.from_numpy(v).double()).numpy()
    ref = obg.window_attention(q, k, v, g, mode)
    np.testing.assert_allclose(out, ref, rtol=1e-9, atol=1e-12)
    out_c = ogt.gather_attend(plan, torch.from_numpy(q).double(), torch.from_numpy(k).double(),
                              torch.from_numpy(v).double(), win_chunk=3).numpy()
    np.testing.assert_allclose(out_c, ref, rtol=1e-9, atol=1e-12)


def test_negative_controls_fail_strengthened_suite():
    """At the benchmark distribution, broken kernels pass max/mean-abs but not the suite."""
    g = obg.Geometry(f_cur=3, f_kv=3, h=24, w=24, block_t=1, bh=8, bw=8, rh=1, rw=1, sym_rt=1)
    q, k, v = _inputs(g, None, n=2, d=128)
    ref = obg.window_attention(q, k, v, g)
    zeros = np.zeros_like(ref)
    assert metrics(zeros, ref)["max_abs"] <= 2e-2        # max-abs alone cannot see it
    assert not passes_attention(zeros, ref)
    # uniform average of V over each window (ignores Q.K)
    uni = np.zeros_like(ref)
    for q_idx, kv_idx in obg.windows(g):
        uni[q_idx] = v[kv_idx].astype(np.float64).mean(0)[None]
    assert passes_abs_bounds_only(uni, ref)
    assert not passes_attention(uni, ref), metrics(uni, ref)
    # a mask mistake: every window sees one more frame than it should
    g_bad = obg.Geometry(f_cur=3, f_kv=3, h=24, w=24, block_t=1, bh=8, bw=8, rh=1, rw=1, sym_rt=2)
    bad = obg.window_attention(q, k, v, g_bad)
    assert not passes_attention(bad, ref), metrics(bad, ref)
    # the oracle itself passes, rounded to bf16 (what a correct bf16 kernel can reach)
    ref_bf16 = torch.from_numpy(ref).to(torch.bfloat16).double().numpy()
    assert passes_attention(ref_bf16, ref), metrics(ref_bf16, ref)
