"""Streaming loop pieces that run on the CPU: the flow-matching schedule and the
patch embedding restated as a GEMM.

The schedule's closed forms: sigmas = linspace(1, 0, 1001)[:-1] shifted by
s' = 5 s / (1 + 4 s) (scheduler.py:118-131 with shift 5, sigma_min 0,
extra_one_step, as sr_dit_wrapper.py:492-494 builds it), so the warped step
list of causal_inference.py:280-282 for (1000, 750, 500, 250) is
1000 * (1, 15/16, 5/6, 5/8).
"""
import pytest
import torch

from sr_dit.model import SRDiT, SRDiTConfig
from sr_dit.stream import FlowMatchSchedule


def test_warped_step_list_closed_form():
    s = FlowMatchSchedule(shift=5.0)
    got = s.warp([1000, 750, 500, 250])
    want = torch.tensor([1000.0, 937.5, 2500.0 / 3.0, 625.0])
    assert torch.allclose(got.double(), want.double(), rtol=0, atol=1e-3), got
    # one past the end of the table is timestep 0 (the "context" level)
    assert float(s.warp([0])[0]) == 0.0


def test_add_noise_uses_nearest_sigma():
    s = FlowMatchSchedule(shift=5.0)
    x0, nz = torch.zeros(4), torch.ones(4)
    assert torch.allclose(s.add_noise(x0, nz, 937.5), torch.full((4,), 0.9375))
    assert torch.allclose(s.add_noise(x0, nz, 1000.0), torch.ones(4))
    # unshifted schedule: sigma = t / 1000 on the grid
    u = FlowMatchSchedule(shift=1.0)
    assert abs(u.sigma(250.0) - 0.25) < 1e-6


def test_patch_embedding_gemm_equals_conv3d():
    cfg = SRDiTConfig(dim=64, ffn_dim=128, num_heads=2, num_layers=0, in_dim=6, out_dim=6,
                      text_dim=16, text_len=4)
    m = SRDiT(cfg).float()
    g = torch.Generator().manual_seed(0)
    with torch.no_grad():
        m.patch_embedding.weight.copy_(torch.randn(m.patch_embedding.weight.shape, generator=g))
        m.patch_embedding.bias.copy_(torch.randn(m.patch_embedding.bias.shape, generator=g))
        lat = torch.randn(6, 3, 8, 10, generator=g)
        x, grid = m.embed_patches(lat)
        ref = m.patch_embedding(lat.unsqueeze(0))
    assert grid == (3, 4, 5)
    ref = ref.flatten(2).transpose(1, 2)[0]
    assert torch.allclose(x, ref, rtol=1e-5, atol=1e-5)


def test_per_frame_harvest_plan_is_stacked_one_frame_plans():
    """The per-frame LQ-anchor harvest runs LR frame i as a one-frame sample with no
    cache (causal_inference.py:455-500).  The reference's rule for that sample
    (f_cur = f_kv = 1, block_t = 3, not streaming, rt clamped to 0;
    attention.py:1583-1603) gives the oracle's one-frame rows; shifted to frame i
    and stacked, they must equal, row for row, the plan of the single three-frame
    harvest forward the loop runs instead (``SRDiT.harvest_geometry``)."""
    import numpy as np
    from oracle import blockgrid as obg

    cfg = SRDiTConfig(dim=64, ffn_dim=128, num_heads=2, num_layers=0, in_dim=4, out_dim=4,
                      text_dim=16, text_len=4)
    m = SRDiT(cfg)
    for (h, w) in ((45, 80), (16, 24)):
        geom = m.harvest_geometry(3, h, w, 4, "cpu", per_frame=True, chunk=3,
                                  block_hw=(4, 4), block_radius_hw=(3, 3))
        got = geom["plan"]["params"].numpy()
        one = np.asarray(obg.params_rows(obg.Geometry(
            f_cur=1, f_kv=1, h=h, w=w, block_t=3, bh=4, bw=4, rh=3, rw=3, rt=0,
            streaming=False))[0], dtype=np.int64)
        want = []
        for t in range(3):
            r = one.copy()
            r[:, 0] += t   # q_t0
            r[:, 6] += t   # kv_t0
            want.append(r)
        want = np.concatenate(want)
        assert got.shape == want.shape
        assert (got == want).all()
        # no row lets a frame see another frame
        assert (got[:, 1] == 1).all() and (got[:, 7] == 1).all() and (got[:, 0] == got[:, 6]).all()


def test_whole_chunk_harvest_plan_sees_the_chunk():
    """per_frame=False: one three-frame sample without a cache; every window sees all
    three frames (the non-streaming rule with block_t = 3, rt = 0)."""
    import numpy as np
    from oracle import blockgrid as obg

    cfg = SRDiTConfig(dim=64, ffn_dim=128, num_heads=2, num_layers=0, in_dim=4, out_dim=4,
                      text_dim=16, text_len=4)
    geom = SRDiT(cfg).harvest_geometry(3, 16, 24, 4, "cpu", per_frame=False, chunk=3,
                                       block_hw=(4, 4), block_radius_hw=(3, 3))
    got = geom["plan"]["params"].numpy()
    want = np.asarray(obg.params_rows(obg.Geometry(
        f_cur=3, f_kv=3, h=16, w=24, block_t=3, bh=4, bw=4, rh=3, rw=3, rt=0,
        streaming=False))[0], dtype=np.int64)
    assert (got == want).all()
    assert (got[:, 6] == 0).all() and (got[:, 7] == 3).all()


def test_streaming_refiner_anchor_arguments():
    from sr_dit.stream import StreamingRefiner

    cfg = SRDiTConfig(dim=64, ffn_dim=128, num_heads=2, num_layers=0, in_dim=4, out_dim=4,
                      text_dim=16, text_len=4)
    m = SRDiT(cfg)
    ctx = torch.zeros(4, 16)
    with pytest.raises(ValueError):
        StreamingRefiner(m, 8, 8, ctx, anchor="window", device="cpu")
    with pytest.raises(ValueError):
        StreamingRefiner(m, 8, 8, ctx, anchor="frame", anchor_mode="q", device="cpu")


def test_rope_table_hw_stride_samples_the_hr_positions():
    """The native anchor's harvest RoPE (models.py:1761-1785): grid row i at HR row
    i*s_h, column j at HR column j*s_w; the temporal axis unchanged."""
    from sr_dit.model import rope_table
    cfg = SRDiTConfig()
    full = rope_table(cfg, 2, 6, 12, t_offset=5, device="cpu").reshape(2, 6, 12, -1)
    thin = rope_table(cfg, 2, 3, 4, t_offset=5, device="cpu", hw_stride=(2, 3)).reshape(2, 3, 4, -1)
    assert torch.equal(thin, full[:, ::2, ::3])
    with pytest.raises(ValueError):
        rope_table(cfg, 1, 2, 2, device="cpu", hw_stride=(0, 1))


@pytest.mark.parametrize("mode", ["frame", "chunk"])
def test_native_anchor_stream_plan_matches_oracle(mode):
    """Anchored steps with the native anchor grid: the plan's rows are the oracle's
    for the same geometry with anchor_hw = the LQ token grid."""
    import numpy as np
    from oracle import blockgrid as obg
    cfg = SRDiTConfig(dim=64, ffn_dim=128, num_heads=2, num_layers=0, in_dim=4, out_dim=4,
                      text_dim=16, text_len=4)
    geom = SRDiT(cfg).stream_geometry(3, 16, 24, 4, "cpu", cached=6, chunk=3, block_hw=(4, 4),
                                      block_radius_hw=(2, 2), anchor=mode, anchor_hw=(8, 12))
    plan = geom["plan"]
    rows, block_m, m_tiles, hr_base, p_stride = obg.params_rows(obg.Geometry(
        f_cur=3, f_kv=9, h=16, w=24, block_t=3, bh=4, bw=4, rh=2, rw=2, rt=2, streaming=True,
        anchor_hw=(8, 12)), mode)
    assert np.array_equal(plan["params"].numpy(), np.asarray(rows, dtype=np.int64))
    assert plan["hr_base"] == hr_base == 3 * 8 * 12 and plan["p_stride"] == p_stride
