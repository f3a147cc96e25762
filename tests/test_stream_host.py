"""Streaming loop pieces that run on the CPU: the flow-matching schedule and the
patch embedding restated as a GEMM.

The schedule's closed forms: sigmas = linspace(1, 0, 1001)[:-1] shifted by
s' = 5 s / (1 + 4 s) (scheduler.py:118-131 with shift 5, sigma_min 0,
extra_one_step, as sr_dit_wrapper.py:492-494 builds it), so the warped step
list of causal_inference.py:280-282 for (1000, 750, 500, 250) is
1000 * (1, 15/16, 5/6, 5/8).
"""
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
