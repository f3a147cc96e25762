"""The forward's ends (models.py:1827-1875 embeddings, :1357-1384 Head,
:2234-2257 unpatchify, :67-77 sinusoidal_embedding_1d) against independent
restatements: the patch embedding against torch's Conv3d on the CPU, the time
embedding against the sinusoid written out with math.cos/sin in float64, the
head against a float64 LayerNorm/modulation/Linear, unpatchify against an
explicit index loop.  A zero-layer SRDiT holds the embedding and head weights.
Each ``check_*`` takes the device the model runs on (the references stay on the
CPU); tests/test_forward_ends_gpu.py runs them on the GPU.
"""
import math

import torch
import torch.nn.functional as F

from sr_dit import model as mdl

CFG = mdl.SRDiTConfig(dim=256, ffn_dim=512, num_heads=2, num_layers=0, freq_dim=64,
                      text_dim=96, text_len=16, in_dim=8, out_dim=8)


def _model(dev="cpu", dtype=torch.bfloat16):
    m = mdl.SRDiT(CFG).to(dtype)
    mdl.init_weights(m, std=0.05, seed=1)
    with torch.no_grad():  # nonzero biases, so a dropped bias fails
        g = torch.Generator("cpu").manual_seed(9)
        for mod in m.modules():
            if isinstance(mod, (torch.nn.Linear, torch.nn.Conv3d)) and mod.bias is not None:
                mod.bias.copy_(torch.randn(mod.bias.shape, generator=g) * 0.1)
    return m.to(dev)


def _w(t):
    return t.detach().double().cpu()


def check_patch_embedding_is_the_conv3d(dev="cpu"):
    m = _model(dev)
    g = torch.Generator("cpu").manual_seed(0)
    lat = torch.randn(CFG.in_dim, 3, 10, 12, generator=g)
    x, grid = m.embed_patches(lat.to(dev))
    assert grid == (3, 5, 6)
    conv = F.conv3d(lat.to(torch.bfloat16).double().unsqueeze(0), _w(m.patch_embedding.weight),
                    _w(m.patch_embedding.bias), stride=CFG.patch_size)  # [1, dim, 3, 5, 6]
    ref = conv.flatten(2).transpose(1, 2)[0]                           # tokens in (f, h, w) order
    assert x.shape == ref.shape and x.dtype == torch.bfloat16
    err = (x.double().cpu() - ref).abs()
    assert err.max().item() <= 2 ** -7 * ref.abs().max().item() + 1e-3


def check_sinusoidal_embedding_closed_form(dev="cpu"):
    pos = torch.tensor([0.0, 1.0, 625.0, 937.5, 999.0], device=dev)
    got = mdl.sinusoidal_embedding_1d(CFG.freq_dim, pos).cpu()
    half = CFG.freq_dim // 2
    for i, p in enumerate(pos.tolist()):
        for j in (0, 1, half // 2, half - 1):
            ang = p * 10000.0 ** (-j / half)
            assert abs(float(got[i, j]) - math.cos(ang)) <= 1e-12
            assert abs(float(got[i, half + j]) - math.sin(ang)) <= 1e-12


def _sinusoid(t, half):
    return torch.tensor([[math.cos(t * 10000.0 ** (-j / half)) for j in range(half)]
                         + [math.sin(t * 10000.0 ** (-j / half)) for j in range(half)]],
                        dtype=torch.float64)


def _lin(mod, x):
    return x @ _w(mod.weight).T + _w(mod.bias)


def check_time_embedding_fp32_mlp(dev="cpu"):
    m = _model(dev)
    e, e0 = m.time_embed(torch.tensor([625.0], device=dev))
    assert e.dtype == torch.float32 and e0.shape == (1, 6, CFG.dim)
    te, tp = m.time_embedding, m.time_projection
    e_ref = _lin(te[2], F.silu(_lin(te[0], _sinusoid(625.0, CFG.freq_dim // 2))))
    e0_ref = _lin(tp[1], F.silu(e_ref)).view(1, 6, CFG.dim)
    assert torch.allclose(e.double().cpu(), e_ref, rtol=1e-4, atol=1e-5)
    assert torch.allclose(e0.double().cpu(), e0_ref, rtol=1e-4, atol=1e-5)


def check_text_embedding_pads_then_mlp(dev="cpu"):
    m = _model(dev)
    g = torch.Generator("cpu").manual_seed(3)
    raw = torch.randn(11, CFG.text_dim, generator=g).to(torch.bfloat16)
    got = m.embed_text(raw.to(dev)).double().cpu()
    assert got.shape == (CFG.text_len, CFG.dim)
    padded = torch.cat([raw.double(), torch.zeros(CFG.text_len - 11, CFG.text_dim, dtype=torch.float64)])
    l0, l2 = m.text_embedding[0], m.text_embedding[2]
    bf = lambda t: t.to(torch.bfloat16).double()  # noqa: E731  (bf16 activations between the Linears)
    ref = _lin(l2, bf(F.gelu(bf(_lin(l0, padded)), approximate="tanh")))
    assert (got - ref).abs().max().item() <= 2 ** -6 * ref.abs().max().item()
    # the padding rows see only the first Linear's bias
    pad = _lin(l2, bf(F.gelu(bf(_w(l0.bias)), approximate="tanh")))
    assert (got[11:] - pad).abs().max().item() <= 2 ** -6 * pad.abs().max().item()


def check_head_fp32(dev="cpu"):
    m = _model(dev)
    g = torch.Generator("cpu").manual_seed(4)
    x = torch.randn(30, CFG.dim, generator=g).to(torch.bfloat16)
    e = torch.randn(1, CFG.dim, generator=g)
    got = m.head(x.to(dev), e.to(dev))
    assert got.dtype == torch.float32 and got.shape == (30, math.prod(CFG.patch_size) * CFG.out_dim)
    xd = x.double()
    mu = xd.mean(-1, keepdim=True)
    var = ((xd - mu) ** 2).mean(-1, keepdim=True)
    # the norm computes in fp32 and returns x's dtype (models.py:443-503)
    ln = ((xd - mu) / torch.sqrt(var + CFG.eps)).to(torch.bfloat16).double()
    mod = _w(m.head.modulation) + e.double().unsqueeze(1)   # [1, 2, dim]: shift, scale
    z = ln * (1 + mod[:, 1]) + mod[:, 0]
    ref = _lin(m.head.head, z)
    assert torch.allclose(got.double().cpu(), ref, rtol=1e-3, atol=1e-3 * ref.abs().max().item())


def check_unpatchify_index_map(dev="cpu"):
    f, h, w = 2, 3, 4
    pt, ph, pw = CFG.patch_size
    c = CFG.out_dim
    x = torch.arange(f * h * w * pt * ph * pw * c, dtype=torch.float32).view(f * h * w, -1)
    out = mdl.unpatchify(x.to(dev), (f, h, w), CFG.patch_size, c).cpu()
    assert out.shape == (c, f * pt, h * ph, w * pw)
    for ff in range(f):
        for hh in range(h):
            for ww in range(w):
                tok = (ff * h + hh) * w + ww
                for p in range(pt):
                    for q in range(ph):
                        for r in range(pw):
                            for cc in range(c):
                                col = ((p * ph + q) * pw + r) * c + cc
                                assert out[cc, ff * pt + p, hh * ph + q, ww * pw + r] == x[tok, col]


def test_patch_embedding_is_the_conv3d():
    check_patch_embedding_is_the_conv3d()


def test_sinusoidal_embedding_closed_form():
    check_sinusoidal_embedding_closed_form()


def test_time_embedding_fp32_mlp():
    check_time_embedding_fp32_mlp()


def test_text_embedding_pads_then_mlp():
    check_text_embedding_pads_then_mlp()


def test_head_fp32():
    check_head_fp32()


def test_unpatchify_index_map():
    check_unpatchify_index_map()
