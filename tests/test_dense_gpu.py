"""The dense Linears at the forward's ends (csrc/dense.hip) against float64
references with torch's rounding points (models.py:1551-1552 patch embedding,
:1553-1556 / :1860-1866 text embedding, :1845-1849 time MLP, :1374-1384 head).

Bounds: an fp32 accumulation over K terms errs by at most K * 2^-24 * sum|a w|
(recursive summation; the kernels' tree orders do better), and each rounding
to bf16 by half an ulp (2^-9 relative).  A wrong k pairing, a dropped slice of
k or a missing bias moves results by far more than these bounds.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from sr_dit import _lib

pytestmark = pytest.mark.gpu

U32 = 2.0 ** -24


def _bf(t):
    return t.to(torch.bfloat16).double()


def _gelu64(x):
    return 0.5 * x * (1 + torch.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))


@pytest.mark.parametrize("M,N,K,gelu", [(1000, 384, 64, False), (512, 256, 4096, True),
                                        (3000, 3072, 64, False), (2100, 4096, 128, True),
                                        (77, 200, 48, False), (130, 96, 32, True),
                                        (50, 37, 32, True), (300, 1027, 64, False)])
def test_bf16_linear_matches_float64(M, N, K, gelu):
    print(f"[case] bf16_linear M={M} N={N} K={K} gelu={gelu}", flush=True)
    g = torch.Generator("cpu").manual_seed(M + N + K)
    a = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) / math.sqrt(K)).to(torch.bfloat16)
    b = (torch.randn(N, generator=g) * 0.3).to(torch.bfloat16)
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    _lib.bf16_linear(a.cuda(), w.cuda(), b.cuda(), out, gelu=gelu)
    torch.cuda.synchronize()
    acc = a.double() @ w.double().T + b.double()
    slack = K * U32 * (a.double().abs() @ w.double().abs().T)
    got = out.double().cpu()
    if not gelu:
        assert ((got - acc).abs() <= 2 ** -8 * acc.abs() + slack * 1.01).all()
        assert (got == _bf(acc)).double().mean() > 0.97
    else:
        # gelu acts on the rounded linear output and rounds again; |gelu'| <= 1.13.
        # Where the fp32 sum sits at a rounding boundary the two roundings of the
        # linear output may pick neighbours: one bf16 ulp (2^-7 relative) apart.
        lin = _bf(acc)
        ref = _bf(_gelu64(lin))
        tol = 2 ** -7 * ref.abs() + 1.13 * (2 ** -7 * lin.abs() + slack) + 1e-6
        assert ((got - ref).abs() <= tol).all()
        # most outputs agree bit for bit with the float64 chain
        assert (got == ref).double().mean() > 0.97
    # a planted mistake (bias dropped) fails the same bound
    if not gelu:
        assert not ((got - (acc - b.double())).abs() <= 2 ** -8 * acc.abs() + slack).all()


@pytest.mark.parametrize("wdt", [torch.bfloat16, torch.float32], ids=["w_bf16", "w_fp32"])
@pytest.mark.parametrize("M,N,K", [(1000, 64, 3072), (70, 40, 80), (33, 13, 48)])
def test_linear_f32_modulated_matches_float64(M, N, K, wdt):
    print(f"[case] linear_f32_modulated M={M} N={N} K={K} w={wdt}", flush=True)
    g = torch.Generator("cpu").manual_seed(M * 7 + K)
    a = torch.randn(M, K, generator=g).to(torch.bfloat16)
    s1 = 1 + torch.randn(K, generator=g) * 0.1
    m0 = torch.randn(K, generator=g) * 0.1
    w = (torch.randn(N, K, generator=g) / math.sqrt(K)).to(wdt)
    b = (torch.randn(N, generator=g) * 0.3).to(wdt)
    out = torch.empty(M, N, dtype=torch.float32, device="cuda")
    _lib.linear_f32_modulated(a.cuda(), s1.cuda(), m0.cuda(), w.cuda(), b.cuda(), out)
    torch.cuda.synchronize()
    # xin rounds after the product and after the sum, in fp32 (torch's two kernels)
    xin = (a.float() * s1).float() + m0
    acc = xin.double() @ w.double().T + b.double()
    slack = (K + 1) * U32 * (xin.double().abs() @ w.double().abs().T + b.double().abs())
    got = out.double().cpu()
    assert ((got - acc).abs() <= slack).all()
    # an fma-contracted modulation or a missing shift fails: check the shift
    bad = (a.float() * s1) @ w.float().T + b.float()
    assert not ((got - bad.double()).abs() <= slack).all()


@pytest.mark.parametrize("wdt", [torch.bfloat16, torch.float32], ids=["w_bf16", "w_fp32"])
@pytest.mark.parametrize("M,N,K", [(1, 18432, 3072), (3, 100, 264), (1, 3072, 256)])
def test_gemv_f32_matches_float64(M, N, K, wdt):
    print(f"[case] gemv_f32 M={M} N={N} K={K} w={wdt}", flush=True)
    g = torch.Generator("cpu").manual_seed(N + K)
    x = torch.randn(M, K, generator=g)
    w = (torch.randn(N, K, generator=g) / math.sqrt(K)).to(wdt)
    b = (torch.randn(N, generator=g) * 0.3).to(wdt)
    out = torch.empty(M, N, dtype=torch.float32, device="cuda")
    _lib.gemv_f32(x.cuda(), w.cuda(), b.cuda(), out)
    torch.cuda.synchronize()
    acc = x.double() @ w.double().T + b.double()
    slack = (K + 1) * U32 * (x.double().abs() @ w.double().abs().T + b.double().abs())
    assert ((out.double().cpu() - acc).abs() <= slack).all()


def test_head_and_embeddings_run_without_torch_gemms():
    """The refiner's ends on the GPU launch only this library's GEMMs: a profile of
    the head, time MLP, patch and text embeddings shows no rocBLAS/hipBLASLt kernel."""
    from torch.profiler import ProfilerActivity, profile

    from sr_dit import model as mdl
    cfg = mdl.SRDiTConfig(dim=256, ffn_dim=512, num_heads=2, num_layers=0, freq_dim=64,
                          text_dim=96, text_len=16, in_dim=8, out_dim=8)
    m = mdl.SRDiT(cfg).to(torch.bfloat16).cuda()
    mdl.init_weights(m, seed=2)
    lat = torch.randn(cfg.in_dim, 3, 8, 8, device="cuda")
    raw = torch.randn(11, cfg.text_dim, device="cuda").to(torch.bfloat16)
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        x, _ = m.embed_patches(lat)
        e, e0 = m.time_embed(torch.tensor([500.0], device="cuda"))
        m.embed_text(raw)
        m.head(x, e)
        torch.cuda.synchronize()
    names = [ev.name for ev in prof.events() if ev.device_type == torch.autograd.DeviceType.CUDA]
    assert any("bf16_linear" in n for n in names), names
    assert not [n for n in names if n.startswith("Cijk") or "gemm" in n.lower()], names
