"""The refiner block stack (fp8 linears, window and cross attention on the HIP
kernels) against a float32 torch restatement of the same computation.

The restatement follows the reference block (models.py:1304-1351, :1256-1262),
WanSelfAttention's window path (:583-676) with complex128 RoPE (:173-214),
WanT2VCrossAttention (:1042-1062) and Fp8Linear (fp8_linear.py:282-297): the
activation is quantised with the reference formula, the product is the fp32
dequantised matmul, window attention is dense fp32 attention under the
oracle's block mask.  bf16 roundings sit at the same points as in the
reference.  Small sizes: two blocks, dim 256, 2 heads of 128, a 3x16x16 grid.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import blockgrid as obg
from parity import rope_table_ref
from sr_dit import model as mdl

pytestmark = pytest.mark.gpu

DEV = "cuda"
F8 = torch.float8_e4m3fn


def _ref_linear(lin, x):
    """Fp8Linear.forward restated: reference quantiser + fp32 dequantised product."""
    x2 = x.reshape(-1, lin.in_features)
    if lin.scaling == "rowwise":
        amax = x2.abs().amax(dim=-1, keepdim=True).float()
        xs = (amax / 448.0).clamp_min(1e-12)
        ws = lin.weight_scale.reshape(1, -1)
    else:
        xs = (x2.abs().amax().float() / 448.0).clamp_min(1e-12)
        ws = lin.weight_scale.reshape(1, 1)
    xq = (x2.float() / xs).clamp(-448, 448).to(F8)
    out = (xq.float() @ lin.weight_fp8.float().T) * xs * ws
    if lin.bias is not None:
        out = out + lin.bias.float()
    return out.to(torch.bfloat16).reshape(*x.shape[:-1], lin.out_features)


def _ref_rope(x, grid, cfg):
    """rope_apply (models.py:173-214) in complex128, on a phasor table built in the
    test from the formulas (parity.rope_table_ref), not from the product's."""
    f, h, w = grid
    s, n, d = x.shape
    c = d // 2
    fr = rope_table_ref(f, h, w, d, cfg.rope_theta, device=x.device)
    xc = torch.view_as_complex(x.to(torch.float64).reshape(s, n, c, 2))
    return torch.view_as_real(xc * fr).flatten(2).to(x.dtype)


def _ref_attention(q, k, v, mask=None):
    """fp32 softmax attention, [s, n, d] layout, P rounded to bf16 before P.V."""
    qf, kf, vf = (t.float().transpose(0, 1) for t in (q, k, v))
    sc = (qf @ kf.transpose(1, 2)) * q.shape[-1] ** -0.5
    if mask is not None:
        sc = sc.masked_fill(~mask, float("-inf"))
    p = torch.softmax(sc, dim=-1)
    return (p.to(torch.bfloat16).float() @ vf).transpose(0, 1).to(torch.bfloat16)


def _jitter(t, gen):
    """Move every element of a bf16 tensor by -1, 0 or +1 unit in the last place, at
    random: the size of a difference in where a bf16 rounding happens."""
    step = torch.randint(-1, 2, t.shape, generator=gen, dtype=torch.int8).to(t.device, torch.int16)
    step = step * (t != 0)  # zeros stay: one step below +-0 is a NaN pattern
    return (t.contiguous().view(torch.int16) + step).view(torch.bfloat16)


def _ref_block(blk, x, e, ctx, grid, mask, cfg, attn=None, jitter=None):
    """One block; ``attn(q, k, v)`` replaces the dense masked self-attention (the
    gather restatement at sizes where a dense mask does not fit).  ``jitter`` (a
    CPU torch.Generator): every bf16 intermediate that the fused kernels round at
    another point (the modulated norms, q/k after RMSNorm + RoPE, the attention
    outputs, the GELU output) moves by up to one unit in the last place, which
    measures how far such differences alone carry through the fp8 quantisers."""
    J = (lambda t: t) if jitter is None else (lambda t: _jitter(t, jitter))  # noqa: E731
    n, d = cfg.num_heads, cfg.head_dim
    dtp = x.dtype
    ep = [t.reshape(1, -1) for t in (blk.modulation.float() + e).chunk(6, dim=1)]
    attn_in = J((blk.norm1(x).float() * (1 + ep[1]) + ep[0]).to(dtp))
    sa = blk.self_attn
    s = x.shape[0]
    q = sa.norm_q(_ref_linear(sa.q, attn_in)).view(s, n, d)
    k = sa.norm_k(_ref_linear(sa.k, attn_in)).view(s, n, d)
    v = _ref_linear(sa.v, attn_in).view(s, n, d)
    q, k = J(_ref_rope(q, grid, cfg)), J(_ref_rope(k, grid, cfg))
    a = J(_ref_attention(q, k, v, mask) if attn is None else attn(q, k, v))
    y = _ref_linear(sa.o, a.reshape(s, n * d))
    x = (x.float() + y.float() * ep[2]).to(dtp)
    ca = blk.cross_attn
    xn = blk.norm3(x)
    lc = ctx.shape[0]
    cq = ca.norm_q(_ref_linear(ca.q, xn)).view(s, n, d)
    ck = ca.norm_k(_ref_linear(ca.k, ctx)).view(lc, n, d)
    cv = _ref_linear(ca.v, ctx).view(lc, n, d)
    x = x + _ref_linear(ca.o, J(_ref_attention(cq, ck, cv)).reshape(s, n * d))
    ffn_in = J((blk.norm2(x).float() * (1 + ep[4]) + ep[3]).to(dtp))
    hmid = J(F.gelu(_ref_linear(blk.ffn[0], ffn_in).float(), approximate="tanh").to(dtp))
    y = _ref_linear(blk.ffn[2], hmid)
    return (x.float() + y.float() * ep[5]).to(dtp)


SMALL = mdl.SRDiTConfig(dim=256, ffn_dim=512, num_heads=2, num_layers=2, text_len=64)


@pytest.mark.parametrize("scaling", ["tensor", "rowwise"])
def test_block_stack_matches_fp32_restatement(scaling):
    print(f"[case] block stack scaling={scaling}", flush=True)
    cfg = SMALL
    model = mdl.build_refiner(cfg, device=DEV, scaling=scaling, seed=3)
    f, h, w = 3, 16, 16
    geom = model.geometry(f, h, w, cfg.text_len, DEV)
    g = torch.Generator("cpu").manual_seed(0)
    x = torch.randn(f * h * w, cfg.dim, generator=g).to(torch.bfloat16).to(DEV)
    ctx = torch.randn(cfg.text_len, cfg.dim, generator=g).to(torch.bfloat16).to(DEV)
    e0 = (torch.randn(1, 6, cfg.dim, generator=g) / cfg.dim ** 0.5).to(DEV)
    geo = obg.Geometry(f_cur=f, f_kv=f, h=h, w=w, block_t=1, bh=8, bw=8, rh=1, rw=1, sym_rt=1)
    mask = torch.from_numpy(obg.dense_mask(geo)).to(DEV)
    with torch.no_grad():
        out = model.blocks_forward(x, e0, ctx, geom)
        ref = x
        for blk in model.blocks:
            ref = _ref_block(blk, ref, e0, ctx, (f, h, w), mask, cfg)
    torch.cuda.synchronize()
    o, r = out.float(), ref.float()
    err = (o - r).abs()
    scale = r.abs().mean().item()
    print(f"[metrics] max {err.max().item():.3e} mean {err.mean().item():.3e} |ref| {scale:.3e}",
          flush=True)
    assert torch.isfinite(o).all()
    assert err.mean().item() <= 2e-3 * max(1.0, scale)
    assert err.max().item() <= 5e-2 * max(1.0, r.abs().max().item())


@pytest.mark.parametrize("scaling", ["tensor", "rowwise"])
def test_one_block_at_full_width_vs_gather_restatement(scaling):
    """One block of the shipped width (3072, 24 heads of 128, FFN 14336, fp8
    per-tensor, or row-wise as the reference's Fp8Linear defaults to,
    fp8_linear.py:93-103) on the 6x45x80 token grid with 512 text tokens,
    against the float32 restatement whose window attention is the gather
    backend (oracle/gather_torch.py, attention.py:660-802) over the oracle's
    windows."""
    from oracle import gather_torch as ogt
    cfg = mdl.SRDiTConfig()
    print(f"[case] one block at 3072 wide, 6x45x80 tokens, 512 text tokens, {scaling}", flush=True)
    model = mdl.build_refiner(cfg, device=DEV, scaling=scaling, seed=5, num_layers=1)
    f, h, w = 6, 45, 80
    geom = model.geometry(f, h, w, cfg.text_len, DEV)
    g = torch.Generator("cpu").manual_seed(2)
    x = torch.randn(f * h * w, cfg.dim, generator=g).to(torch.bfloat16).to(DEV)
    ctx = torch.randn(cfg.text_len, cfg.dim, generator=g).to(torch.bfloat16).to(DEV)
    e0 = (torch.randn(1, 6, cfg.dim, generator=g) / cfg.dim ** 0.5).to(DEV)
    geo = obg.Geometry(f_cur=f, f_kv=f, h=h, w=w, block_t=1, bh=8, bw=8, rh=1, rw=1, sym_rt=1)
    plan = ogt.GatherPlan(geo, None, device=DEV)

    def attn(q, k, v):
        return ogt.gather_attend(plan, q.float(), k.float(), v.float(), win_chunk=64,
                                 math_backend=True).to(q.dtype)

    with torch.no_grad():
        out = model.blocks_forward(x, e0, ctx, geom)
        ref = _ref_block(model.blocks[0], x, e0, ctx, (f, h, w), None, cfg, attn=attn)
        ref_j = _ref_block(model.blocks[0], x, e0, ctx, (f, h, w), None, cfg, attn=attn,
                           jitter=torch.Generator("cpu").manual_seed(1))
    torch.cuda.synchronize()
    o, r = out.float(), ref.float()
    upd = (r - x.float()).norm()
    rel = ((o - r).norm() / upd).item()                   # over the block's update
    floor = ((ref_j.float() - r).norm() / upd).item()     # one-ulp rounding moves alone
    err = (o - r).abs()
    print(f"[metrics] max {err.max().item():.3e} mean {err.mean().item():.3e} update rel-L2 "
          f"{rel:.3e}; restatement with one-ulp moves: {floor:.3e}", flush=True)
    assert torch.isfinite(o).all()
    # the product sits no farther from the restatement than the restatement moves
    # under one-ulp differences in its bf16 intermediates (fp8 rounding flips)
    assert rel <= 1.5 * floor, (rel, floor)
    assert err.max().item() <= 5e-2 * max(1.0, r.abs().max().item())


def test_rope_fp32_matches_complex128():
    cfg = mdl.SRDiTConfig()
    f, h, w = 3, 9, 10
    x = torch.randn(f * h * w, 24, 128, generator=torch.Generator("cpu").manual_seed(1)).to(
        torch.bfloat16).to(DEV)
    ours = mdl.rope_apply(x, mdl.rope_table(cfg, f, h, w, 0, DEV))
    ref = _ref_rope(x, (f, h, w), cfg)
    diff = (ours.float() - ref.float()).abs()
    # equal after the bf16 rounding except where the fp64 product sits on a rounding
    # boundary; such elements differ by one bf16 step
    assert (diff > 0).float().mean().item() < 1e-3
    assert diff.max().item() <= 2 ** -7 * ref.float().abs().max().item()


@pytest.mark.parametrize("scaling", ["tensor", "rowwise"])
def test_qkv_pack_and_stacked_modulations_match_the_separate_paths(scaling, monkeypatch):
    """Each block's q, k, v from one split-output GEMM (q and k only, when K and V
    go to caller buffers) and every block's modulation from one stacked add
    equal the per-Linear GEMMs and per-block adds bit for bit: the block stack's
    output and the K/V it writes."""
    print(f"[case] packed q/k/v and stacked modulations, {scaling}", flush=True)
    cfg = SMALL
    model = mdl.build_refiner(cfg, device=DEV, scaling=scaling, seed=8, num_layers=3)
    f, h, w = 3, 16, 16
    s = f * h * w
    geom = model.geometry(f, h, w, cfg.text_len, DEV)
    g = torch.Generator("cpu").manual_seed(5)
    ctx = torch.randn(cfg.text_len, cfg.dim, generator=g).to(torch.bfloat16).to(DEV)
    x = torch.randn(s, cfg.dim, generator=g).to(torch.bfloat16).to(DEV)
    e0 = (torch.randn(1, 6, cfg.dim, generator=g) / cfg.dim ** 0.5).to(DEV)

    def run():
        out = model.blocks_forward(x, e0, ctx, geom)
        kv = [(torch.empty(s, cfg.dim, dtype=torch.bfloat16, device=DEV),
               torch.empty(s, cfg.dim, dtype=torch.bfloat16, device=DEV)) for _ in model.blocks]
        out_kv = model.blocks_forward(x, e0, ctx, geom, kv_outs=kv)
        torch.cuda.synchronize()
        return out, out_kv, kv

    with torch.no_grad():
        a, a_kv, kv_a = run()
        assert all(blk.__dict__.get("_qkv_pack_cache") is not None for blk in model.blocks)
        assert model.__dict__.get("_mod_stack") is not None
        monkeypatch.setattr(mdl, "QKV_PACK", False)
        monkeypatch.setattr(mdl.SRDiT, "block_mods", lambda self, e0: None)
        b, b_kv, kv_b = run()
    assert torch.isfinite(a.float()).all()
    assert torch.equal(a, b) and torch.equal(a_kv, b_kv)
    for (k1, v1), (k2, v2) in zip(kv_a, kv_b):
        assert torch.equal(k1, k2) and torch.equal(v1, v2)


@pytest.mark.parametrize("scaling", ["tensor", "rowwise"])
def test_packed_text_kv_and_gelu_epilogue_match_the_separate_paths(scaling, monkeypatch):
    """Every layer's text K/V from one split-output GEMM equal the per-layer
    Linears bit for bit, and the per-tensor FFN with the GELU and amax in the
    first GEMM's epilogue equals the table path bit for bit."""
    print(f"[case] packed text K/V and GELU epilogue, {scaling}", flush=True)
    cfg = SMALL
    model = mdl.build_refiner(cfg, device=DEV, scaling=scaling, seed=6, num_layers=3)
    f, h, w = 3, 16, 16
    geom = model.geometry(f, h, w, cfg.text_len, DEV)
    g = torch.Generator("cpu").manual_seed(2)
    ctx = torch.randn(cfg.text_len, cfg.dim, generator=g).to(torch.bfloat16).to(DEV)
    with torch.no_grad():
        packed = model.cross_cache(ctx, geom)
        assert model.__dict__.get("_kv_pack") is not None
        separate = [blk.cross_kv(ctx, geom) for blk in model.blocks]
        torch.cuda.synchronize()
        for (k1, v1), (k2, v2) in zip(packed, separate):
            assert torch.equal(k1, k2) and torch.equal(v1, v2)
        x = torch.randn(f * h * w, cfg.dim, generator=g).to(torch.bfloat16).to(DEV)
        e0 = (torch.randn(1, 6, cfg.dim, generator=g) / cfg.dim ** 0.5).to(DEV)
        monkeypatch.setattr(mdl, "FFN_GELU_IN_GEMM", True)
        a = model.blocks_forward(x, e0, ctx, geom)
        monkeypatch.setattr(mdl, "FFN_GELU_IN_GEMM", False)
        b = model.blocks_forward(x, e0, ctx, geom)
        torch.cuda.synchronize()
        assert torch.equal(a, b)


def test_whole_30_layer_forward_graph_equals_eager():
    """The whole refiner forward at the shipped size (models.py:1877-2002): time
    and text embeddings, the patch embedding of a 48x6x90x160 latent, 30 blocks
    (fp8 per-tensor), head and unpatchify.  Finite and deterministic; captured
    once in a HIP graph, every replay (with eager work and synchronisations
    between replays) equals the eager forward bit for bit, also after new
    inputs are copied into the captured buffers."""
    cfg = mdl.SRDiTConfig()
    print("[case] whole 30-layer forward, graph vs eager", flush=True)
    model = mdl.build_refiner(cfg, device=DEV, scaling="tensor", seed=0)
    assert len(model.blocks) == 30
    f, h, w = 6, 45, 80
    geom = model.geometry(f, h, w, cfg.text_len, DEV)
    g = torch.Generator("cpu").manual_seed(3)
    latent = torch.randn(cfg.in_dim, f, 2 * h, 2 * w, generator=g).to(DEV)
    ctx = torch.randn(cfg.text_len, cfg.text_dim, generator=g).to(torch.bfloat16).to(DEV)
    t = torch.tensor([625.0], device=DEV)
    with torch.no_grad():
        want = model.forward(latent, t, ctx, geom)
        again = model.forward(latent, t, ctx, geom)
        torch.cuda.synchronize()
        assert want.shape == (cfg.out_dim, f, 2 * h, 2 * w)
        assert torch.isfinite(want).all() and want.float().std().item() > 0
        assert torch.equal(want, again)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            y = model.forward(latent, t, ctx, geom)
        for i in range(3):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(y, want), f"replay {i}"
            junk = torch.randn(1024, 1024, device=DEV) @ torch.randn(1024, 1024, device=DEV)
            torch.cuda.synchronize()
            del junk
        # new inputs through the captured buffers
        latent.copy_(torch.randn(latent.shape, generator=g).to(DEV))
        t.fill_(250.0)
        want2 = model.forward(latent, t, ctx, geom)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(want2).all() and not torch.equal(want2, want)
        assert torch.equal(y, want2)


def test_full_size_step_in_a_graph():
    """30 blocks at the 2K grid (fp8 per-tensor), captured once and replayed: finite,
    and every replay equals the eager forward on new inputs."""
    cfg = mdl.SRDiTConfig()
    print("[case] full-size refiner step graph", flush=True)
    model = mdl.build_refiner(cfg, device=DEV, scaling="tensor", seed=0, num_layers=4)
    f, h, w = 6, 45, 80
    geom = model.geometry(f, h, w, cfg.text_len, DEV)
    g = torch.Generator("cpu").manual_seed(0)
    x = torch.randn(f * h * w, cfg.dim, generator=g).to(torch.bfloat16).to(DEV)
    ctx = torch.randn(cfg.text_len, cfg.dim, generator=g).to(torch.bfloat16).to(DEV)
    e0 = (torch.randn(1, 6, cfg.dim, generator=g) / cfg.dim ** 0.5).to(DEV)
    with torch.no_grad():
        model.blocks_forward(x, e0, ctx, geom)         # plans, workspaces, device tables
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            y = model.blocks_forward(x, e0, ctx, geom)
        for it in range(3):
            x.copy_(torch.randn(x.shape, generator=g).to(torch.bfloat16).to(DEV))
            graph.replay()
            torch.cuda.synchronize()
            want = model.blocks_forward(x, e0, ctx, geom)
            torch.cuda.synchronize()
            assert torch.isfinite(y.float()).all()
            assert torch.equal(y, want), it


def _bf16_close(got, ref, frac=1e-3, scale=None, atol=1e-30):
    """Equal except in a small fraction of elements, which differ by at most one bf16
    step of `scale` (default: the values themselves; pass the magnitude of the terms
    when the result can cancel towards zero) plus `atol`."""
    g, r = got.float(), ref.float()
    diff = (g - r).abs()
    mag = torch.maximum(r.abs(), g.abs()) if scale is None else scale
    step = mag * 2 ** -7 + atol
    assert (diff <= step).all(), float((diff / step).max())
    assert (diff > 0).float().mean().item() <= frac, (diff > 0).float().mean().item()


def test_fused_ln_modulate_and_amax():
    from sr_dit import _lib
    g = torch.Generator("cpu").manual_seed(5)
    x = (torch.randn(700, 3072, generator=g) * 3 + 0.5).to(torch.bfloat16).to(DEV)
    sc = (torch.randn(3072, generator=g) * 0.1).to(DEV)
    sh = (torch.randn(3072, generator=g) * 0.1).to(DEV)
    w = (torch.randn(3072, generator=g) * 0.5 + 1).to(torch.bfloat16).to(DEV)
    b = (torch.randn(3072, generator=g) * 0.1).to(torch.bfloat16).to(DEV)
    out = torch.empty_like(x)
    zero = torch.zeros(3072, device=DEV)
    ln = F.layer_norm(x.float(), (3072,), None, None, 1e-6).to(torch.bfloat16)
    _lib.ln_modulate(x, None, None, zero, zero, 1e-6, out, None)      # the LayerNorm stage alone
    # (x - mean) cancels where x ~ mean, and the fp32 mean differs from torch's in
    # its last bits: an absolute 1e-4 / 2^7 on these unit-variance outputs
    _bf16_close(out, ln, atol=1e-4 * 2 ** -7)
    amax = torch.full((1,), 7, dtype=torch.int32, device=DEV)
    _lib.ln_modulate(x, None, None, sc, sh, 1e-6, out, amax)
    ref = (ln.float() * (1 + sc) + sh).to(torch.bfloat16)
    # a one-step change of the LayerNorm value moves the output by |ln (1 + sc)| / 2^8
    _bf16_close(out, ref, scale=ln.float().abs() * (1 + sc).abs() + ref.float().abs(),
                atol=1e-4 * 2 ** -7)
    bits = out.float().abs().max().to(torch.float32).view(torch.int32)
    assert amax.item() == bits.item()
    _lib.ln_modulate(x, w, b, None, None, 1e-6, out, None)
    ref = F.layer_norm(x.float(), (3072,), w.float(), b.float(), 1e-6).to(torch.bfloat16)
    _bf16_close(out, ref, scale=ln.float().abs() * w.float().abs() + ref.float().abs(),
                atol=1e-4 * 2 ** -7)


@pytest.mark.parametrize("M,K,affine", [(700, 3072, False), (700, 3072, True), (37, 8, False),
                                         (129, 1000, True), (64, 6144, False)])
def test_fused_residual_ln_modulate_matches_the_two_kernels(M, K, affine):
    """srdit_residual_ln_modulate == srdit_residual_gate then srdit_ln_modulate, bit for
    bit (both outputs and the amax word), on strided x rows, ragged widths and the
    K > 4096 path that runs the two kernels."""
    from sr_dit import _lib
    g = torch.Generator("cpu").manual_seed(9)
    x = (torch.randn(M, K + 16, generator=g) * 2).to(torch.bfloat16).to(DEV)[:, 8:8 + K]
    y = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV)
    gate = torch.randn(K, generator=g).to(DEV)
    w = (torch.randn(K, generator=g) * 0.5 + 1).to(torch.bfloat16).to(DEV) if affine else None
    b = (torch.randn(K, generator=g) * 0.1).to(torch.bfloat16).to(DEV) if affine else None
    sc = None if affine else (torch.randn(K, generator=g) * 0.1).to(DEV)
    sh = None if affine else (torch.randn(K, generator=g) * 0.1).to(DEV)
    x1_ref = torch.empty(M, K, dtype=torch.bfloat16, device=DEV)
    out_ref = torch.empty_like(x1_ref)
    am_ref = torch.full((1,), 5, dtype=torch.int32, device=DEV)
    _lib.residual_gate(x, y, gate, x1_ref)
    _lib.ln_modulate(x1_ref, w, b, sc, sh, 1e-6, out_ref, am_ref)
    x1, out = torch.empty_like(x1_ref), torch.empty_like(x1_ref)
    am = torch.full((1,), 5, dtype=torch.int32, device=DEV)
    _lib.residual_ln_modulate(x, y, gate, x1, w, b, sc, sh, 1e-6, out, am)
    assert torch.equal(x1, (x.float() + y.float() * gate).to(torch.bfloat16))
    assert torch.equal(x1, x1_ref)
    assert torch.equal(out, out_ref)
    assert am.item() == am_ref.item() == out.float().abs().max().view(torch.int32).item()
    with pytest.raises(RuntimeError):
        _lib.residual_ln_modulate(x, y, gate, x1, w, b, sc, sh, 1e-6, x1, am)  # out aliases x_out


def test_fused_residual_gate_bit_exact():
    from sr_dit import _lib
    g = torch.Generator("cpu").manual_seed(6)
    x = torch.randn(513, 3072, generator=g).to(torch.bfloat16).to(DEV)
    y = torch.randn(513, 3072, generator=g).to(torch.bfloat16).to(DEV)
    gate = torch.randn(3072, generator=g).to(DEV)
    out = torch.empty_like(x)
    _lib.residual_gate(x, y, gate, out)
    assert torch.equal(out, (x.float() + y.float() * gate).to(torch.bfloat16))
    _lib.residual_gate(x, y, gate, x)          # in place
    assert torch.equal(x, out)


def test_fused_rmsnorm_rope():
    from sr_dit import _lib
    cfg = mdl.SRDiTConfig()
    f, h, w = 2, 9, 10
    s = f * h * w
    g = torch.Generator("cpu").manual_seed(7)
    x = (torch.randn(s, 9216, generator=g) * 2).to(torch.bfloat16).to(DEV)[:, 3072:6144]  # strided rows
    wt = (torch.randn(3072, generator=g) * 0.3 + 1).to(torch.bfloat16).to(DEV)
    tab = mdl.rope_table(cfg, f, h, w, 0, DEV)
    cs = torch.view_as_real(tab).reshape(s, -1).contiguous()
    out = torch.empty(s, 3072, dtype=torch.bfloat16, device=DEV)
    _lib.rmsnorm_rope(x, wt, 1e-6, cs, 128, out)
    xf = x.float()
    y = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16) * wt
    ref = _ref_rope(y.view(s, 24, 128), (f, h, w), cfg).view(s, 3072)
    # a rotated pair can cancel: bound by the magnitude of the pair
    yp = y.float().view(s, 1536, 2).abs().sum(-1, keepdim=True).expand(s, 1536, 2).reshape(s, 3072)
    _bf16_close(out, ref, frac=2e-3, scale=yp)
    _lib.rmsnorm_rope(x, wt, 1e-6, None, 128, out)
    _bf16_close(out, y, frac=2e-3)


def test_gemm_gelu_epilogue_and_amax():
    from sr_dit import _lib
    g = torch.Generator("cpu").manual_seed(8)
    a = (torch.randn(300, 384, generator=g) * 0.5).to(F8).to(DEV)
    b = (torch.randn(272, 384, generator=g) * 0.5).to(F8).to(DEV)
    sa = torch.tensor([0.7], device=DEV)
    sb = torch.tensor([1.3], device=DEV)
    bias = (torch.randn(272, generator=g)).to(torch.bfloat16).to(DEV)
    plain = torch.empty(300, 272, dtype=torch.bfloat16, device=DEV)
    _lib.fp8_gemm(a, b, sa, sb, bias, plain)
    out = torch.empty_like(plain)
    amax = torch.zeros(1, dtype=torch.int32, device=DEV)
    _lib.fp8_gemm_ex(a, b, sa, sb, bias, out, epilogue=1, amax_out=amax)
    # 1 + tanh(.) cancels for negative inputs: bound by the input's magnitude
    _bf16_close(out, F.gelu(plain.float(), approximate="tanh").to(torch.bfloat16), frac=5e-3,
                scale=plain.float().abs())
    assert amax.item() == out.float().abs().max().view(torch.int32).item()
    _lib.fp8_gemm_ex(a, b, sa, sb, bias, out, epilogue=0, amax_out=None)
    assert torch.equal(out, plain)


@pytest.mark.parametrize("scaling", ["tensor", "rowwise"])
def test_fused_block_matches_unfused(scaling):
    print(f"[case] fused vs op-by-op blocks, scaling={scaling}", flush=True)
    cfg = SMALL
    model = mdl.build_refiner(cfg, device=DEV, scaling=scaling, seed=4)
    f, h, w = 3, 16, 16
    geom = model.geometry(f, h, w, cfg.text_len, DEV)
    g = torch.Generator("cpu").manual_seed(1)
    x = torch.randn(f * h * w, cfg.dim, generator=g).to(torch.bfloat16).to(DEV)
    ctx = torch.randn(cfg.text_len, cfg.dim, generator=g).to(torch.bfloat16).to(DEV)
    e0 = (torch.randn(1, 6, cfg.dim, generator=g) / cfg.dim ** 0.5).to(DEV)
    with torch.no_grad():
        assert all(b.fusable() for b in model.blocks)
        fused = model.blocks_forward(x, e0, ctx, geom)
        mdl.FUSED = False
        try:
            plain = model.blocks_forward(x, e0, ctx, geom)
        finally:
            mdl.FUSED = True
    torch.cuda.synchronize()
    err = (fused.float() - plain.float()).abs()
    print(f"[metrics] fused vs op-by-op: max {err.max().item():.3e} mean {err.mean().item():.3e}",
          flush=True)
    assert err.mean().item() <= 2e-3 * plain.float().abs().mean().item()


def test_gelu_quantiser_matches_stored_gelu_then_quantiser():
    """srdit_fp8_quant_tensor_gelu: h == torch's bf16(gelu_tanh(x)) and the codes
    and scale == the per-tensor quantiser of that h, bit for bit, with h stored
    into a separate buffer and without h (x left untouched)."""
    from sr_dit import _lib
    g = torch.Generator("cpu").manual_seed(12)
    for M, K in ((300, 384), (2048, 14336), (37, 8)):
        x = (torch.randn(M, K, generator=g) * 3).to(torch.bfloat16).to(DEV)
        h = F.gelu(x.float(), approximate="tanh").to(torch.bfloat16)
        want_q = torch.empty(M, K, dtype=F8, device=DEV)
        want_s = torch.empty(1, dtype=torch.float32, device=DEV)
        ws = torch.zeros(1, dtype=torch.int32, device=DEV)
        _lib.fp8_quant_tensor(h, want_q, want_s, ws)
        got_q = torch.empty_like(want_q)
        got_s = torch.empty_like(want_s)
        ws2 = torch.zeros(1, dtype=torch.int32, device=DEV)
        hbuf = torch.empty_like(x)
        _lib.fp8_quant_tensor_gelu(x, got_q, got_s, ws2, h=hbuf)       # separate h
        torch.cuda.synchronize()
        assert torch.equal(hbuf, h)
        assert torch.equal(got_s, want_s), (got_s.item(), want_s.item())
        assert torch.equal(got_q.view(torch.uint8), want_q.view(torch.uint8))
        assert torch.equal(ws2, ws)                                      # the amax word
        x0 = x.clone()
        got_q.zero_()
        _lib.fp8_quant_tensor_gelu(x, got_q, got_s, ws2)                # no h
        torch.cuda.synchronize()
        assert torch.equal(x, x0)
        assert torch.equal(got_s, want_s)
        assert torch.equal(got_q.view(torch.uint8), want_q.view(torch.uint8))


def test_gelu_table_covers_every_bf16_value():
    """The GELU table against torch's GELU for all 65,536 bf16 inputs: finite
    outputs bit for bit, NaN exactly where torch gives NaN."""
    from sr_dit import _lib
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    x = bits.reshape(128, 512).to(DEV)
    want = F.gelu(x.float(), approximate="tanh").to(torch.bfloat16)
    h = torch.empty_like(x)
    q = torch.empty(128, 512, dtype=F8, device=DEV)
    sc = torch.empty(1, dtype=torch.float32, device=DEV)
    ws = torch.zeros(1, dtype=torch.int32, device=DEV)
    _lib.fp8_quant_tensor_gelu(x, q, sc, ws, h=h)
    torch.cuda.synchronize()
    nan_w, nan_h = torch.isnan(want), torch.isnan(h)
    assert torch.equal(nan_w, nan_h)
    ok = ~nan_w
    assert torch.equal(h[ok].view(torch.int16), want[ok].view(torch.int16))
    print(f"[metrics] gelu table: {int(ok.sum())} finite-or-inf outputs bit-exact, "
          f"{int(nan_w.sum())} NaN", flush=True)

@pytest.mark.parametrize("bound", [0.5, 8.0, 300.0])
def test_gelu_codes_for_every_bf16_input(bound):
    """The quantise pass's codes (a table of the 65,536 inputs' codes at the
    call's scale, looked up per element) against torch's GELU followed by the
    plain per-tensor quantiser, bit for bit, for every finite bf16 x with
    |x| <= bound (the bound sets the scale, so the codes span the e4m3 range)."""
    from sr_dit import _lib
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    xs = bits[torch.isfinite(bits.float()) & (bits.float().abs() <= bound)]
    n = xs.numel()
    pad = (-n) % 512
    x = torch.cat([xs, xs[:pad]]).reshape(-1, 512).to(DEV)
    h = F.gelu(x.float(), approximate="tanh").to(torch.bfloat16)
    want_q = torch.empty(x.shape, dtype=F8, device=DEV)
    want_s = torch.empty(1, dtype=torch.float32, device=DEV)
    _lib.fp8_quant_tensor(h, want_q, want_s, torch.zeros(1, dtype=torch.int32, device=DEV))
    got_q = torch.empty_like(want_q)
    got_s = torch.empty_like(want_s)
    _lib.fp8_quant_tensor_gelu(x, got_q, got_s, torch.zeros(1, dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    print(f"[metrics] {n} inputs, scale {got_s.item():.4e}, "
          f"{int(torch.unique(got_q.view(torch.uint8)).numel())} distinct codes", flush=True)
    assert torch.equal(got_s, want_s)
    assert torch.equal(got_q.view(torch.uint8), want_q.view(torch.uint8))


def test_gelu_amax_shortcut_holds_over_every_bf16_value():
    """The facts the amax shortcut rests on, over all 65,536 bf16 inputs of the
    table: h = bf16(gelu(x)) is non-decreasing over x >= 0, and |h| below 0 stays
    under h(0.375) (the shortcut's threshold)."""
    from sr_dit import _lib
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    x = bits.reshape(128, 512).to(DEV)
    h = torch.empty_like(x)
    q = torch.empty(128, 512, dtype=F8, device=DEV)
    sc = torch.empty(1, dtype=torch.float32, device=DEV)
    ws = torch.zeros(1, dtype=torch.int32, device=DEV)
    _lib.fp8_quant_tensor_gelu(x, q, sc, ws, h=h)
    xf, hf = x.float().reshape(-1), h.float().reshape(-1)
    fin = torch.isfinite(xf)
    pos = fin & (xf >= 0)
    order = torch.argsort(xf[pos])
    hp = hf[pos][order]
    assert bool((hp[1:] >= hp[:-1]).all())
    neg = fin & (xf < 0)
    thr = hf[(xf == 0.375).nonzero()[0, 0]].item()
    assert hf[neg].abs().max().item() < thr, (hf[neg].abs().max().item(), thr)


@pytest.mark.parametrize("shift", [0.0, -30.0], ids=["shortcut", "fallback"])
def test_gelu_amax_shortcut_gives_the_same_codes(shift):
    """The FFN's first GEMM writing its largest positive output, then the table
    quantiser with that word: codes and scale equal the plain call's, both when
    the word decides the amax (shortcut) and when it does not (outputs shifted
    below 0.375: the full amax pass runs)."""
    from sr_dit import _lib
    g = torch.Generator("cpu").manual_seed(21)
    M, N, K = 2048, 2304, 512
    a = (torch.randn(M, K, generator=g) * 0.5).to(F8).to(DEV)
    b = (torch.randn(N, K, generator=g) * 0.5).to(F8).to(DEV)
    sa = torch.tensor([1.0], device=DEV)
    sb = torch.tensor([0.1], device=DEV)   # outputs ~ N(0, 0.57^2), then shifted
    bias = torch.full((N,), shift, dtype=torch.bfloat16, device=DEV)
    x = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    xpos = torch.zeros(1, dtype=torch.int32, device=DEV)
    _lib.fp8_gemm_ex(a, b, sa, sb, bias, x, epilogue=_lib.GEMM_AMAX_POS, amax_out=xpos)
    torch.cuda.synchronize()
    want_pos = x.float().clamp_min(0).max()
    assert xpos.view(torch.float32).item() == want_pos.item()
    q1, q2 = (torch.empty(M, N, dtype=F8, device=DEV) for _ in range(2))
    s1, s2 = (torch.empty(1, dtype=torch.float32, device=DEV) for _ in range(2))
    w1, w2 = (torch.zeros(1, dtype=torch.int32, device=DEV) for _ in range(2))
    _lib.fp8_quant_tensor_gelu(x, q1, s1, w1)
    _lib.fp8_quant_tensor_gelu(x, q2, s2, w2, xmax_pos=xpos)
    torch.cuda.synchronize()
    print(f"[metrics] largest positive output {want_pos.item():.4f}", flush=True)
    assert (want_pos.item() >= 0.375) == (shift == 0.0)
    assert torch.equal(w1, w2) and torch.equal(s1, s2)
    assert torch.equal(q1.view(torch.uint8), q2.view(torch.uint8))
