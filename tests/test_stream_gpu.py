"""The streaming denoise loop on the GPU (sr_dit.stream.StreamingRefiner).

A two-layer refiner of the shipped width (3072, 24 heads, fp8 per-tensor
Linears) on a 16x24-token grid, 3-frame chunks, a 6-frame cache (so the rings
wrap), the shipped 4x4/r3 window:
  * in-place rings against every layer reading the reference's concatenation
    of its cache with the chunk (causal_inference.py:858-976 through
    attention.py:1506-1510): bit-identical chunks and caches;
  * HIP-graph replays (one graph per cache length, reused while the ring head
    and the RoPE offset move) bit-identical to eager forwards;
  * the same with the LQ anchor (both alignments): the harvest forward writes
    each layer's anchor K/V into its ring's prefix, the denoising steps read
    it there, against every layer reading the reference's concatenation
    ``cat([anchor, cache, chunk])`` (attention.py:868-874).
"""
import pytest
import torch

from sr_dit import model as mdl
from sr_dit.stream import StreamingRefiner

pytestmark = pytest.mark.gpu

DEV = "cuda"
H, W, CHUNK, KV = 16, 24, 3, 6


@pytest.fixture(scope="module")
def refiner_model():
    cfg = mdl.SRDiTConfig(num_layers=2)
    return mdl.build_refiner(cfg, device=DEV, scaling="tensor", seed=0)


def _inputs(cfg, chunks):
    g = torch.Generator("cpu").manual_seed(5)
    noise = torch.randn(cfg.in_dim, CHUNK * chunks, 2 * H, 2 * W, generator=g).to(DEV)
    ctx = torch.randn(77, cfg.text_dim, generator=g).to(torch.bfloat16).to(DEV)
    lq = torch.randn(cfg.in_dim, CHUNK * chunks, 2 * H, 2 * W, generator=g).to(DEV)
    return noise, ctx, lq


def _stream(model, noise, ctx, lq=None, **kw):
    r = StreamingRefiner(model, H, W, ctx, chunk=CHUNK, kv_len=KV, seed=1, device=DEV, **kw)
    outs = []
    r.heads_seen = []
    for c in range(noise.shape[1] // CHUNK):
        r.heads_seen.append(r.rings[0].head)
        print(f"[case] stream chunk {c} cached={r.rings[0].cached} head={r.rings[0].head} {kw}",
              flush=True)
        sl = slice(c * CHUNK, (c + 1) * CHUNK)
        outs.append(r.refine_chunk(noise[:, sl], c * CHUNK,
                                   None if lq is None else lq[:, sl]).clone())
    torch.cuda.synchronize()
    return r, outs


def test_stream_ring_in_place_equals_concatenation(refiner_model):
    noise, ctx, _ = _inputs(refiner_model.cfg, 4)
    ra, a = _stream(refiner_model, noise, ctx, use_graph=False)
    rb, b = _stream(refiner_model, noise, ctx, use_graph=False, ring_cat=True)
    assert any(hd != 0 for hd in ra.heads_seen)  # a chunk ran with the ring wrapped
    for c, (x, y) in enumerate(zip(a, b)):
        assert torch.isfinite(x).all()
        assert torch.equal(x, y), f"chunk {c}"
    for la, lb in zip(ra.rings, rb.rings):
        ka, va = la.logical(0)
        kb, vb = lb.logical(0)
        assert torch.equal(ka, kb) and torch.equal(va, vb)


def test_stream_graph_replays_match_eager(refiner_model):
    noise, ctx, _ = _inputs(refiner_model.cfg, 5)
    rg, g = _stream(refiner_model, noise, ctx, use_graph=True)
    re_, e = _stream(refiner_model, noise, ctx, use_graph=False)
    # one step graph and one refresh graph (K/V only) per cache length
    assert sorted(rg._graphs) == [("plain", 0), ("plain", 3), ("plain", 6),
                                  ("refresh", 0), ("refresh", 3), ("refresh", 6)]
    for c, (x, y) in enumerate(zip(g, e)):
        err = (x - y).abs().max().item()
        scale = y.abs().max().item()
        print(f"[metrics] chunk {c}: max|graph - eager| = {err:.3e} (max|x0| {scale:.3e})",
              flush=True)
        assert torch.equal(x, y), f"chunk {c}"


@pytest.mark.parametrize("anchor", ["frame", "chunk"])
def test_stream_lq_anchor_in_place_equals_concatenation(refiner_model, anchor):
    noise, ctx, lq = _inputs(refiner_model.cfg, 4)
    ra, a = _stream(refiner_model, noise, ctx, lq=lq, use_graph=False, anchor=anchor)
    rb, b = _stream(refiner_model, noise, ctx, lq=lq, use_graph=False, ring_cat=True,
                    anchor=anchor)
    assert any(hd != 0 for hd in ra.heads_seen)
    for c, (x, y) in enumerate(zip(a, b)):
        assert torch.isfinite(x).all()
        assert torch.equal(x, y), f"chunk {c}"
    for la, lb in zip(ra.rings, rb.rings):
        ka, va = la.logical(0)
        kb, vb = lb.logical(0)
        assert torch.equal(ka, kb) and torch.equal(va, vb)
        assert torch.equal(la.anchor_k(0), lb.anchor_k(0))
        assert torch.equal(la.anchor_v(0), lb.anchor_v(0))
        assert torch.isfinite(la.anchor_k(0).float()).all() and la.anchor_v(0).abs().max() > 0


def test_stream_lq_anchor_is_used(refiner_model):
    """The anchored chunk differs from the same chunk without the anchor, and
    differs again with another LQ input; the refresh pass (no anchor) leaves a
    cache whose first chunk depends on the anchor only through x0."""
    noise, ctx, lq = _inputs(refiner_model.cfg, 1)
    _, a = _stream(refiner_model, noise, ctx, lq=lq, use_graph=False, anchor="frame")
    _, b = _stream(refiner_model, noise, ctx, use_graph=False)
    _, c = _stream(refiner_model, noise, ctx, lq=lq.flip(-1), use_graph=False, anchor="frame")
    assert not torch.equal(a[0], b[0])
    assert not torch.equal(a[0], c[0])


def test_stream_lq_anchor_graph_replays_match_eager(refiner_model):
    noise, ctx, lq = _inputs(refiner_model.cfg, 4)
    rg, g = _stream(refiner_model, noise, ctx, lq=lq, use_graph=True, anchor="frame")
    re_, e = _stream(refiner_model, noise, ctx, lq=lq, use_graph=False, anchor="frame")
    assert sorted(rg._graphs) == [("anchored", 0), ("anchored", 3), ("anchored", 6),
                                  ("harvest", 0), ("refresh", 0), ("refresh", 3), ("refresh", 6)]
    for c, (x, y) in enumerate(zip(g, e)):
        err = (x - y).abs().max().item()
        scale = y.abs().max().item()
        print(f"[metrics] anchored chunk {c}: max|graph - eager| = {err:.3e} (max|x0| {scale:.3e})",
              flush=True)
        assert torch.equal(x, y), f"chunk {c}"


def test_stream_anchor_scale_mode_and_harvest_noise(refiner_model):
    """The anchor scale multiplies V (mode "v") or K (mode "k") of the harvested
    anchor, rounded to bf16 as models.py:638-643 computes it (a scale of 0.5 is
    exact); a harvest at timestep > 0 noises the LQ input first
    (causal_inference.py:468-471) and gives another, finite anchor."""
    _, ctx, lq = _inputs(refiner_model.cfg, 1)
    chunk = lq[:, :CHUNK]

    def harvested(**kw):
        r = StreamingRefiner(refiner_model, H, W, ctx, chunk=CHUNK, kv_len=KV, seed=1, device=DEV,
                             use_graph=False, anchor="frame", **kw)
        print(f"[case] harvest {kw}", flush=True)
        r.harvest(chunk, 0)
        torch.cuda.synchronize()
        return [(ring.anchor_k(0).clone(), ring.anchor_v(0).clone()) for ring in r.rings]

    base = harvested()
    for mode in ("v", "k"):
        scaled = harvested(anchor_scale=0.5, anchor_mode=mode)
        for (k0, v0), (k1, v1) in zip(base, scaled):
            if mode == "v":
                assert torch.equal(k1, k0) and torch.equal(v1, (v0.float() * 0.5).to(v0.dtype))
            else:
                assert torch.equal(v1, v0) and torch.equal(k1, (k0.float() * 0.5).to(k0.dtype))
    noised = harvested(anchor_harvest_t=500)
    for (k0, v0), (k1, v1) in zip(base, noised):
        assert torch.isfinite(k1.float()).all() and torch.isfinite(v1.float()).all()
        assert not torch.equal(v1, v0)


def test_stream_per_step_anchor_scales(refiner_model):
    """Per-step anchor scales (lq_guidance_scale as a list, causal_inference.py:904-906):
    step i reads bf16(unscaled anchor * scale_i), the last scale repeating; the kept
    unscaled anchor is the one-scale harvest; graph replays (the scale read from device
    memory) equal eager forwards; and the scales change the result."""
    noise, ctx, lq = _inputs(refiner_model.cfg, 2)
    scales = [1.0, 0.5, 2.0]  # four steps (sigma_start 1): the last two use 2.0
    rg, g = _stream(refiner_model, noise, ctx, lq=lq, use_graph=True, anchor="frame",
                    anchor_scale=scales, sigma_start=1.0)
    re_, e = _stream(refiner_model, noise, ctx, lq=lq, use_graph=False, anchor="frame",
                     anchor_scale=scales, sigma_start=1.0)
    r1, one = _stream(refiner_model, noise, ctx, lq=lq, use_graph=False, anchor="frame",
                      sigma_start=1.0)
    for c, (x, y) in enumerate(zip(g, e)):
        err = (x - y).abs().max().item()
        print(f"[metrics] per-step scales chunk {c}: max|graph - eager| = {err:.3e}", flush=True)
        assert torch.equal(x, y), f"chunk {c}"
    for ring_e, src, ring_1 in zip(re_.rings, re_._anchor_src, r1.rings):
        assert torch.equal(src, ring_1.anchor_v(0))
        assert torch.equal(ring_e.anchor_v(0), (src.float() * 2.0).to(src.dtype))
        assert torch.equal(ring_e.anchor_k(0), ring_1.anchor_k(0))
    assert not torch.equal(e[0], one[0])


@pytest.mark.parametrize("anchor", ["frame", "chunk"])
def test_stream_native_lq_anchor(refiner_model, anchor):
    """The native LQ anchor ("true" scheme, causal_inference.py:725-752): the harvest
    runs on the 8x12 LQ token grid with RoPE at HR positions, the anchored steps read
    the coarser anchor (anchor_hw); ring in place equals every layer reading the
    concatenation, and graph replays equal eager forwards."""
    noise, ctx, _ = _inputs(refiner_model.cfg, 3)
    g = torch.Generator("cpu").manual_seed(9)
    lqn = torch.randn(refiner_model.cfg.in_dim, 3 * CHUNK, 16, 24, generator=g).to(DEV)
    kw = dict(anchor=anchor, anchor_lq_hw=(8, 12), anchor_native_scheme="true")
    ra, a = _stream(refiner_model, noise, ctx, lq=lqn, use_graph=False, **kw)
    rb, b = _stream(refiner_model, noise, ctx, lq=lqn, use_graph=False, ring_cat=True, **kw)
    rg, gg = _stream(refiner_model, noise, ctx, lq=lqn, use_graph=True, **kw)
    assert ra.rings[0].A == CHUNK * 8 * 12
    for c, (x, y) in enumerate(zip(a, b)):
        assert torch.isfinite(x).all()
        assert torch.equal(x, y), f"chunk {c}"
    for c, (x, y) in enumerate(zip(gg, a)):
        err = (x - y).abs().max().item()
        print(f"[metrics] native anchor {anchor} chunk {c}: max|graph - eager| = {err:.3e}", flush=True)
        assert torch.equal(x, y), f"chunk {c}"


def test_stream_native_anchor_repeat_scheme(refiner_model):
    """Native anchor, "repeat" scheme (causal_inference.py:104-140): the harvested LQ
    K/V, copied into s_h x s_w HR blocks, become an HR-grid anchor; it equals the
    nearest-neighbour expansion of the "true" scheme's anchor; ring in place equals
    the concatenation and graph replays equal eager forwards."""
    noise, ctx, _ = _inputs(refiner_model.cfg, 2)
    g = torch.Generator("cpu").manual_seed(11)
    lqn = torch.randn(refiner_model.cfg.in_dim, 2 * CHUNK, 16, 24, generator=g).to(DEV)

    def make(**kw):
        return StreamingRefiner(refiner_model, H, W, ctx, chunk=CHUNK, kv_len=KV, seed=1,
                                device=DEV, use_graph=False, anchor="frame",
                                anchor_lq_hw=(8, 12), **kw)
    rt, rr = make(anchor_native_scheme="true"), make()  # "repeat" is the default
    print("[case] native repeat harvest", flush=True)
    rt.harvest(lqn[:, :CHUNK], 0)
    rr.harvest(lqn[:, :CHUNK], 0)
    torch.cuda.synchronize()
    for a, b in zip(rt.rings, rr.rings):
        assert b.A == CHUNK * H * W
        for lq_t, hr_t in ((a.anchor_k(0), b.anchor_k(0)), (a.anchor_v(0), b.anchor_v(0))):
            n, d = lq_t.shape[1], lq_t.shape[2]
            want = lq_t.view(CHUNK, 8, 1, 12, 1, n, d).expand(CHUNK, 8, 2, 12, 2, n, d)
            assert torch.equal(hr_t.view(CHUNK, 8, 2, 12, 2, n, d), want)
    kw = dict(anchor="frame", anchor_lq_hw=(8, 12), anchor_native_scheme="repeat")
    ra, a = _stream(refiner_model, noise, ctx, lq=lqn, use_graph=False, **kw)
    rb, b = _stream(refiner_model, noise, ctx, lq=lqn, use_graph=False, ring_cat=True, **kw)
    rg, gg = _stream(refiner_model, noise, ctx, lq=lqn, use_graph=True, **kw)
    for c, (x, y) in enumerate(zip(a, b)):
        assert torch.equal(x, y), f"chunk {c}"
    for c, (x, y) in enumerate(zip(gg, a)):
        assert torch.equal(x, y), f"chunk {c}"


def test_stream_rowwise_linears():
    """Row-wise fp8 Linears (the reference's default scaling) in the streaming loop:
    the fused block runs with the ring; ring in place equals the concatenation and
    graph replays equal eager forwards, bit for bit, over 4 chunks (ring wrapped)."""
    cfg = mdl.SRDiTConfig(num_layers=2)
    model = mdl.build_refiner(cfg, device=DEV, scaling="rowwise", seed=0)
    assert all(b.fusable() for b in model.blocks)
    noise, ctx, _ = _inputs(cfg, 4)
    ra, a = _stream(model, noise, ctx, use_graph=False)
    rb, b = _stream(model, noise, ctx, use_graph=False, ring_cat=True)
    rg, g = _stream(model, noise, ctx, use_graph=True)
    assert any(hd != 0 for hd in ra.heads_seen)
    for c, (x, y, z) in enumerate(zip(a, b, g)):
        assert torch.isfinite(x).all()
        assert torch.equal(x, y), f"chunk {c}"
        assert torch.equal(x, z), f"chunk {c}"
    # row-wise and per-tensor scales give different (both finite) results
    _, t = _stream(refiner_model_tensor(), noise, ctx, use_graph=False)
    assert not torch.equal(a[0], t[0])


def refiner_model_tensor():
    return mdl.build_refiner(mdl.SRDiTConfig(num_layers=2), device=DEV, scaling="tensor", seed=0)
