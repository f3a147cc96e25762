"""The streaming denoise loop on the GPU (sr_dit.stream.StreamingRefiner).

A two-layer refiner of the shipped width (3072, 24 heads, fp8 per-tensor
Linears) on a 16x24-token grid, 3-frame chunks, a 6-frame cache (so the rings
wrap), the shipped 4x4/r3 window:
  * in-place rings against every layer reading the reference's concatenation
    of its cache with the chunk (causal_inference.py:858-976 through
    attention.py:1506-1510): bit-identical chunks and caches;
  * HIP-graph replays (one graph per cache length, reused while the ring head
    and the RoPE offset move) against eager forwards.
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
    return noise, ctx


def _stream(model, noise, ctx, **kw):
    r = StreamingRefiner(model, H, W, ctx, chunk=CHUNK, kv_len=KV, seed=1, device=DEV, **kw)
    outs = []
    r.heads_seen = []
    for c in range(noise.shape[1] // CHUNK):
        r.heads_seen.append(r.rings[0].head)
        print(f"[case] stream chunk {c} cached={r.rings[0].cached} head={r.rings[0].head} {kw}",
              flush=True)
        outs.append(r.refine_chunk(noise[:, c * CHUNK:(c + 1) * CHUNK], c * CHUNK).clone())
    torch.cuda.synchronize()
    return r, outs


def test_stream_ring_in_place_equals_concatenation(refiner_model):
    noise, ctx = _inputs(refiner_model.cfg, 4)
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
    noise, ctx = _inputs(refiner_model.cfg, 5)
    rg, g = _stream(refiner_model, noise, ctx, use_graph=True)
    re_, e = _stream(refiner_model, noise, ctx, use_graph=False)
    assert sorted(rg._graphs) == [0, 3, 6]  # one graph per cache length
    for c, (x, y) in enumerate(zip(g, e)):
        err = (x - y).abs().max().item()
        scale = y.abs().max().item()
        print(f"[metrics] chunk {c}: max|graph - eager| = {err:.3e} (max|x0| {scale:.3e})",
              flush=True)
        assert err <= 1e-3 * scale, f"chunk {c}"
