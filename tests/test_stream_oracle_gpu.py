"""The streaming denoise loop (sr_dit.stream.StreamingRefiner) against a float32
restatement of the reference's loop, written out here from
causal_inference.py:858-976 (per chunk: the step list, x0 from the flow
prediction, add_noise before every step but the last, the refresh pass at
context_noise whose K/V become the cache), sr_dit_wrapper.py:551-558
(x0 = x_t - t/1000 * flow in float64), scheduler.py:159-177 (add_noise with the
sigma of the nearest timestep) and models.py:780-833 (each layer attends
cat(cache, chunk) and keeps the last kv_len frames; RoPE at the chunk's
temporal offset).  The blocks are the float32 restatement of
tests/test_model_gpu.py with the block-grid streaming mask of the oracle;
the step list is the closed form of the shift-5 flow-match schedule,
t(k) = 1000 * 5u / (1 + 4u) with u = k / 1000; the embeddings and head are the
product's own (pinned by tests/test_forward_ends_*.py).

Two layers of width 256 (2 heads of 128), 16x24 tokens a frame, 3-frame chunks,
a 6-frame cache and 4 chunks, so the last chunk runs with the ring wrapped;
sharpened q/k norms (weight 2), a self-attention gate near 1 and a time
projection scaled by 20, so the output depends on which keys attention sees and
on the timestep.  (At q/k weight 4 a 2^-8 relative perturbation of the roped
q/k alone moves x0 by 6-14% in the float32 restatement; at weight 2 by 1%.)  Compared per chunk: x0 (its error over
the model's share of x0) and every layer's cache after the refresh pass.
Planted mistakes in the restatement (cache not truncated, RoPE offset fixed at
0, the flow's sign flipped, the refresh at the step's timestep) each move it
to at least twice the bound the product meets.

The anchored loop (the shipped per-frame LQ anchor, run_inference.sh:59-65)
adds, per chunk, the harvest of causal_inference.py:426-508 (each LR frame of
the chunk through the model as its own one-frame sample at harvest_t = 0, RoPE
at base_offset + i, no cache; every layer's RoPE'd K and V of those frames
become that layer's anchor) before the denoising steps, whose self-attention
then attends cat(anchor, cache, chunk) (attention.py:868-874) with HR frame i
seeing only anchor frame i within its spatial window (the oracle's dense mask,
anchor mode "frame"); the refresh pass runs without the anchor (:949-956).
The product measures x0 errors up to 0.036 and cache errors up to 0.039 there.
Planted mistakes, each at 0.127 or more: the anchor of the neighbouring frame,
the steps without the anchor, the anchor's V doubled (a wrong anchor scale,
models.py:638-643).  (Two weaker candidates move the loop by less than twice
the bound and are not planted: the harvest run as one chunk whose frames attend
each other, 0.052, and the harvest's RoPE at temporal offset 0, 0.076.)
"""
import numpy as np
import pytest
import torch

from oracle import blockgrid as obg
from parity import rope_table_ref
from sr_dit import model as mdl
from sr_dit.stream import StreamingRefiner
from test_model_gpu import _ref_attention, _ref_linear

pytestmark = pytest.mark.gpu

DEV = "cuda"
H, W, CHUNK, KV, CHUNKS = 16, 24, 3, 6, 4
CFG = mdl.SRDiTConfig(dim=256, ffn_dim=512, num_heads=2, num_layers=2, text_len=32)
# x0 error relative to the model's share of x0 (x0 - x_t = -t/1000 * flow), and
# cache rel-L2 error.  The product measures up to 0.040: every fp8 quantiser
# turns a one-ulp bf16 difference upstream (the fused kernels round at other
# points) into a flip of one e4m3 step (1/8) for a few percent of its inputs.
# Every planted mistake measures 0.19 or more.
BOUND = 6e-2


def _steps(sigma_start):
    ts = [1000.0 * 5 * u / (1 + 4 * u) for u in (1.0, 0.75, 0.5, 0.25)]
    keep = [t for t in ts if t <= sigma_start * 1000 + 1e-3]
    return keep or ts[-1:]


@pytest.fixture(scope="module")
def model():
    m = mdl.build_refiner(CFG, device=DEV, scaling="tensor", seed=2)
    with torch.no_grad():
        for blk in m.blocks:
            blk.self_attn.norm_q.weight.fill_(2.0)
            blk.self_attn.norm_k.weight.fill_(2.0)
            blk.modulation[:, 2] += 1.0   # self-attention gate ~1: attention shows in x0
        m.time_projection[1].weight.mul_(20.0)  # the timestep moves the modulation
    return m


def _mask(cached):
    f_kv = cached + CHUNK
    g = obg.Geometry(f_cur=CHUNK, f_kv=f_kv, h=H, w=W, block_t=CHUNK, bh=4, bw=4, rh=3, rw=3,
                     rt=max(f_kv // CHUNK - 1, 0), streaming=True)
    return torch.from_numpy(obg.dense_mask(g)).to(DEV)


def _rope(x, t_offset):
    s, n, d = x.shape
    fr = rope_table_ref(CHUNK, H, W, d, CFG.rope_theta, t_offset=t_offset, device=x.device)
    xc = torch.view_as_complex(x.to(torch.float64).reshape(s, n, d // 2, 2))
    return torch.view_as_real(xc * fr).flatten(2).to(x.dtype)


def _anchor_mask(cached):
    f_kv = cached + CHUNK
    g = obg.Geometry(f_cur=CHUNK, f_kv=f_kv, h=H, w=W, block_t=CHUNK, bh=4, bw=4, rh=3, rw=3,
                     rt=max(f_kv // CHUNK - 1, 0), streaming=True)
    return torch.from_numpy(obg.dense_mask(g, "frame")).to(DEV)


def _harvest_mask():
    """The harvest's self-attention: each LR frame its own one-frame sample, so a
    query frame sees only its own frame."""
    g = obg.Geometry(f_cur=CHUNK, f_kv=CHUNK, h=H, w=W, block_t=1, bh=4, bw=4, rh=3, rw=3,
                     sym_rt=0)
    return torch.from_numpy(obg.dense_mask(g)).to(DEV)


def _ref_stream_block(blk, x, e0, ctx, cache, t_offset, mistakes, anchor=None, harvest=None):
    """One block in stream mode: models.py:1304-1351 with the self-attention of
    :780-833 (cat(cache, chunk), keep the last KV frames).  ``anchor``: this
    layer's (k, v) anchor, attended first (attention.py:868-874).  ``harvest``:
    the harvest's mask instead of the streaming one, no cache; the layer's
    RoPE'd K and V are returned as its anchor."""
    n, d = CFG.num_heads, CFG.head_dim
    dtp = x.dtype
    ep = [t.reshape(1, -1) for t in (blk.modulation.float() + e0).chunk(6, dim=1)]
    attn_in = (blk.norm1(x).float() * (1 + ep[1]) + ep[0]).to(dtp)
    sa = blk.self_attn
    s = x.shape[0]
    off = 0 if "rope_offset_0" in mistakes else t_offset
    q = _rope(sa.norm_q(_ref_linear(sa.q, attn_in)).view(s, n, d), off)
    k = _rope(sa.norm_k(_ref_linear(sa.k, attn_in)).view(s, n, d), off)
    v = _ref_linear(sa.v, attn_in).view(s, n, d)
    full_k = k if cache is None else torch.cat([cache[0], k])
    full_v = v if cache is None else torch.cat([cache[1], v])
    cached = full_k.shape[0] // (H * W) - CHUNK
    if harvest is not None:
        attn = _ref_attention(q, k, v, harvest)
    elif anchor is not None:
        attn = _ref_attention(q, torch.cat([anchor[0], full_k]), torch.cat([anchor[1], full_v]),
                              _anchor_mask(cached))
    else:
        attn = _ref_attention(q, full_k, full_v, _mask(cached))
    y = _ref_linear(sa.o, attn.reshape(s, n * d))
    keep = full_k.shape[0] if "no_truncate" in mistakes else KV * H * W
    new_cache = (k, v) if harvest is not None else (full_k[-keep:], full_v[-keep:])
    x = (x.float() + y.float() * ep[2]).to(dtp)
    ca = blk.cross_attn
    xn = blk.norm3(x)
    lc = ctx.shape[0]
    cq = ca.norm_q(_ref_linear(ca.q, xn)).view(s, n, d)
    ck = ca.norm_k(_ref_linear(ca.k, ctx)).view(lc, n, d)
    cv = _ref_linear(ca.v, ctx).view(lc, n, d)
    x = x + _ref_linear(ca.o, _ref_attention(cq, ck, cv).reshape(s, n * d))
    ffn_in = (blk.norm2(x).float() * (1 + ep[4]) + ep[3]).to(dtp)
    hmid = torch.nn.functional.gelu(_ref_linear(blk.ffn[0], ffn_in).float(),
                                    approximate="tanh").to(dtp)
    y = _ref_linear(blk.ffn[2], hmid)
    return (x.float() + y.float() * ep[5]).to(dtp), new_cache


def _ref_forward(m, latent, t, ctx, caches, t_offset, mistakes, anchors=None, harvest=None):
    e, e0 = m.time_embed(torch.tensor([float(t)], device=DEV))
    x, grid = m.embed_patches(latent)
    new = []
    for i, (blk, cache) in enumerate(zip(m.blocks, caches)):
        x, kv = _ref_stream_block(blk, x, e0, ctx, cache, t_offset, mistakes,
                                  anchor=None if anchors is None else anchors[i], harvest=harvest)
        new.append(kv)
    return mdl.unpatchify(m.head(x, e), grid, CFG.patch_size, CFG.out_dim), new


def _ref_loop_anchored(m, noise, lq, ctx_raw, steps, seed, mistakes=()):
    """causal_inference.py:858-976 for one sample with the per-frame LQ anchor:
    per chunk the harvest (:426-508, :877-899), the anchored steps (:901-945),
    the refresh without the anchor (:949-956)."""
    ctx = m.embed_text(ctx_raw)
    caches = [None] * len(m.blocks)
    gen = torch.Generator(device=DEV).manual_seed(seed)
    outs, lasts, kept = [], [], []
    L = H * W
    for c in range(noise.shape[1] // CHUNK):
        t_offset = c * CHUNK
        sl = slice(c * CHUNK, (c + 1) * CHUNK)
        _, anchors = _ref_forward(m, lq[:, sl], 0.0, ctx, [None] * len(m.blocks), t_offset,
                                  mistakes, harvest=_harvest_mask())
        if "anchor_v_doubled" in mistakes:  # an anchor scale of 2 (models.py:638-643)
            anchors = [(k, v * 2) for k, v in anchors]
        if "anchor_wrong_frame" in mistakes:  # HR frame i sees LQ frame i + 1
            anchors = [(torch.roll(k, -L, 0), torch.roll(v, -L, 0)) for k, v in anchors]
        if "no_anchor" in mistakes:
            anchors = None
        noisy = noise[:, sl]
        x0 = None
        for i, t in enumerate(steps):
            flow, _ = _ref_forward(m, noisy, t, ctx, caches, t_offset, mistakes, anchors=anchors)
            x0 = (noisy.double() - (t / 1000.0) * flow.double()).to(flow.dtype)
            if i + 1 < len(steps):
                z = torch.randn(x0.shape, generator=gen, device=DEV, dtype=x0.dtype)
                sig = steps[i + 1] / 1000.0
                noisy = ((1 - sig) * x0 + sig * z).type_as(z)
        outs.append(x0)
        lasts.append(noisy)
        _, caches = _ref_forward(m, x0, 0.0, ctx, caches, t_offset, mistakes)
        kept.append([(k[-KV * H * W:], v[-KV * H * W:]) for k, v in caches])
    return outs, lasts, kept


def _ref_loop(m, noise, ctx_raw, steps, seed, mistakes=()):
    """causal_inference.py:858-976 for one sample, no anchor."""
    ctx = m.embed_text(ctx_raw)
    caches = [None] * len(m.blocks)
    gen = torch.Generator(device=DEV).manual_seed(seed)
    outs, lasts, kept = [], [], []
    for c in range(noise.shape[1] // CHUNK):
        t_offset = c * CHUNK
        noisy = noise[:, c * CHUNK:(c + 1) * CHUNK]
        x0 = None
        for i, t in enumerate(steps):
            flow, _ = _ref_forward(m, noisy, t, ctx, caches, t_offset, mistakes)
            sign = -1.0 if "flow_sign" in mistakes else 1.0
            x0 = (noisy.double() - sign * (t / 1000.0) * flow.double()).to(flow.dtype)
            if i + 1 < len(steps):
                z = torch.randn(x0.shape, generator=gen, device=DEV, dtype=x0.dtype)
                sig = steps[i + 1] / 1000.0
                noisy = ((1 - sig) * x0 + sig * z).type_as(z)
        outs.append(x0)
        lasts.append(noisy)
        t_ref = steps[-1] if "refresh_at_step_t" in mistakes else 0.0
        _, caches = _ref_forward(m, x0, t_ref, ctx, caches, t_offset, mistakes)
        kept.append([(k[-KV * H * W:], v[-KV * H * W:]) for k, v in caches])
    return outs, lasts, kept


def _inputs():
    g = torch.Generator("cpu").manual_seed(7)
    noise = torch.randn(CFG.in_dim, CHUNK * CHUNKS, 2 * H, 2 * W, generator=g).to(DEV)
    ctx = torch.randn(20, CFG.text_dim, generator=g).to(torch.bfloat16).to(DEV)
    return noise, ctx


def _product(m, noise, ctx, sigma_start, use_graph):
    r = StreamingRefiner(m, H, W, ctx, chunk=CHUNK, kv_len=KV, seed=1, device=DEV,
                         sigma_start=sigma_start, use_graph=use_graph)
    outs, heads = [], []
    for c in range(CHUNKS):
        heads.append(r.rings[0].head)
        outs.append(r.refine_chunk(noise[:, c * CHUNK:(c + 1) * CHUNK], c * CHUNK).clone())
    torch.cuda.synchronize()
    return r, outs, heads


def _err(x, ref, noisy):
    """x0 error relative to the model's share of x0 (x0 - x_t = -t/1000 * flow at the
    chunk's last step)."""
    return ((x.double() - ref.double()).norm() / (ref.double() - noisy.double()).norm()).item()


def _cache_err(ring_state, ref_state):
    return max(((a.float() - b.float()).norm() / b.float().norm()).item()
               for (ka, va), (kb, vb) in zip(ring_state, ref_state) for a, b in ((ka, kb), (va, vb)))


def _errors(prod, ref):
    """Per chunk: the x0 error and the worst layer cache (K or V) rel-L2 error."""
    (outs, caches), (ref_outs, lasts, kept) = prod, ref
    return ([_err(o, r, n) for o, r, n in zip(outs, ref_outs, lasts)],
            [_cache_err(c, k) for c, k in zip(caches, kept)])


def _run_product(m, noise, ctx, sigma_start, use_graph, lq=None):
    r = StreamingRefiner(m, H, W, ctx, chunk=CHUNK, kv_len=KV, seed=1, device=DEV,
                         sigma_start=sigma_start, use_graph=use_graph,
                         anchor=None if lq is None else "frame")
    outs, caches, heads = [], [], []
    for c in range(CHUNKS):
        sl = slice(c * CHUNK, (c + 1) * CHUNK)
        heads.append(r.rings[0].head)
        outs.append(r.refine_chunk(noise[:, sl], c * CHUNK,
                                   None if lq is None else lq[:, sl]).clone())
        caches.append([ring.logical(0) for ring in r.rings])
    torch.cuda.synchronize()
    return r, (outs, caches), heads


def _lq_input():
    """An LR latent for the anchor: the noise's own low-frequency content plus a
    fresh perturbation, so the anchor resembles, but is not, the chunk."""
    g = torch.Generator("cpu").manual_seed(11)
    base = torch.randn(CFG.in_dim, CHUNK * CHUNKS, H, W, generator=g)
    return torch.nn.functional.interpolate(base, size=(2 * H, 2 * W), mode="bilinear",
                                           align_corners=False).to(DEV)


@pytest.mark.parametrize("sigma_start", [0.6251, 1.0], ids=["one_step", "four_steps"])
def test_stream_loop_matches_restated_loop(model, sigma_start):
    print(f"[case] stream loop oracle sigma_start={sigma_start}", flush=True)
    noise, ctx = _inputs()
    steps = _steps(sigma_start)
    r, prod, heads = _run_product(model, noise, ctx, sigma_start, use_graph=True)
    assert [round(t, 3) for t in r.steps] == [round(t, 3) for t in steps]
    assert heads[-1] != 0, heads  # the last chunk ran with the ring wrapped
    with torch.no_grad():
        ref = _ref_loop(model, noise, ctx, steps, seed=1)
    ex, ec = _errors(prod, ref)
    print(f"[metrics] x0 error per chunk {np.round(ex, 5).tolist()}; "
          f"cache error per chunk {np.round(ec, 5).tolist()}", flush=True)
    assert all(o.shape == x.shape for o, x in zip(prod[0], ref[0]))
    assert max(ex) <= BOUND and max(ec) <= BOUND, (ex, ec)


@pytest.mark.parametrize("mistake", ["no_truncate", "rope_offset_0", "flow_sign",
                                     "refresh_at_step_t"])
def test_stream_loop_bound_rejects_planted_mistakes(model, mistake):
    print(f"[case] stream loop planted mistake {mistake}", flush=True)
    noise, ctx = _inputs()
    steps = _steps(1.0)
    _, prod, _ = _run_product(model, noise, ctx, 1.0, use_graph=False)
    with torch.no_grad():
        bad = _ref_loop(model, noise, ctx, steps, seed=1, mistakes=(mistake,))
    ex, ec = _errors(prod, bad)
    print(f"[metrics] {mistake}: x0 error {np.round(ex, 4).tolist()}, "
          f"cache error {np.round(ec, 4).tolist()}", flush=True)
    assert max(ex + ec) >= 2 * BOUND, (ex, ec)


@pytest.mark.parametrize("sigma_start", [0.6251, 1.0], ids=["one_step", "four_steps"])
def test_anchored_stream_loop_matches_restated_loop(model, sigma_start):
    """The shipped configuration: per-frame LQ anchor, harvest then anchored
    steps then refresh, per chunk, against the restated anchored loop."""
    print(f"[case] anchored stream loop oracle sigma_start={sigma_start}", flush=True)
    noise, ctx = _inputs()
    lq = _lq_input()
    steps = _steps(sigma_start)
    r, prod, heads = _run_product(model, noise, ctx, sigma_start, use_graph=True, lq=lq)
    assert heads[-1] != 0, heads
    with torch.no_grad():
        ref = _ref_loop_anchored(model, noise, lq, ctx, steps, seed=1)
    ex, ec = _errors(prod, ref)
    print(f"[metrics] anchored: x0 error per chunk {np.round(ex, 5).tolist()}; "
          f"cache error per chunk {np.round(ec, 5).tolist()}", flush=True)
    assert max(ex) <= BOUND and max(ec) <= BOUND, (ex, ec)


@pytest.mark.parametrize("mistake", ["anchor_wrong_frame", "no_anchor", "anchor_v_doubled"])
def test_anchored_stream_loop_bound_rejects_planted_mistakes(model, mistake):
    print(f"[case] anchored stream loop planted mistake {mistake}", flush=True)
    noise, ctx = _inputs()
    lq = _lq_input()
    steps = _steps(0.6251)
    _, prod, _ = _run_product(model, noise, ctx, 0.6251, use_graph=False, lq=lq)
    with torch.no_grad():
        bad = _ref_loop_anchored(model, noise, lq, ctx, steps, seed=1, mistakes=(mistake,))
    ex, ec = _errors(prod, bad)
    print(f"[metrics] {mistake}: x0 error {np.round(ex, 4).tolist()}, "
          f"cache error {np.round(ec, 4).tolist()}", flush=True)
    assert max(ex + ec) >= 2 * BOUND, (ex, ec)
