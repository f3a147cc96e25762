"""Streaming SR denoise loop: chunks of latent frames, few-step flow matching,
KV-cache refresh, on the in-place ring caches and HIP graphs.

Restates the per-chunk loop of CausalInferencePipeline.inference_sr
(video_refiner/pipeline_sr/causal_inference.py:858-976) for one sample:

  for each chunk of ``chunk`` latent frames (temporal offset advancing by chunk):
      [LQ anchor] harvest: model(lq chunk, harvest_t) with no cache; each layer's
                  K/V of the LQ frames become that layer's anchor (:426-508, :877-899)
      for each timestep t of the step list:
          flow = model(noisy, t)             # attends [anchor] + cached frames + the chunk
          x0   = noisy - (t / 1000) * flow   # sr_dit_wrapper.py:551-558, in float64
          if not the last step: noisy = add_noise(x0, randn, next t)
      model(x0, context_noise)               # the refresh pass: its K/V become the cache
      keep the last kv_len frames of the cache

The step list and ``add_noise`` are the FlowMatchScheduler's
(video_refiner/utils/scheduler.py:106-177, built as sr_dit_wrapper.py:492-494:
shift 5, sigma_min 0, extra_one_step) with the warped step list of
causal_inference.py:278-282 and the sigma_start filter of :831-834.

What is MI355X-specific: the per-layer caches are ``KVRing``s (the refresh
pass writes the chunk's K/V in place and ``commit`` moves them into the ring,
no per-call concatenation); the harvest forward writes each layer's anchor K/V
straight into its ring's anchor prefix, where the window kernels read it (no
anchor list, no concatenation); the text K/V of every layer are computed once
per video; and each model forward is one HIP graph replay, captured once per
kind (harvest, anchored step, plain step) and cache length (the ring's
position is read by the kernels from device memory, so one graph serves every
chunk once the cache is full).
"""
from __future__ import annotations

import torch

from . import _lib
from .kv_ring import KVRing
from .model import rope_axis_tables, rope_positions, rope_table_from_axes


class FlowMatchSchedule:
    """Host restatement of FlowMatchScheduler.set_timesteps / add_noise
    (scheduler.py:108-177) for the refiner's settings."""

    def __init__(self, shift=5.0, num_train_timesteps=1000, sigma_min=0.0, sigma_max=1.0,
                 extra_one_step=True):
        n = num_train_timesteps
        if extra_one_step:
            sig = torch.linspace(sigma_max, sigma_min, n + 1)[:-1]
        else:
            sig = torch.linspace(sigma_max, sigma_min, n)
        self.sigmas = shift * sig / (1 + (shift - 1) * sig)
        self.timesteps = self.sigmas * n
        self.num_train_timesteps = n

    def warp(self, step_list):
        """causal_inference.py:280-282: step k of the list -> timesteps[1000 - k] (0 past the end)."""
        ts = torch.cat([self.timesteps, torch.tensor([0.0])])
        return ts[self.num_train_timesteps - torch.tensor(step_list, dtype=torch.long)]

    def sigma(self, t) -> float:
        i = int(torch.argmin((self.timesteps - float(t)).abs()))
        return float(self.sigmas[i])

    def add_noise(self, x0, noise, t):
        s = self.sigma(t)
        return ((1 - s) * x0 + s * noise).type_as(noise)


class StreamingRefiner:
    """The chunked denoise loop over a ``SRDiT`` for one sample of ``h x w`` tokens
    per latent frame (the latent is 2h x 2w).

    ``kv_len`` cached frames per layer (sr_dit_5b.yaml:55), ``chunk`` frames per
    step (:45), window ``block_hw``/``block_radius_hw`` (:51-52), step list and
    ``context_noise`` of :10-17.  ``use_graph`` replays each forward from a HIP
    graph (captured at the first forward of each kind and cache length).
    ``ring_cat`` (tests only) makes every layer read the reference's
    concatenation of its anchor, cache and chunk instead of the ring in place.

    LQ anchor (run_inference.sh:59-65; causal_inference.py:636-700): ``anchor``
    "frame" (HR frame i attends LQ frame i; the shipped default) or "chunk"
    (every HR frame attends the whole LQ chunk), None to run without it.
    ``anchor_scale`` multiplies the anchor's V (``anchor_mode`` "v") or K
    ("k") as models.py:638-643 does; a sequence gives one scale per
    denoising step, the last one repeating, as ``lq_guidance_scale`` does
    (causal_inference.py:904-906).  ``anchor_harvest_t`` is the harvest's
    timestep (default ``context_noise``, :663-665).  ``anchor_lq_hw`` (h_a, w_a):
    the native LQ anchor, harvested on the LQ token grid with RoPE at HR
    positions; h and w must be multiples of h_a and w_a.  Its
    ``anchor_native_scheme`` is the reference's default "repeat"
    (causal_inference.py:650, inference_sr.py:295): every LQ token's K/V is
    copied into its s_h x s_w HR block (causal_inference.py:104-140) and the
    anchor is attended on the HR grid; "true" (causal_inference.py:725-752)
    keeps the coarser grid in attention, which lowers the anchor's softmax
    mass by about s_h*s_w against what the anchor LoRA was distilled with.

    ``sigma_start`` defaults to the shipped 0.6251 (sr_dit_5b.yaml:65,
    run_inference.sh:38): the warped step list 1000/937.5/833.3/625 keeps the
    single step t=625, so an anchored chunk is three forwards (harvest, step,
    refresh); 1.0 keeps all four steps.
    """

    def __init__(self, model, h, w, context_raw, *, chunk=3, kv_len=9,
                 step_list=(1000, 750, 500, 250), warp=True, context_noise=0,
                 sigma_start=0.6251, shift=5.0, block_hw=(4, 4), block_radius_hw=(3, 3),
                 anchor=None, anchor_scale=1.0, anchor_mode="v", anchor_harvest_t=None,
                 anchor_lq_hw=None, anchor_native_scheme="repeat", use_graph=True, seed=0,
                 device="cuda", ring_cat=False):
        cfg = model.cfg
        if anchor not in (None, "frame", "chunk"):
            raise ValueError(f"anchor must be None, 'frame' or 'chunk', got {anchor!r}.")
        if anchor_mode not in ("k", "v"):
            raise ValueError(f"anchor_mode must be 'k' or 'v', got {anchor_mode!r}.")
        scales = ([float(anchor_scale)] if isinstance(anchor_scale, (int, float))
                  else [float(x) for x in anchor_scale] or [1.0])
        self.anchor, self.anchor_mode, self.anchor_scales = anchor, anchor_mode, scales
        # One scale: applied once, in the harvest.  Several: the harvest keeps the
        # unscaled anchor aside and each anchored step writes its scaled copy.
        self._vary_scale = anchor is not None and any(x != scales[0] for x in scales)
        self.anchor_scale = 1.0 if self._vary_scale else scales[0]
        self.harvest_t = float(int(context_noise if anchor_harvest_t is None else anchor_harvest_t))
        self.sigma_start = float(sigma_start)
        if anchor_native_scheme not in ("true", "repeat"):
            raise ValueError(f"anchor_native_scheme must be 'true' or 'repeat', got "
                             f"{anchor_native_scheme!r}.")
        self.anchor_hw = (h, w)     # the harvest's token grid
        self._repeat = False        # the harvest grid is expanded to the HR grid
        if anchor is not None and anchor_lq_hw is not None:
            h_a, w_a = int(anchor_lq_hw[0]), int(anchor_lq_hw[1])
            if h_a < 1 or w_a < 1 or h % h_a or w % w_a:
                raise ValueError(f"StreamingRefiner: the native LQ anchor needs an integer token-grid "
                                 f"ratio, HR {(h, w)} vs LQ {(h_a, w_a)}.")
            self.anchor_hw = (h_a, w_a)
            self._repeat = anchor_native_scheme == "repeat" and (h_a, w_a) != (h, w)
        self.model, self.h, self.w, self.chunk = model, h, w, chunk
        self.device = torch.device(device)
        self.block_hw, self.block_radius_hw = tuple(block_hw), tuple(block_radius_hw)
        self.sched = FlowMatchSchedule(shift=shift)
        steps = self.sched.warp(step_list) if warp else torch.tensor(step_list, dtype=torch.float32)
        keep = steps[steps <= sigma_start * 1000 + 1e-3]
        self.steps = [float(t) for t in (keep if len(keep) else steps[-1:])]
        self.context_noise = float(context_noise)
        self.use_graph = use_graph
        self.ring_cat = bool(ring_cat)
        L = h * w
        grid_a = (h, w) if self._repeat else self.anchor_hw  # the anchor's grid in attention
        a_tok = chunk * grid_a[0] * grid_a[1] if anchor else 0
        self.rings = [KVRing(1, kv_len, chunk, L, cfg.num_heads, cfg.head_dim,
                             anchor_tokens=a_tok, device=self.device) for _ in model.blocks]
        self.gen = torch.Generator(device=self.device).manual_seed(seed)
        with torch.no_grad():
            self.ctx = model.embed_text(context_raw.to(self.device))
            g0 = self._geom(("plain", 0), 0)
            self.cross = model.cross_cache(self.ctx, g0)
        # static inputs of the captured forwards
        self._lat = torch.zeros(cfg.in_dim, chunk, 2 * h, 2 * w, dtype=torch.float32,
                                device=self.device)
        self._lat_lq = self._lat
        if self.anchor_hw != (h, w):
            self._lat_lq = torch.zeros(cfg.in_dim, chunk, 2 * self.anchor_hw[0],
                                       2 * self.anchor_hw[1], dtype=torch.float32, device=self.device)
        self._e = torch.zeros(1, cfg.dim, dtype=torch.float32, device=self.device)
        self._e0 = torch.zeros(1, 6, cfg.dim, dtype=torch.float32, device=self.device)
        # A forward's timestep and RoPE table reach the device by device-side
        # writes: a blocking host-to-device copy would wait for the forwards
        # already queued and leave the GPU idle while the host prepares the next.
        self._t_dev = torch.zeros(1, dtype=torch.float32, device=self.device)
        self._rope_axes = None  # per-axis RoPE tables on the device (rope_axis_tables)
        self._geoms = {}
        self._graphs = {}
        self.forwards = 0
        self._anchor_src = None
        self._lq_kv = None
        if self._repeat:  # the harvest's K/V on the LQ grid, expanded after the forward
            n_lq = chunk * self.anchor_hw[0] * self.anchor_hw[1]
            self._lq_kv = [(torch.empty(n_lq, cfg.num_heads, cfg.head_dim, dtype=r.k.dtype,
                                        device=self.device),
                            torch.empty(n_lq, cfg.num_heads, cfg.head_dim, dtype=r.v.dtype,
                                        device=self.device)) for r in self.rings]
        if self._vary_scale:
            self._anchor_src = [torch.empty_like(self._scaled_part(r)) for r in self.rings]
            self._scale_dev = torch.ones(1, dtype=torch.float32, device=self.device)

    # ---- one model forward --------------------------------------------------
    def _geom(self, key, t_offset):
        """Geometry of a forward kind: ("harvest", 0), ("anchored", cached),
        ("plain", cached) or ("refresh", cached) (the plain geometry)."""
        kind, cached = key
        kw = dict(chunk=self.chunk, t_offset=t_offset, block_hw=self.block_hw,
                  block_radius_hw=self.block_radius_hw)
        args = (self.chunk, self.h, self.w, self.ctx.shape[0], self.device)
        if kind == "harvest":
            h_a, w_a = self.anchor_hw
            return self.model.harvest_geometry(self.chunk, h_a, w_a, self.ctx.shape[0], self.device,
                                               per_frame=self.anchor == "frame",
                                               hw_stride=(self.h // h_a, self.w // w_a), **kw)
        return self.model.stream_geometry(*args, cached=cached,
                                          anchor=self.anchor if kind == "anchored" else None,
                                          anchor_hw=None if self._repeat else self.anchor_hw, **kw)

    def _static_geom(self, key, t_offset):
        """The geometry for this forward kind and cache length, its RoPE table
        refreshed in place for ``t_offset`` (so a captured graph sees the new table)."""
        g = self._geoms.get(key)
        if g is None:
            g = self._geoms[key] = self._geom(key, t_offset)
            g["t_offset"] = t_offset
            g["ring_cat"] = self.ring_cat
        elif g["t_offset"] != t_offset:
            f, gh, gw = g["grid"]
            rope = self._rope_on_device(f, gh, gw, t_offset, g["hw_stride"])
            g["rope"].copy_(rope)
            g["rope_cs"].copy_(torch.view_as_real(rope).reshape(g["rope_cs"].shape))
            g["t_offset"] = t_offset
        return g

    def _rope_on_device(self, f, h, w, t_offset, hw_stride):
        """The RoPE table of a (f, h, w) grid at frame offset ``t_offset``,
        gathered on the device from per-axis tables kept there (the same values
        as model.rope_table); the tables are rebuilt only when a position runs
        past them."""
        cfg = self.model.cfg
        n_pos = rope_positions(cfg, f, h, w, t_offset, hw_stride)
        if self._rope_axes is None or self._rope_axes[0].shape[0] < n_pos:
            self._rope_axes = rope_axis_tables(cfg, n_pos, self.device)
        return rope_table_from_axes(self._rope_axes, f, h, w, t_offset, hw_stride)

    def _run(self, geom):
        return self.model.forward_embedded(self._lat, self._e, self._e0, self.ctx, geom,
                                           rings=self.rings, cross=self.cross)

    def _run_refresh(self, geom):
        """The refresh pass: the clean chunk through the stack for its K/V alone
        (the flow output of causal_inference.py's refresh forward is discarded);
        the last layer stops once its K/V are in the ring and the head is skipped."""
        return self.model.forward_embedded(self._lat, self._e, self._e0, self.ctx, geom,
                                           rings=self.rings, cross=self.cross, kv_only=True)

    def _scaled_part(self, ring):
        return ring.anchor_v(0) if self.anchor_mode == "v" else ring.anchor_k(0)

    def _run_anchored(self, geom):
        """An anchored step; with per-step scales the anchor is first rewritten as
        bf16(unscaled * scale), the scale read from device memory (so one captured
        graph serves every step)."""
        if self._vary_scale:
            for r, src in zip(self.rings, self._anchor_src):
                torch.mul(src, self._scale_dev, out=self._scaled_part(r))
        return self._run(geom)

    def _run_harvest(self, geom):
        """The harvest forward: every layer's K/V land in its ring's anchor prefix
        (the flow output is not used, as causal_inference.py:490-508 keeps only
        the caches), then the anchor scale (models.py:638-643)."""
        s = self.chunk * self.anchor_hw[0] * self.anchor_hw[1]
        dim = self.model.cfg.dim
        if self._repeat:
            kv = [(k.view(s, dim), v.view(s, dim)) for k, v in self._lq_kv]
        else:
            kv = [(r.anchor_k(0).view(s, dim), r.anchor_v(0).view(s, dim)) for r in self.rings]
        out = self.model.forward_embedded(self._lat_lq, self._e, self._e0, self.ctx, geom,
                                          cross=self.cross, kv_outs=kv, kv_only=True)
        if self._repeat:  # LQ (i, j) -> HR (s_h i .. s_h i + s_h - 1, s_w j .. s_w j + s_w - 1)
            f, (h_a, w_a) = self.chunk, self.anchor_hw
            s_h, s_w = self.h // h_a, self.w // w_a
            for r, (k, v) in zip(self.rings, self._lq_kv):
                for src, dst in ((k, r.anchor_k(0)), (v, r.anchor_v(0))):
                    n, d = src.shape[1], src.shape[2]
                    dst.view(f, h_a, s_h, w_a, s_w, n, d).copy_(
                        src.view(f, h_a, 1, w_a, 1, n, d).expand(f, h_a, s_h, w_a, s_w, n, d))
        if self._vary_scale:
            for r, src in zip(self.rings, self._anchor_src):
                src.copy_(self._scaled_part(r))
        elif self.anchor_scale != 1.0:
            for r in self.rings:
                self._scaled_part(r).mul_(self.anchor_scale)
        return out

    def _launch(self, key, t, latent, t_offset, fn):
        with torch.no_grad():
            self._t_dev.fill_(float(t))
            e, e0 = self.model.time_embed(self._t_dev)
            self._e.copy_(e)
            self._e0.copy_(e0)
            (self._lat_lq if key[0] == "harvest" else self._lat).copy_(latent)
            geom = self._static_geom(key, t_offset)
            self.forwards += 1
            if not self.use_graph:
                return fn(geom)
            entry = self._graphs.get(key)
            if entry is None:
                fn(geom)  # plans, device tables, library handles: outside capture
                torch.cuda.synchronize(self.device)
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=_lib.capture_stream(self.device)):
                    out = fn(geom)
                entry = self._graphs[key] = (graph, out)
            entry[0].replay()
            return entry[1]

    def forward(self, latent, t, t_offset, anchored=False):
        """Flow prediction for the chunk ``latent`` [in_dim, chunk, 2h, 2w] at timestep
        ``t``, attending the cached frames (and, ``anchored``, the harvested LQ
        anchor); writes the chunk's K/V into the rings' current regions (kept
        only by ``commit``)."""
        kind = "anchored" if anchored and self.anchor is not None else "plain"
        fn = self._run_anchored if kind == "anchored" else self._run
        return self._launch((kind, self.rings[0].cached), t, latent, t_offset, fn)

    def refresh(self, x0, t_offset):
        """The cache refresh of a denoised chunk (no anchor): the chunk's K/V at
        ``context_noise`` go into the rings' current regions (kept by ``commit``)."""
        self._launch(("refresh", self.rings[0].cached), self.context_noise, x0, t_offset,
                     self._run_refresh)

    def harvest(self, lq, t_offset):
        """LQ-anchor harvest of one chunk (causal_inference.py:426-508): ``lq``
        [in_dim, chunk, 2h, 2w] (the upsampled LR latent; with the native anchor
        the LR latent itself, [in_dim, chunk, 2h_a, 2w_a]), noised to
        ``anchor_harvest_t`` when that is above 0, through the model at that
        timestep with no cache; each layer's K/V become its ring's anchor."""
        if self.anchor is None:
            raise RuntimeError("StreamingRefiner.harvest: the refiner was built without an anchor.")
        x = lq
        if self.harvest_t > 0:
            sig = self.harvest_t / self.sched.num_train_timesteps
            noise = torch.randn(lq.shape, generator=self.gen, device=self.device, dtype=lq.dtype)
            x = (1.0 - sig) * lq + sig * noise
        self._launch(("harvest", 0), self.harvest_t, x, t_offset, self._run_harvest)

    def commit(self):
        for r in self.rings:
            r.commit(self.chunk)

    # ---- the loop -----------------------------------------------------------
    def refine_chunk(self, noisy, t_offset, lq=None):
        """Denoise one chunk from ``noisy`` (at the first step's noise level) and
        refresh the caches with it; returns x0 [out_dim, chunk, 2h, 2w] fp32.
        ``lq``: the chunk's upsampled LR latent, harvested as the anchor first
        (required with an anchor)."""
        if self.anchor is not None:
            if lq is None:
                raise ValueError("StreamingRefiner: an anchored refiner needs the LQ chunk.")
            self.harvest(lq, t_offset)
        x0 = None
        for i, t in enumerate(self.steps):
            if self._vary_scale:
                self._scale_dev.fill_(self.anchor_scales[min(i, len(self.anchor_scales) - 1)])
            flow = self.forward(noisy, t, t_offset, anchored=True)
            x0 = (noisy.double() - (t / self.sched.num_train_timesteps) * flow.double()).to(flow.dtype)
            if i + 1 < len(self.steps):
                noise = torch.randn(x0.shape, generator=self.gen, device=self.device,
                                    dtype=x0.dtype)
                noisy = self.sched.add_noise(x0, noise, self.steps[i + 1])
        self.refresh(x0, t_offset)
        self.commit()
        return x0

    def run(self, noise, t_offset=0, lq=None, lq_anchor=None):
        """``noise`` [in_dim, F, 2h, 2w] with F a multiple of ``chunk``: refine every
        chunk in order; returns the refined latent [out_dim, F, 2h, 2w].  ``lq``
        (same shape): the upsampled LR latent; the first noisy input is then
        ``(1 - sigma_start) * lq + sigma_start * noise`` (causal_inference.py:667-668)
        and each chunk's anchor is harvested from it, or from ``lq_anchor`` (the
        native LR latent, [in_dim, F, 2h_a, 2w_a]) with the native anchor."""
        frames = noise.shape[1]
        if frames % self.chunk:
            raise ValueError(f"StreamingRefiner: {frames} frames is not a multiple of {self.chunk}.")
        if lq is not None and lq.shape != noise.shape:
            raise ValueError("StreamingRefiner.run: lq and noise must have the same shape.")
        noisy = noise if lq is None else (1.0 - self.sigma_start) * lq + self.sigma_start * noise
        src = lq if lq_anchor is None else lq_anchor
        outs = []
        for c0 in range(0, frames, self.chunk):
            sl = slice(c0, c0 + self.chunk)
            outs.append(self.refine_chunk(noisy[:, sl], t_offset + c0,
                                          None if src is None else src[:, sl]))
        return torch.cat(outs, 1)
