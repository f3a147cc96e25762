"""Streaming SR denoise loop: chunks of latent frames, few-step flow matching,
KV-cache refresh, on the in-place ring caches and HIP graphs.

Restates the per-chunk loop of CausalInferencePipeline.inference_sr
(video_refiner/pipeline_sr/causal_inference.py:858-976) for one sample without
the LQ anchor:

  for each chunk of ``chunk`` latent frames (temporal offset advancing by chunk):
      for each timestep t of the step list:
          flow = model(noisy, t)             # attends the cached frames + the chunk
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
no per-call concatenation); the text K/V of every layer are computed once per
video; and each model forward is one HIP graph replay, captured once per cache
length (the ring's position is read by the kernels from device memory, so one
graph serves every chunk once the cache is full).
"""
from __future__ import annotations

import torch

from .kv_ring import KVRing
from .model import rope_table


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
    graph (captured at the first forward with a given cache length).
    ``ring_cat`` (tests only) makes every layer read the reference's
    concatenation of its cache with the chunk instead of the ring in place.
    """

    def __init__(self, model, h, w, context_raw, *, chunk=3, kv_len=9,
                 step_list=(1000, 750, 500, 250), warp=True, context_noise=0,
                 sigma_start=1.0, shift=5.0, block_hw=(4, 4), block_radius_hw=(3, 3),
                 use_graph=True, seed=0, device="cuda", ring_cat=False):
        cfg = model.cfg
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
        self.rings = [KVRing(1, kv_len, chunk, L, cfg.num_heads, cfg.head_dim,
                             device=self.device) for _ in model.blocks]
        self.gen = torch.Generator(device=self.device).manual_seed(seed)
        with torch.no_grad():
            self.ctx = model.embed_text(context_raw.to(self.device))
            g0 = self._geom(0, 0)
            self.cross = model.cross_cache(self.ctx, g0)
        # static inputs of the captured forwards
        self._lat = torch.zeros(cfg.in_dim, chunk, 2 * h, 2 * w, dtype=torch.float32,
                                device=self.device)
        self._e = torch.zeros(1, cfg.dim, dtype=torch.float32, device=self.device)
        self._e0 = torch.zeros(1, 6, cfg.dim, dtype=torch.float32, device=self.device)
        self._geoms = {}
        self._graphs = {}
        self.forwards = 0

    # ---- one model forward --------------------------------------------------
    def _geom(self, cached, t_offset):
        return self.model.stream_geometry(self.chunk, self.h, self.w, self.ctx.shape[0],
                                          self.device, cached=cached, chunk=self.chunk,
                                          t_offset=t_offset, block_hw=self.block_hw,
                                          block_radius_hw=self.block_radius_hw)

    def _static_geom(self, cached, t_offset):
        """The geometry for this cache length, its RoPE table refreshed in place for
        ``t_offset`` (so a captured graph sees the new table)."""
        g = self._geoms.get(cached)
        if g is None:
            g = self._geoms[cached] = self._geom(cached, t_offset)
            g["t_offset"] = t_offset
            g["ring_cat"] = self.ring_cat
        elif g["t_offset"] != t_offset:
            rope = rope_table(self.model.cfg, self.chunk, self.h, self.w, t_offset, self.device)
            g["rope"].copy_(rope)
            g["rope_cs"].copy_(torch.view_as_real(rope).reshape(g["rope_cs"].shape))
            g["t_offset"] = t_offset
        return g

    def _run(self, geom):
        return self.model.forward_embedded(self._lat, self._e, self._e0, self.ctx, geom,
                                           rings=self.rings, cross=self.cross)

    def forward(self, latent, t, t_offset):
        """Flow prediction for the chunk ``latent`` [in_dim, chunk, 2h, 2w] at timestep
        ``t``, attending the cached frames; writes the chunk's K/V into the rings'
        current regions (kept only by ``commit``)."""
        cached = self.rings[0].cached
        with torch.no_grad():
            e, e0 = self.model.time_embed(torch.tensor([float(t)], device=self.device))
            self._e.copy_(e)
            self._e0.copy_(e0)
            self._lat.copy_(latent)
            geom = self._static_geom(cached, t_offset)
            self.forwards += 1
            if not self.use_graph:
                return self._run(geom)
            entry = self._graphs.get(cached)
            if entry is None:
                self._run(geom)  # plans, device tables, library handles: outside capture
                torch.cuda.synchronize(self.device)
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    out = self._run(geom)
                entry = self._graphs[cached] = (graph, out)
            entry[0].replay()
            return entry[1]

    def commit(self):
        for r in self.rings:
            r.commit(self.chunk)

    # ---- the loop -----------------------------------------------------------
    def refine_chunk(self, noisy, t_offset):
        """Denoise one chunk from ``noisy`` (at the first step's noise level) and
        refresh the caches with it; returns x0 [out_dim, chunk, 2h, 2w] fp32."""
        x0 = None
        for i, t in enumerate(self.steps):
            flow = self.forward(noisy, t, t_offset)
            x0 = (noisy.double() - (t / self.sched.num_train_timesteps) * flow.double()).to(flow.dtype)
            if i + 1 < len(self.steps):
                noise = torch.randn(x0.shape, generator=self.gen, device=self.device,
                                    dtype=x0.dtype)
                noisy = self.sched.add_noise(x0, noise, self.steps[i + 1])
        self.forward(x0, self.context_noise, t_offset)  # refresh pass
        self.commit()
        return x0

    def run(self, noise, t_offset=0):
        """``noise`` [in_dim, F, 2h, 2w] with F a multiple of ``chunk``: refine every
        chunk in order; returns the refined latent [out_dim, F, 2h, 2w]."""
        frames = noise.shape[1]
        if frames % self.chunk:
            raise ValueError(f"StreamingRefiner: {frames} frames is not a multiple of {self.chunk}.")
        outs = []
        for c0 in range(0, frames, self.chunk):
            outs.append(self.refine_chunk(noise[:, c0:c0 + self.chunk], t_offset + c0))
        return torch.cat(outs, 1)
