"""In-place streaming KV cache for the block-grid window attention.

The reference keeps each layer's streaming cache as a tensor, and every call
of the op concatenates it with the chunk's K/V and slices the last ``kv_len``
frames off as the next cache (video_refiner/wan/modules/sr_dit/attention.py:
1506-1510, :964-974).  That copies the whole cache on every layer of every
denoising step.  ``KVRing`` keeps one buffer per layer instead, laid out as

    [anchor prefix: A tokens][ring: R = kv_len slots of L tokens][current chunk: F frames of L]

with the cached frames in the ring, oldest first starting at slot ``head``,
and the chunk being denoised in the fixed region after it.  The window kernels
map logical KV frame ``f`` (the frame index of the plan) to slot
``(head + f) % R`` for ``f < cached`` and to ``R + (f - cached)`` otherwise, so
an attention call copies nothing but the chunk's own K/V (nothing at all when
the producer writes into ``current_k``/``current_v``).  ``commit`` moves the
chunk into the ring -- the reference's "keep the tail" -- by copying ``F``
frames and advancing ``head``.  ``head`` also lives in a device int32 that the
kernels read at launch, so a captured launch follows the ring across chunks.
"""
from __future__ import annotations

import torch


class KVRing:
    """Streaming K/V cache of one attention layer, kept in place.

    ``batch`` samples share one ring position (they advance chunk by chunk
    together).  ``kv_len`` is the reference's cache budget in latent frames
    (the ring's slot count R); ``chunk_frames`` the largest chunk (F);
    ``frame_tokens`` = h*w; ``anchor_tokens`` reserves the LQ-anchor prefix
    (f_cur * anchor frame tokens, 0 without an anchor).
    """

    def __init__(self, batch, kv_len, chunk_frames, frame_tokens, n_heads, head_dim, *,
                 anchor_tokens=0, dtype=torch.bfloat16, device="cuda"):
        if kv_len is None or int(kv_len) < 1:
            raise ValueError(f"KVRing needs kv_len >= 1 frames, got {kv_len!r}.")
        if int(chunk_frames) < 1 or int(frame_tokens) < 1 or int(batch) < 1:
            raise ValueError("KVRing: batch, chunk_frames and frame_tokens must be positive.")
        self.R = int(kv_len)
        self.F = int(chunk_frames)
        self.L = int(frame_tokens)
        self.A = int(anchor_tokens)
        self.n_heads, self.head_dim = int(n_heads), int(head_dim)
        tokens = self.A + (self.R + self.F) * self.L
        shape = (int(batch), tokens, self.n_heads, self.head_dim)
        self.k = torch.zeros(shape, dtype=dtype, device=device)
        self.v = torch.zeros(shape, dtype=dtype, device=device)
        self.head_dev = torch.zeros(1, dtype=torch.int32, device=device)
        self.head = 0     # slot of the oldest cached frame (host copy of head_dev)
        self.cached = 0   # cached frames, <= R

    # ---- layout ---------------------------------------------------------------
    @property
    def batch(self) -> int:
        return self.k.shape[0]

    def physical_frame(self, f: int) -> int:
        """Frame index within the HR region of logical KV frame ``f`` (the kernels' mapping)."""
        if f < self.cached:
            return (self.head + f) % self.R
        return self.R + (f - self.cached)

    def _hr(self, t, i, frame, nframes=1):
        s = self.A + frame * self.L
        return t[i, s:s + nframes * self.L]

    def current_k(self, i: int, f_cur: int | None = None) -> torch.Tensor:
        """``[f_cur*L, n, d]`` view of sample ``i``'s chunk K (write the chunk's K here)."""
        return self._hr(self.k, i, self.R, self.F if f_cur is None else f_cur)

    def current_v(self, i: int, f_cur: int | None = None) -> torch.Tensor:
        return self._hr(self.v, i, self.R, self.F if f_cur is None else f_cur)

    def anchor_k(self, i: int, tokens: int | None = None) -> torch.Tensor:
        return self.k[i, :self.A if tokens is None else tokens]

    def anchor_v(self, i: int, tokens: int | None = None) -> torch.Tensor:
        return self.v[i, :self.A if tokens is None else tokens]

    def kernel_ring(self):
        """``(ring_frames, ring_cached, head)`` as the launcher takes it."""
        return (self.R, self.cached, self.head_dev)

    # ---- state ----------------------------------------------------------------
    def logical(self, i: int):
        """Sample ``i``'s cached K/V in frame order, ``[cached*L, n, d]`` copies: what the
        reference holds as its cache tensor."""
        if self.cached == 0:
            empty = self.k.new_empty(0, self.n_heads, self.head_dim)
            return empty, empty.clone()
        fr = [self.physical_frame(f) for f in range(self.cached)]
        k = torch.cat([self._hr(self.k, i, p) for p in fr], 0)
        v = torch.cat([self._hr(self.v, i, p) for p in fr], 0)
        return k, v

    def load(self, cache_k, cache_v):
        """Start from an existing cache ``[b, frames*L, n, d]`` (the reference's
        layout; the last ``kv_len`` frames are kept)."""
        if cache_k.shape != cache_v.shape or cache_k.shape[0] != self.batch:
            raise ValueError("KVRing.load: cache_k/cache_v must be [batch, frames*L, n, d].")
        frames = cache_k.shape[1] // self.L
        if frames * self.L != cache_k.shape[1]:
            raise ValueError("KVRing.load: the cache is not aligned to whole frames.")
        keep = min(frames, self.R)
        first = frames - keep
        for i in range(self.batch):
            for f in range(keep):
                src = slice((first + f) * self.L, (first + f + 1) * self.L)
                self._hr(self.k, i, f).copy_(cache_k[i, src])
                self._hr(self.v, i, f).copy_(cache_v[i, src])
        self.head, self.cached = 0, keep
        self.head_dev.fill_(0)

    def reset(self):
        self.head, self.cached = 0, 0
        self.head_dev.fill_(0)

    def write_current(self, i: int, k_i: torch.Tensor, v_i: torch.Tensor):
        """Copy the chunk's K/V of sample ``i`` into the current region, unless the
        producer already wrote them there."""
        f_tok = k_i.shape[0]
        if f_tok % self.L or f_tok // self.L > self.F or v_i.shape != k_i.shape:
            raise ValueError(f"KVRing: chunk of {f_tok} tokens does not fit {self.F} frames "
                             f"of {self.L} tokens.")
        for src, dst in ((k_i, self.current_k(i, f_tok // self.L)),
                         (v_i, self.current_v(i, f_tok // self.L))):
            if src.data_ptr() != dst.data_ptr():
                dst.copy_(src)

    def write_anchor(self, i: int, ak: torch.Tensor, av: torch.Tensor):
        n = ak.shape[0]
        if n > self.A or av.shape != ak.shape:
            raise ValueError(f"KVRing: anchor of {n} tokens does not fit the {self.A}-token prefix.")
        for src, dst in ((ak, self.anchor_k(i, n)), (av, self.anchor_v(i, n))):
            if src.data_ptr() != dst.data_ptr():
                dst.copy_(src)

    def commit(self, f_new: int):
        """Append the current chunk's first ``f_new`` frames to the cache, keeping the
        last ``kv_len`` frames: the reference's cat + tail slice, done by copying the
        new frames into the slots of the evicted ones."""
        f_new = int(f_new)
        if not 0 <= f_new <= self.F:
            raise ValueError(f"KVRing.commit: {f_new} frames, the chunk region holds {self.F}.")
        total = self.cached + f_new
        keep = min(total, self.R)
        evict = total - keep
        for j in range(f_new):
            if self.cached + j - evict < 0:
                continue  # older than the last kv_len frames
            slot = (self.head + self.cached + j) % self.R
            dst = self.A + slot * self.L
            src = self.A + (self.R + j) * self.L
            for t in (self.k, self.v):
                t[:, dst:dst + self.L].copy_(t[:, src:src + self.L])
        self.head = (self.head + evict) % self.R
        self.cached = keep
        self.head_dev.fill_(self.head)
