"""Block-grid window self-attention: geometry and the op entry.

Query blocks hard-partition the ``(f, h, w)`` latent grid into
``(block_t, bh, bw)`` cuboids; every block attends its boundary-clamped
``(rh, rw)`` spatial block neighbourhood over a temporal span given by a
temporal rule.  Visibility is the set of addressed KV tokens, so the path is
mask-free.

This module mirrors the reference op surface
(video_refiner/wan/modules/sr_dit/attention.py):

* ``_blockgrid_neighbours`` / ``_blockgrid_axis_blocks``     (attention.py:261-290)
* ``_anchor_grid_stride``                                     (attention.py:293-328)
* ``_BlockGridSpec`` with ``temporal_runs``                   (attention.py:348-512)
* ``_truncate_kv_cache``                                      (attention.py:964-974)
* ``mask_free_window_attention``                              (attention.py:1376-1648)

with one execution backend, ``attn_impl="hip"`` (the fused HIP kernel in
``libsrdit_hip.so``).  The reference's gather / flex / magi / triton backends
are not provided here; asking for them raises rather than silently running
something else.

One addition: the symmetric temporal rule (``sym_radius_t``): query frame
``t`` sees KV frames ``[t - r, t + r]`` clamped to the grid, expressed as
per-frame runs in the same ``(q_f0, q_f1, kv_f0, kv_f1)`` format.  The
reference has no such rule; it is selected only by the new keyword and every
reference code path is unchanged when it is absent.
"""
from __future__ import annotations

import warnings

from typing import NamedTuple

import torch

from . import blockgrid_hip as _bgh

#: Looked up as a module global at call time, so tests can swap the launcher
#: (the seam of attention.py:45-46).
_run_blockgrid_hip = _bgh.run_blockgrid_hip

#: Backends this op accepts.  Only "hip" executes; it is also what "auto"
#: resolves to.  Anything else raises (attention.py:805-808, :1493-1497).
BLOCKGRID_IMPLS = ("auto", "hip")


def _blockgrid_neighbours(nb, b, radius):
    """Inclusive clamped neighbour block range ``[max(0, b-r), min(nb-1, b+r)]``.

    Clamping keeps the range contiguous, so a neighbourhood is one KV interval
    (attention.py:261-269).
    """
    return max(0, b - radius), min(nb - 1, b + radius)


def _blockgrid_axis_blocks(size, block, radius):
    """Per-block ``(q_start, q_len, kv_start, kv_len)`` along one axis.

    Blocks tile ``[0, size)``; the last block is shorter when ``block`` does not
    divide ``size``.  The KV span of block ``b`` is the token interval covered
    by its neighbour blocks (attention.py:272-290).
    """
    nb = -(-size // block)
    out = []
    for b in range(nb):
        q0 = b * block
        q1 = min(q0 + block, size)
        lo, hi = _blockgrid_neighbours(nb, b, radius)
        k0 = lo * block
        k1 = min((hi + 1) * block, size)
        out.append((q0, q1 - q0, k0, k1 - k0))
    return out


def _anchor_grid_stride(h, w, bh, bw, anchor_hw):
    """``(s_h, s_w)`` of a coarser anchor grid; raises unless it divides exactly.

    The anchor grid ``(h_a, w_a)`` must divide the query grid, and the stride
    must divide the block size, so every window's anchor extent is an integer
    (attention.py:293-328).
    """
    if anchor_hw is None:
        return 1, 1
    h_a, w_a = int(anchor_hw[0]), int(anchor_hw[1])
    if h_a <= 0 or w_a <= 0:
        raise ValueError(f"anchor_hw must be positive, got {(h_a, w_a)}.")
    if h % h_a or w % w_a:
        raise ValueError(
            f"anchor grid {(h_a, w_a)} must divide the query token grid {(h, w)}: "
            f"h % h_a = {h % h_a}, w % w_a = {w % w_a}.")
    s_h, s_w = h // h_a, w // w_a
    if bh % s_h or bw % s_w:
        raise ValueError(
            f"anchor stride {(s_h, s_w)} must divide the query block size {(bh, bw)}: "
            f"bh % s_h = {bh % s_h}, bw % s_w = {bw % s_w}.")
    return s_h, s_w


class _BlockGridSpec(NamedTuple):
    """One block-grid window geometry: the single definition of visibility.

    Fields follow attention.py:387-401; ``sym_rt`` is appended (default None).

    f_cur, f_kv: query / KV latent frame counts (f_kv > f_cur means a cache).
    h, w: token grid.  block_t, bh, bw: query block size.  rh, rw: spatial
    radius in blocks.  hist: chunk-anchored history depth in frames (None
    selects the legacy ``rt`` rule).  rt: legacy temporal radius in block_t
    units.  chunk_frames: frames per causal chunk.  streaming: a cache and/or
    an anchor is present.  query_grain: "grid" or "chunk".  anchor_hw: the
    anchor's own coarser grid, or None.  sym_rt: symmetric temporal radius in
    frames (per-frame query runs); None keeps the reference rules.
    """

    f_cur: int
    f_kv: int
    h: int
    w: int
    block_t: int
    bh: int
    bw: int
    rh: int
    rw: int
    hist: int | None = None
    rt: int = 0
    chunk_frames: int | None = None
    streaming: bool = False
    query_grain: str = "grid"
    anchor_hw: tuple | None = None
    sym_rt: int | None = None

    def h_blocks(self):
        return _blockgrid_axis_blocks(self.h, self.bh, self.rh)

    def w_blocks(self):
        return _blockgrid_axis_blocks(self.w, self.bw, self.rw)

    def anchor_stride(self):
        return _anchor_grid_stride(self.h, self.w, self.bh, self.bw, self.anchor_hw)

    def anchor_h_blocks(self):
        """Per-block anchor row extent: the HR extent divided by the stride."""
        s = self.anchor_stride()[0]
        return [(q0, qL, k0 // s, kL // s) for (q0, qL, k0, kL) in self.h_blocks()]

    def anchor_w_blocks(self):
        s = self.anchor_stride()[1]
        return [(q0, qL, k0 // s, kL // s) for (q0, qL, k0, kL) in self.w_blocks()]

    @property
    def anchor_grid(self):
        if self.anchor_hw is None:
            return int(self.h), int(self.w)
        return int(self.anchor_hw[0]), int(self.anchor_hw[1])

    @property
    def anchor_frame_tokens(self) -> int:
        h_a, w_a = self.anchor_grid
        return h_a * w_a

    @property
    def one_query_run(self) -> bool:
        """The query time axis is one run (streaming, chunk grain or a longer KV)."""
        return (bool(self.streaming) or self.query_grain != "grid"
                or self.f_kv != self.f_cur)

    def temporal_runs(self):
        """``(q_f0, q_f1, kv_f0, kv_f1)`` frame runs partitioning the query frames.

        Rules (attention.py:457-512):
          * ``hist`` set, chunk-anchored: chunk ``[c0, c1)`` sees
            ``[max(0, c0 - hist), c1)``; a single run sees
            ``[max(0, f_kv - f_cur - hist), f_kv)``.
          * ``hist`` None, legacy: query block ``i`` sees
            ``[max(0, i - rt) * bt, (i + 1) * bt)``; a single run sees the tail
            ``[max(0, f_kv - (rt + 1) * bt), f_kv)``; a sub-block query grid
            sees everything.
          * ``sym_rt`` set (an addition, not a reference rule): query frame ``t`` (KV frame
            ``t + f_kv - f_cur``) sees ``[t' - r, t' + r]`` clamped to
            ``[0, f_kv)``.
        """
        f_cur, f_kv = int(self.f_cur), int(self.f_kv)
        if self.query_grain not in ("grid", "chunk"):
            raise ValueError(
                f"query_grain must be 'grid'|'chunk', got {self.query_grain!r}.")
        if self.sym_rt is not None:
            r = int(self.sym_rt)
            if r < 0:
                raise ValueError(f"sym_rt must be >= 0, got {r}.")
            off = f_kv - f_cur
            runs = [(t, t + 1, max(0, t + off - r), min(f_kv, t + off + r + 1))
                    for t in range(f_cur)]
        elif self.hist is not None:
            hist = int(self.hist)
            cf = int(self.chunk_frames) if self.chunk_frames else max(1, f_cur)
            if self.one_query_run or f_cur <= cf:
                runs = [(0, f_cur, max(0, f_kv - f_cur - hist), f_kv)]
            else:
                runs = [(c0, min(c0 + cf, f_cur), max(0, c0 - hist),
                         min(f_kv, min(c0 + cf, f_cur)))
                        for c0 in range(0, f_cur, cf)]
        else:
            bt, rt = int(self.block_t), int(self.rt)
            if self.one_query_run:
                runs = [(0, f_cur, max(0, f_kv - (rt + 1) * bt), f_kv)]
            elif f_cur < bt:
                runs = [(0, f_cur, 0, f_kv)]
            else:
                runs = [(i * bt, (i + 1) * bt, max(0, i - rt) * bt, (i + 1) * bt)
                        for i in range(f_cur // bt)]
        covered = sum(q1 - q0 for (q0, q1, _, _) in runs)
        if not runs or covered != f_cur or runs[0][0] != 0 or runs[-1][1] != f_cur:
            raise ValueError(
                f"temporal runs {runs} do not partition the {f_cur} query frames "
                f"(covered {covered}); block_t={self.block_t} must divide f_cur in "
                f"the partitioned regimes.")
        return runs


def _truncate_kv_cache(full_k, full_v, kv_len, L, f_kv):
    """Keep the last ``kv_len`` frames of the KV (a view; attention.py:964-974)."""
    if kv_len is None or f_kv <= kv_len:
        return full_k, full_v
    keep = int(kv_len) * L
    return full_k[-keep:], full_v[-keep:]


def _blockgrid_hip_attend(spec, q_i, full_k, full_v, *, anchor_k=None,
                          anchor_v=None, anchor_align="frame",
                          anchor_window_scope="window", ring=None, sample=0):
    """Fused execution of one sample's windows -> ``[f_cur*h*w, n, d]``.

    Guards follow attention.py:842-863 and raise instead of degrading:
    not a GPU tensor, a head dim other than 64 or 128, autograd, a global
    anchor scope, an unsupported dtype.  With ``ring`` (a ``KVRing`` whose
    current region already holds the chunk) ``full_k``/``full_v`` are unused:
    the anchor is written into the ring's prefix and the kernel reads the
    cache in place.
    """
    f_cur, h, w = spec.f_cur, spec.h, spec.w
    n, d = q_i.shape[1], q_i.shape[2]
    anchor_given = anchor_k is not None
    if not q_i.is_cuda:
        raise RuntimeError('attn_impl="hip" runs on the GPU only; q is on the CPU.')
    if d not in (64, 128):
        raise ValueError(f'attn_impl="hip" supports head_dim 64 or 128, got {d}.')
    if q_i.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f'attn_impl="hip" needs bf16 or fp16 inputs, got {q_i.dtype}.')
    if torch.is_grad_enabled() and any(
            t is not None and t.requires_grad
            for t in (q_i, full_k, full_v, anchor_k, anchor_v)):
        raise RuntimeError(
            'attn_impl="hip" is forward-only (the kernel records nothing for '
            "autograd), but grad is enabled and an input requires grad.")
    if anchor_given and anchor_window_scope != "window":
        raise ValueError(
            f'attn_impl="hip" only supports anchor_window_scope="window", got '
            f"{anchor_window_scope!r}: a params row carries one spatial extent "
            f"shared by the anchor and the HR cuboid.")
    anchor_mode = (None if not anchor_given
                   else ("frame" if anchor_align == "frame" else "chunk"))
    plan = _bgh.cached_plan(spec, anchor_mode=anchor_mode)
    if ring is not None:
        if anchor_given:
            ring.write_anchor(sample, anchor_k, anchor_v)
        out_i = q_i.new_empty(f_cur * h * w, n, d)
        return _run_blockgrid_hip(
            q_i.contiguous(), ring.k[sample], ring.v[sample], out_i, plan=plan, f_cur=f_cur,
            h=h, w=w, n=n, d=d, anchor_mode=anchor_mode, ring=ring.kernel_ring(),
            hr_base=ring.A)
    if anchor_given:
        k_ext = torch.cat([anchor_k, full_k], dim=0)
        v_ext = torch.cat([anchor_v, full_v], dim=0)
    else:
        k_ext, v_ext = full_k, full_v
    out_i = q_i.new_empty(f_cur * h * w, n, d)
    return _run_blockgrid_hip(
        q_i.contiguous(), k_ext.contiguous(), v_ext.contiguous(), out_i,
        plan=plan, f_cur=f_cur, h=h, w=w, n=n, d=d, anchor_mode=anchor_mode)


def _check_ring(ring, gs, b, n, d, pre_cache_k, pre_cache_v, kv_len):
    """Argument checks of the in-place cache path (raise, never degrade)."""
    if pre_cache_k is not None or pre_cache_v is not None:
        raise ValueError("mask_free_window_attention: pass either kv_ring or "
                         "pre_cache_k/pre_cache_v, not both.")
    if kv_len is not None and int(kv_len) != ring.R:
        raise ValueError(f"mask_free_window_attention: kv_len={kv_len} but the ring keeps "
                         f"{ring.R} frames.")
    if ring.batch != b or ring.n_heads != n or ring.head_dim != d:
        raise ValueError("mask_free_window_attention: kv_ring shape does not match q.")
    if any(list(g) != list(gs[0]) for g in gs):
        raise ValueError("mask_free_window_attention: a kv_ring advances all samples "
                         "together; grid_sizes must be equal.")
    f_cur, h, w = (int(x) for x in gs[0])
    if h * w != ring.L or f_cur > ring.F:
        raise ValueError(f"mask_free_window_attention: grid {(f_cur, h, w)} does not fit the "
                         f"ring ({ring.F} frames of {ring.L} tokens).")


def mask_free_window_attention(
    q, k, v, grid_sizes,
    pre_cache_k=None,
    pre_cache_v=None,
    kv_len=None,
    anchor_k=None,
    anchor_v=None,
    anchor_align="frame",
    anchor_window_scope="window",
    anchor_hw=None,
    anchor_keep=None,
    attn_impl="auto",
    win_chunk=None,
    causal_chunk_frames=None,
    causal_kv_span=None,
    block_t=None,
    block_hw=(4, 4),
    block_radius_hw=(2, 2),
    block_radius_t=None,
    sym_radius_t=None,
    kv_ring=None,
    kv_commit=False,
):
    """Mask-free block-grid window self-attention with an optional KV cache.

    Signature and return contract of attention.py:1376-1395 / :1645-1648:
    ``q, k, v`` are ``[b, s_cur, n, d]`` (q and k already RoPE'd),
    ``grid_sizes`` is ``[b, 3] = (f_cur, h, w)``; the return value is
    ``(out [b, s_cur, n, d], new_cache_k, new_cache_v)`` with the caches
    ``[b, kept*h*w, n, d]``.  ``win_chunk`` is accepted for signature
    compatibility; the fused kernel never gathers, so it has no effect.

    ``sym_radius_t`` (not in the reference): select the symmetric temporal
    rule, query frame ``t`` seeing frames ``[t - r, t + r]``.

    ``kv_ring`` (not in the reference): a ``sr_dit.kv_ring.KVRing`` holding
    the streaming cache in place of ``pre_cache_k``/``pre_cache_v``.  The
    chunk's K/V go into the ring's current region (no copy when ``k``/``v``
    already are those views), the attention reads the cache where it lies,
    and with ``kv_commit`` the chunk is appended to the cache afterwards,
    keeping the last ``kv_ring.R`` frames (the reference's cat + tail slice,
    attention.py:1506-1510, :964-974).  The second and third return values
    are then the ring itself.  A ring counts as a cache for the streaming
    rule even while it is empty, as an empty cache tensor does.
    """
    b, s_cur, n, d = q.shape
    impl = str(attn_impl)
    if impl not in BLOCKGRID_IMPLS:
        raise ValueError(f"attn_impl must be one of {BLOCKGRID_IMPLS}, got {impl!r}.")
    if sym_radius_t is not None and block_radius_t is not None:
        raise ValueError("sym_radius_t and block_radius_t select different temporal "
                         "rules; pass one of them.")
    outs, new_ck, new_cv = [], [], []
    anchor_hw_arg = None if anchor_hw is None else (int(anchor_hw[0]), int(anchor_hw[1]))
    gs = grid_sizes.tolist() if torch.is_tensor(grid_sizes) else [list(g) for g in grid_sizes]
    if kv_ring is not None:
        _check_ring(kv_ring, gs, b, n, d, pre_cache_k, pre_cache_v, kv_len)
    for i in range(b):
        f_cur, h, w = (int(x) for x in gs[i])
        if f_cur * h * w != s_cur:
            raise ValueError(f"grid {(f_cur, h, w)} inconsistent with s_cur={s_cur}")
        q_i, k_i, v_i = q[i], k[i], v[i]
        if kv_ring is not None:
            kv_ring.write_current(i, k_i, v_i)
            full_k = full_v = None
            f_kv = kv_ring.cached + f_cur
        else:
            if pre_cache_k is not None and pre_cache_v is not None:
                full_k = torch.cat([pre_cache_k[i], k_i], dim=0)
                full_v = torch.cat([pre_cache_v[i], v_i], dim=0)
            else:
                full_k, full_v = k_i, v_i
            s_kv = full_k.shape[0]
            f_kv = s_kv // (h * w)
            if f_kv * h * w != s_kv:
                raise ValueError("KV cache is not aligned to whole frames")

        anchor_given = (anchor_k is not None) or (anchor_v is not None)
        use_anchor = anchor_given
        a_hw = None if anchor_hw_arg is None or anchor_hw_arg == (h, w) else anchor_hw_arg
        if anchor_given:
            if anchor_k is None or anchor_v is None:
                raise ValueError("mask_free_window_attention: anchor_k and anchor_v "
                                 "must be provided together.")
            if (causal_chunk_frames is not None and causal_kv_span is not None
                    and pre_cache_k is None and pre_cache_v is None):
                raise NotImplementedError(
                    "LQ-anchor in the parallel chunk-causal window path is not "
                    "supported; anchor injection requires the streaming path (KV "
                    "cache present) or a plain bidirectional window forward.")
            s_h, s_w = _anchor_grid_stride(h, w, int(block_hw[0]), int(block_hw[1]), a_hw)
            L_a = (h // s_h) * (w // s_w)
            if anchor_align not in ("frame", "chunk"):
                raise ValueError(f"anchor_align must be 'frame' or 'chunk', got {anchor_align!r}.")
            if anchor_window_scope not in ("window", "global"):
                raise ValueError("anchor_window_scope must be 'window' or 'global', "
                                 f"got {anchor_window_scope!r}.")
            if anchor_k.shape[1] != f_cur * L_a:
                raise ValueError(
                    f"frame-aligned LQ-anchor needs f_cur*L_a = {f_cur * L_a} tokens "
                    f"per sample, got anchor_k sequence length {anchor_k.shape[1]}.")
            if anchor_keep is not None:
                keep_i = (anchor_keep.view(-1)[i] if torch.is_tensor(anchor_keep)
                          else anchor_keep[i])
                use_anchor = bool(keep_i)

        if block_t is None and causal_chunk_frames is None:
            # attention.py:1575 evaluates int(None) here and raises TypeError.
            raise TypeError("mask_free_window_attention: block_t or causal_chunk_frames "
                            "must be given for the block-grid path.")
        bt = int(block_t if block_t is not None else causal_chunk_frames)
        if bt <= 0:
            raise ValueError(f"block_t must be positive, got {bt}.")
        is_streaming = (pre_cache_k is not None or pre_cache_v is not None or anchor_given
                        or kv_ring is not None)
        hist = None if block_radius_t is None else (2 * int(block_radius_t) + 1) * bt
        if sym_radius_t is None:
            if hist is None:
                if not is_streaming and f_cur % bt != 0 and f_cur >= bt:
                    raise ValueError(
                        f"block-grid window attention needs f_cur ({f_cur}) to be a "
                        f"multiple of block_t ({bt}).")
            elif not is_streaming and causal_chunk_frames:
                cf = int(causal_chunk_frames)
                if f_cur % cf != 0 and f_cur >= cf:
                    raise ValueError(
                        f"chunk-anchored block-grid windows need f_cur ({f_cur}) to be "
                        f"a multiple of causal_chunk_frames ({cf}).")
        rt = (int(causal_kv_span) // bt - 1) if causal_kv_span is not None else (f_kv // bt - 1)
        rt = max(rt, 0)
        spec = _BlockGridSpec(
            f_cur=f_cur, f_kv=f_kv, h=h, w=w, block_t=bt,
            bh=int(block_hw[0]), bw=int(block_hw[1]),
            rh=int(block_radius_hw[0]), rw=int(block_radius_hw[1]),
            hist=hist, rt=rt,
            chunk_frames=None if causal_chunk_frames is None else int(causal_chunk_frames),
            streaming=is_streaming,
            anchor_hw=(a_hw if anchor_given else None),
            sym_rt=None if sym_radius_t is None else int(sym_radius_t))
        out_i = _blockgrid_hip_attend(
            spec, q_i, full_k, full_v,
            anchor_k=(anchor_k[i] if use_anchor else None),
            anchor_v=(anchor_v[i] if use_anchor else None),
            anchor_align=anchor_align, anchor_window_scope=anchor_window_scope,
            ring=kv_ring, sample=i)
        outs.append(out_i)
        if kv_ring is None:
            ck_i, cv_i = _truncate_kv_cache(full_k, full_v, kv_len, h * w, f_kv)
            new_ck.append(ck_i)
            new_cv.append(cv_i)

    if kv_ring is not None:
        if kv_commit:
            kv_ring.commit(int(gs[0][0]))
        out = outs[0].unsqueeze(0) if b == 1 else torch.stack(outs, 0)
        return out, kv_ring, kv_ring
    if b == 1:
        return outs[0].unsqueeze(0), new_ck[0].unsqueeze(0), new_cv[0].unsqueeze(0)
    return torch.stack(outs, 0), torch.stack(new_ck, 0), torch.stack(new_cv, 0)


def prewarm_blockgrid_hip(*, h, w, bt, bh, bw, rh, rw, n, d, variants,
                          block_radius_t=None, f_kv=None, device=None,
                          dtype=torch.bfloat16, anchor_hw=None):
    """Counterpart of ``prewarm_blockgrid_triton`` (attention.py:883-961).

    The HIP kernels are compiled ahead of time, so nothing is JIT-compiled;
    each ``(f_cur, anchor_mode)`` variant is still launched once on zero
    tensors of the production geometry, which builds its plan, uploads the
    plan's device tables (params, launch order, member tables) and pays the
    first launch before inference.  Same signature and return contract: the
    variants warmed, ``[]`` without a GPU; a variant the planner or the
    launcher rejects is skipped with a warning, never raised.
    """
    if not torch.cuda.is_available():
        return []
    dev = torch.device(device if device is not None else "cuda")
    if dev.type != "cuda":
        return []
    a_hw = (None if anchor_hw is None or (int(anchor_hw[0]), int(anchor_hw[1])) == (h, w)
            else (int(anchor_hw[0]), int(anchor_hw[1])))
    hw = int(h) * int(w)
    hw_a = hw if a_hw is None else a_hw[0] * a_hw[1]
    warmed = []
    for f_cur, anchor_mode in variants:
        try:
            if anchor_mode not in (None, "frame", "chunk"):
                raise ValueError(f"anchor_mode must be None, 'frame' or 'chunk', got {anchor_mode!r}")
            f_cur = int(f_cur)
            fkv = int(f_kv) if f_kv is not None else max(f_cur, int(bt))
            spec = _BlockGridSpec(
                f_cur=f_cur, f_kv=fkv, h=h, w=w, block_t=int(bt),
                bh=int(bh), bw=int(bw), rh=int(rh), rw=int(rw),
                hist=(None if block_radius_t is None else (2 * int(block_radius_t) + 1) * int(bt)),
                rt=max(0, fkv // int(bt) - 1), chunk_frames=None,
                streaming=True, anchor_hw=a_hw)
            plan = _bgh.cached_plan(spec, anchor_mode=anchor_mode)
            n_anchor = f_cur * hw_a if anchor_mode is not None else 0
            q = torch.zeros(f_cur * hw, n, d, device=dev, dtype=dtype)
            kv = torch.zeros(n_anchor + fkv * hw, n, d, device=dev, dtype=dtype)
            _bgh.run_blockgrid_hip(q, kv, kv, torch.empty_like(q), plan=plan, f_cur=f_cur, h=h,
                                   w=w, n=n, d=d, anchor_mode=anchor_mode)
            warmed.append((f_cur, anchor_mode))
        except (RuntimeError, ValueError, TypeError) as e:
            warnings.warn(f"prewarm_blockgrid_hip: variant (f_cur={f_cur}, "
                          f"anchor_mode={anchor_mode!r}) skipped: {type(e).__name__}: {e}")
    if warmed:
        torch.cuda.synchronize(dev)
    return warmed