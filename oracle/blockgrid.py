"""Oracle for block-grid window attention (test infrastructure, see oracle/__init__.py).

Restates, on the CPU:
  * the spatial rule  ``_blockgrid_axis_blocks``      attention.py:261-290
  * the temporal rules ``_BlockGridSpec.temporal_runs`` attention.py:457-512
    (+ the symmetric +-r frame rule the benchmark configurations use)
  * the params rows    ``build_plan``                 blockgrid_triton.py:83-150
  * the gather index rows ``_win_lin_indices`` / ``_get_win_meta_blockgrid``
                                                       attention.py:238-255, :515-636
  * the anchor columns ``_anchor_kv_index``            attention.py:690-724
  * the kernel math    (scale, softmax, P rounding)    blockgrid_triton.py:184-278
and adds an independent per-token visibility predicate (block distance) used
as the brute-force check of all of the above.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


# ---------------------------------------------------------------- geometry --

def axis_blocks(size, block, radius):
    """attention.py:272-290: per block (q0, qL, k0, kL) along one axis."""
    nb = (size + block - 1) // block
    res = []
    for b in range(nb):
        lo = max(0, b - radius)                        # attention.py:269
        hi = min(nb - 1, b + radius)
        q0, q1 = b * block, min((b + 1) * block, size)
        k0, k1 = lo * block, min((hi + 1) * block, size)
        res.append((q0, q1 - q0, k0, k1 - k0))
    return res


@dataclass(frozen=True)
class Geometry:
    """The fields of _BlockGridSpec (attention.py:387-401) plus ``sym_rt``."""
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

    @property
    def one_query_run(self):                           # attention.py:444-455
        return self.streaming or self.query_grain != "grid" or self.f_kv != self.f_cur

    @property
    def stride(self):                                  # attention.py:293-328
        if self.anchor_hw is None:
            return 1, 1
        return self.h // self.anchor_hw[0], self.w // self.anchor_hw[1]

    @property
    def anchor_grid(self):
        return (self.h, self.w) if self.anchor_hw is None else tuple(self.anchor_hw)


def temporal_runs(g: Geometry):
    """attention.py:457-512 (plus the symmetric rule)."""
    f_cur, f_kv = g.f_cur, g.f_kv
    if g.sym_rt is not None:
        off = f_kv - f_cur
        return [(t, t + 1, max(0, t + off - g.sym_rt), min(f_kv, t + off + g.sym_rt + 1))
                for t in range(f_cur)]
    if g.hist is not None:
        cf = g.chunk_frames if g.chunk_frames else max(1, f_cur)
        if g.one_query_run or f_cur <= cf:
            return [(0, f_cur, max(0, f_kv - f_cur - g.hist), f_kv)]
        out = []
        c0 = 0
        while c0 < f_cur:
            c1 = min(c0 + cf, f_cur)
            out.append((c0, c1, max(0, c0 - g.hist), min(f_kv, c1)))
            c0 += cf
        return out
    bt, rt = g.block_t, g.rt
    if g.one_query_run:
        return [(0, f_cur, max(0, f_kv - (rt + 1) * bt), f_kv)]
    if f_cur < bt:
        return [(0, f_cur, 0, f_kv)]
    return [(i * bt, (i + 1) * bt, max(0, i - rt) * bt, (i + 1) * bt) for i in range(f_cur // bt)]


def params_rows(g: Geometry, anchor_mode=None):
    """blockgrid_triton.py:83-150: (rows, block_m, m_tiles, hr_base, p_stride)."""
    hb = axis_blocks(g.h, g.bh, g.rh)
    wb = axis_blocks(g.w, g.bw, g.rw)
    s_h, s_w = g.stride
    # attention.py:414-429: anchor extent = HR extent / stride
    hb_a = [(a, b, c // s_h, d // s_h) for (a, b, c, d) in hb]
    wb_a = [(a, b, c // s_w, d // s_w) for (a, b, c, d) in wb]
    a_h, a_w = g.anchor_grid
    runs = temporal_runs(g)
    rows, lqs = [], []
    if anchor_mode == "frame":
        assert len(runs) == 1 and runs[0][:2] == (0, g.f_cur)
        kv0, kv1 = runs[0][2], runs[0][3]
        for i, (qh0, qhL, kh0, khL) in enumerate(hb):
            for j, (qw0, qwL, kw0, kwL) in enumerate(wb):
                rows.append([qh0, qw0, qhL, qwL, kv0, kv1 - kv0, kh0, khL, kw0, kwL, g.f_cur,
                             hb_a[i][2], hb_a[i][3], wb_a[j][2], wb_a[j][3], a_h, a_w])
                lqs.append(g.f_cur * qhL * qwL)
    else:
        af = g.f_cur if anchor_mode == "chunk" else 0
        for (q0, q1, kv0, kv1) in runs:
            for i, (qh0, qhL, kh0, khL) in enumerate(hb):
                for j, (qw0, qwL, kw0, kwL) in enumerate(wb):
                    rows.append([q0, q1 - q0, qh0, qw0, qhL, qwL, kv0, kv1 - kv0, kh0, khL,
                                 kw0, kwL, af, hb_a[i][2], hb_a[i][3], wb_a[j][2], wb_a[j][3],
                                 a_h, a_w])
                    lqs.append((q1 - q0) * qhL * qwL)
    bm = 1
    while bm < max(lqs):
        bm *= 2
    block_m = max(16, min(bm, 64))
    m_tiles = max((x + block_m - 1) // block_m for x in lqs)
    hr_base = g.f_cur * a_h * a_w if anchor_mode is not None else 0
    return rows, block_m, m_tiles, hr_base, (17 if anchor_mode == "frame" else 19)


# ------------------------------------------------------- gather index rows --

def lin_indices(T, h, w, h0, w0, wh, ww, t0=0):
    """attention.py:238-255 for one window: flat (t, row, col) indices, t-major."""
    t = np.arange(t0, t0 + T)[:, None, None]
    r = (h0 + np.arange(wh))[None, :, None]
    c = (w0 + np.arange(ww))[None, None, :]
    return (t * (h * w) + r * w + c).reshape(-1)


def windows(g: Geometry, anchor_mode=None):
    """Per window: (q_idx, kv_idx) into q and into the extended KV [anchor | HR].

    Frame-aligned anchors split each window into one pass per query frame
    (attention.py:782-801), each with its own anchor frame columns.
    """
    hb = axis_blocks(g.h, g.bh, g.rh)
    wb = axis_blocks(g.w, g.bw, g.rw)
    s_h, s_w = g.stride
    a_h, a_w = g.anchor_grid
    L_a = a_h * a_w
    hr_base = g.f_cur * L_a if anchor_mode is not None else 0
    out = []
    runs = temporal_runs(g)
    for (q0, q1, kv0, kv1) in runs:
        for (qh0, qhL, kh0, khL) in hb:
            for (qw0, qwL, kw0, kwL) in wb:
                q_idx = lin_indices(q1 - q0, g.h, g.w, qh0, qw0, qhL, qwL, q0)
                kv_idx = hr_base + lin_indices(kv1 - kv0, g.h, g.w, kh0, kw0, khL, kwL, kv0)
                if anchor_mode is None:
                    out.append((q_idx, kv_idx))
                    continue
                sp = lin_indices(1, a_h, a_w, kh0 // s_h, kw0 // s_w, khL // s_h, kwL // s_w)
                if anchor_mode == "chunk":                   # attention.py:716-719
                    a_idx = (np.arange(g.f_cur)[:, None] * L_a + sp[None, :]).reshape(-1)
                    out.append((q_idx, np.concatenate([a_idx, kv_idx])))
                else:                                       # frame: attention.py:720
                    per = qhL * qwL
                    for f in range(q1 - q0):
                        out.append((q_idx[f * per:(f + 1) * per],
                                    np.concatenate([sp + (q0 + f) * L_a, kv_idx])))
    return out


# --------------------------------------------------- per-token visibility --

def frame_visible(g: Geometry, tq, tk):
    """Is HR KV frame ``tk`` visible from query frame ``tq``: the temporal rules
    stated per frame pair instead of per run."""
    f_cur, f_kv = g.f_cur, g.f_kv
    if g.sym_rt is not None:
        return abs(tk - (tq + f_kv - f_cur)) <= g.sym_rt
    if g.hist is not None:
        cf = g.chunk_frames if g.chunk_frames else max(1, f_cur)
        if g.one_query_run or f_cur <= cf:
            return max(0, f_kv - f_cur - g.hist) <= tk < f_kv
        c0 = (tq // cf) * cf
        return max(0, c0 - g.hist) <= tk < min(f_kv, c0 + cf)
    bt, rt = g.block_t, g.rt
    if g.one_query_run:
        return max(0, f_kv - (rt + 1) * bt) <= tk < f_kv
    if f_cur < bt:
        return True
    i = tq // bt
    return max(0, i - rt) * bt <= tk < (i + 1) * bt


def dense_mask(g: Geometry, anchor_mode=None):
    """Boolean [f_cur*h*w, n_anchor + f_kv*h*w] visibility, token by token.

    Spatial rule by block distance: KV position (y', x') is visible from query
    position (y, x) iff |y'//bh - y//bh| <= rh and |x'//bw - x//bw| <= rw.
    Anchor position (ya, xa) on the coarser grid stands for HR position
    (ya*s_h, xa*s_w).
    """
    h, w = g.h, g.w
    yq = np.arange(h)[:, None].repeat(w, 1).reshape(-1)
    xq = np.arange(w)[None, :].repeat(h, 0).reshape(-1)
    sp_ok = ((np.abs(yq[None, :] // g.bh - yq[:, None] // g.bh) <= g.rh) &
             (np.abs(xq[None, :] // g.bw - xq[:, None] // g.bw) <= g.rw))      # [L, L]
    L = h * w
    n_a = 0
    if anchor_mode is not None:
        a_h, a_w = g.anchor_grid
        s_h, s_w = g.stride
        ya = np.arange(a_h)[:, None].repeat(a_w, 1).reshape(-1) * s_h
        xa = np.arange(a_w)[None, :].repeat(a_h, 0).reshape(-1) * s_w
        asp_ok = ((np.abs(ya[None, :] // g.bh - yq[:, None] // g.bh) <= g.rh) &
                  (np.abs(xa[None, :] // g.bw - xq[:, None] // g.bw) <= g.rw))  # [L, L_a]
        n_a = g.f_cur * a_h * a_w
        L_a = a_h * a_w
    mask = np.zeros((g.f_cur * L, n_a + g.f_kv * L), dtype=bool)
    for tq in range(g.f_cur):
        rows = slice(tq * L, (tq + 1) * L)
        if anchor_mode is not None:
            for ta in range(g.f_cur):
                if anchor_mode == "chunk" or ta == tq:
                    mask[rows, ta * L_a:(ta + 1) * L_a] = asp_ok
        for tk in range(g.f_kv):
            if frame_visible(g, tq, tk):
                mask[rows, n_a + tk * L:n_a + (tk + 1) * L] = sp_ok
    return mask


def rows_mask(rows, g: Geometry, anchor_mode=None, kv_total=None):
    """Visibility implied by a params table (plain or frame rows), token by token."""
    h, w = g.h, g.w
    L = h * w
    a_h, a_w = g.anchor_grid
    L_a = a_h * a_w
    n_a = g.f_cur * L_a if anchor_mode is not None else 0
    if kv_total is None:
        kv_total = n_a + g.f_kv * L
    mask = np.zeros((g.f_cur * L, kv_total), dtype=bool)
    for r in rows:
        if anchor_mode == "frame":
            qh0, qw0, qhL, qwL, kv0, kvL, kh0, khL, kw0, kwL, fc, kh0a, khLa, kw0a, kwLa, ha, wa = r
            qt0, qtL, af = 0, fc, 0
        else:
            qt0, qtL, qh0, qw0, qhL, qwL, kv0, kvL, kh0, khL, kw0, kwL, af, kh0a, khLa, kw0a, kwLa, ha, wa = r
        hr_cols = n_a + lin_indices(kvL, h, w, kh0, kw0, khL, kwL, kv0)
        sp_a = lin_indices(1, ha, wa, kh0a, kw0a, khLa, kwLa)
        for t in range(qtL):
            q_idx = lin_indices(1, h, w, qh0, qw0, qhL, qwL, qt0 + t)
            cols = [hr_cols]
            if anchor_mode == "frame":
                cols.append(sp_a + (qt0 + t) * ha * wa)
            elif af:
                cols.append((np.arange(af)[:, None] * ha * wa + sp_a[None, :]).reshape(-1))
            c = np.concatenate(cols)
            mask[np.ix_(q_idx, c)] = True
    return mask


# --------------------------------------------------------------- attention --

def window_attention(q, k_ext, v_ext, g: Geometry, anchor_mode=None, scale=None,
                     p_dtype=None):
    """Gather restatement in float64: for every window, softmax(q k^T * scale) v.

    q [f_cur*h*w, n, d]; k_ext, v_ext [n_anchor + f_kv*h*w, n, d] (numpy).
    ``p_dtype`` rounds P before P.V the way the kernel does (e.g. a bf16 round
    function); None keeps float64.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k_ext, dtype=np.float64)
    v = np.asarray(v_ext, dtype=np.float64)
    d = q.shape[-1]
    scale = d ** -0.5 if scale is None else scale
    out = np.zeros_like(q)
    seen = np.zeros(q.shape[0], dtype=np.int64)
    for q_idx, kv_idx in windows(g, anchor_mode):
        qs = q[q_idx].transpose(1, 0, 2)            # [n, Lq, d]
        ks = k[kv_idx].transpose(1, 0, 2)           # [n, Lkv, d]
        vs = v[kv_idx].transpose(1, 0, 2)
        s = qs @ ks.transpose(0, 2, 1) * scale
        s -= s.max(-1, keepdims=True)
        p = np.exp(s)
        l = p.sum(-1, keepdims=True)
        if p_dtype is not None:
            p = p_dtype(p)
        out[q_idx] = (p @ vs / l).transpose(1, 0, 2)
        seen[q_idx] += 1
    assert (seen == 1).all(), "query windows must partition the tokens exactly once"
    return out


def dense_attention(q, k_ext, v_ext, mask, scale=None):
    """Brute force: softmax over all KV with a boolean mask, float64."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k_ext, dtype=np.float64)
    v = np.asarray(v_ext, dtype=np.float64)
    d = q.shape[-1]
    scale = d ** -0.5 if scale is None else scale
    s = np.einsum("qnd,knd->nqk", q, k) * scale
    s = np.where(mask[None], s, -np.inf)
    s -= s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return np.einsum("nqk,knd->qnd", p, v)


def useful_flops(g: Geometry, anchor_mode=None, n_heads=24, d=128):
    """Sum over windows and heads of 4 * Lq * Lkv * d (QK^T plus PV)."""
    tot = 0
    for q_idx, kv_idx in windows(g, anchor_mode):
        tot += 4 * len(q_idx) * len(kv_idx) * d
    return tot * n_heads
