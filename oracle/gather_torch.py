"""Torch restatement of the reference's gather backend (test infrastructure).

Follows video_refiner/wan/modules/sr_dit/attention.py:
  * _get_win_meta_blockgrid  :515-636  windows bucketed by (Lq, Lkv)
  * _win_gather_attend       :660-687  index_select gather, one batched SDPA
  * _win_attend              :650-657  F.scaled_dot_product_attention
  * _blockgrid_gather_attend :727-802  index_copy_ scatter, anchor columns
Used as the CPU baseline of bench.py (timed on the host cores) and, in fp32 on
the GPU, as the reference for full-size parity tests.  There the tests pass
``math_backend=True``, which pins SDPA to its math backend (an explicit
softmax(q k^T * scale) v in the input dtype), so no fused or memory-efficient
kernel of the library stands between the reference and the formula; a GPU test
checks sampled windows of that reference against the float64 oracle
(oracle/blockgrid.py).  It is test infrastructure, not the product: nothing
under dreamx-creator_amd/ imports it.
"""
from __future__ import annotations

import numpy as np
import contextlib

import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from . import blockgrid as bg


class GatherPlan:
    """Bucketed window index rows on one device (attention.py:602-636)."""

    def __init__(self, g: bg.Geometry, anchor_mode=None, device="cpu"):
        buckets: dict = {}
        for q_idx, kv_idx in bg.windows(g, anchor_mode):
            key = (len(q_idx), len(kv_idx))
            buckets.setdefault(key, ([], []))
            buckets[key][0].append(q_idx)
            buckets[key][1].append(kv_idx)
        self.groups = []
        for (lq, lkv), (qs, kvs) in buckets.items():
            self.groups.append({
                "q": torch.from_numpy(np.concatenate(qs)).to(device=device, dtype=torch.long),
                "kv": torch.from_numpy(np.concatenate(kvs)).to(device=device, dtype=torch.long),
                "Nw": len(qs), "Lq": lq, "Lkv": lkv})
        self.n_q = g.f_cur * g.h * g.w


def gather_attend(plan: GatherPlan, q, k_ext, v_ext, win_chunk=None, math_backend=False):
    """q [s, n, d], k_ext/v_ext [s_kv, n, d] -> [s, n, d] (same dtype as q).
    ``math_backend``: run SDPA on its math backend only."""
    with sdpa_kernel([SDPBackend.MATH]) if math_backend else contextlib.nullcontext():
        return _gather_attend(plan, q, k_ext, v_ext, win_chunk)


def _gather_attend(plan: GatherPlan, q, k_ext, v_ext, win_chunk):
    n, d = q.shape[1], q.shape[2]
    out = q.new_empty(plan.n_q, n, d)
    for g in plan.groups:
        Nw, Lq, Lkv = g["Nw"], g["Lq"], g["Lkv"]
        chunk = Nw if (win_chunk is None or win_chunk <= 0) else min(int(win_chunk), Nw)
        res = q.new_empty(Nw * Lq, n, d)
        for a in range(0, Nw, chunk):
            b = min(a + chunk, Nw)
            qg = q.index_select(0, g["q"][a * Lq:b * Lq]).view(b - a, Lq, n, d)
            kg = k_ext.index_select(0, g["kv"][a * Lkv:b * Lkv]).view(b - a, Lkv, n, d)
            vg = v_ext.index_select(0, g["kv"][a * Lkv:b * Lkv]).view(b - a, Lkv, n, d)
            o = F.scaled_dot_product_attention(
                qg.transpose(1, 2), kg.transpose(1, 2), vg.transpose(1, 2)).transpose(1, 2)
            res[a * Lq:b * Lq] = o.reshape((b - a) * Lq, n, d)
        out.index_copy_(0, g["q"], res)
    return out
