"""Parity metrics for floating-point outputs.

The stated window-attention bar is max-abs <= 2e-2 and mean-abs <= 2e-3 against
an fp32 reference.  At the benchmark input distribution (Q/K/V ~ N(0,1)/sqrt(128))
softmax is nearly uniform and outputs are ~2e-3 in magnitude, so an all-zero
output would pass that bar.  Every attention check therefore also bounds the
relative L2 error and the worst per-row relative error, which an all-zero or a
uniform-average output fails (see tests/test_oracle.py negative controls).
"""
from __future__ import annotations

import numpy as np
import torch

MAX_ABS = 2e-2
MEAN_ABS = 2e-3
# bf16 has 8 significant bits; the kernel rounds P and O to bf16 once each,
# which gives a relative L2 error near 1.5e-3 against an fp32 reference.  A
# uniform average of V (softmax ignored) measures ~7.7e-3 at the benchmark
# distribution, so 4e-3 separates the two with a 2x margin on both sides.
REL_L2 = 4e-3
ROW_REL = 2e-2


def _np(x):
    if torch.is_tensor(x):
        return x.detach().float().cpu().numpy().astype(np.float64)
    return np.asarray(x, dtype=np.float64)


def metrics(out, ref):
    o, r = _np(out), _np(ref)
    err = np.abs(o - r)
    rows_o = o.reshape(-1, o.shape[-1])
    rows_r = r.reshape(-1, r.shape[-1])
    row_err = np.linalg.norm(rows_o - rows_r, axis=1) / np.maximum(np.linalg.norm(rows_r, axis=1), 1e-30)
    return {
        "max_abs": float(err.max()),
        "mean_abs": float(err.mean()),
        "rel_l2": float(np.linalg.norm(o - r) / max(np.linalg.norm(r), 1e-30)),
        "row_rel_max": float(row_err.max()),
        "finite": bool(np.isfinite(o).all()),
    }


def check_attention(out, ref, *, rel_l2=REL_L2, row_rel=ROW_REL, label=""):
    m = metrics(out, ref)
    ok = (m["finite"] and m["max_abs"] <= MAX_ABS and m["mean_abs"] <= MEAN_ABS
          and m["rel_l2"] <= rel_l2 and m["row_rel_max"] <= row_rel)
    assert ok, f"{label} parity failed: {m}"
    return m


def passes_attention(out, ref, *, rel_l2=REL_L2, row_rel=ROW_REL):
    m = metrics(out, ref)
    return (m["finite"] and m["max_abs"] <= MAX_ABS and m["mean_abs"] <= MEAN_ABS
            and m["rel_l2"] <= rel_l2 and m["row_rel_max"] <= row_rel)


def passes_abs_bounds_only(out, ref):
    m = metrics(out, ref)
    return m["max_abs"] <= MAX_ABS and m["mean_abs"] <= MEAN_ABS


def rope_table_ref(f, h, w, head_dim=128, theta=10000.0, t_offset=0, device="cpu"):
    """Per-token RoPE phasors [f*h*w, 1, head_dim/2] (complex128) straight from the
    formulas of models.py:80-97 and :173-214: complex pair c of a head is
    exp(i * pos * theta^(-2 c'/dim_axis)) with the pairs split 22/21/21 (for
    head_dim 128) over frame (pos = t_offset + t), row and column, in that order."""
    c = head_dim // 2
    ch = c // 3
    ct = c - 2 * ch
    def axis(n, pairs, off=0):
        pos = torch.arange(n, dtype=torch.float64) + off
        inv = theta ** (-2.0 * torch.arange(pairs, dtype=torch.float64) / (2 * pairs))
        ang = pos[:, None] * inv[None, :]
        return torch.complex(torch.cos(ang), torch.sin(ang))
    ft, fh, fw = axis(f, ct, t_offset), axis(h, ch), axis(w, ch)
    tab = torch.cat([ft.view(f, 1, 1, ct).expand(f, h, w, ct),
                     fh.view(1, h, 1, ch).expand(f, h, w, ch),
                     fw.view(1, 1, w, ch).expand(f, h, w, ch)], dim=-1)
    return tab.reshape(f * h * w, 1, c).to(device)
