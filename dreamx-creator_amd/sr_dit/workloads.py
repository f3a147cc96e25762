"""Window-attention workloads: geometries, seeded inputs and useful-FLOP counts.

Geometries (24 heads x 128, 8x8-token query blocks, 3x3 block neighbourhood):
  c1  3x16x16   (768 tokens)    +-1 frame, fp32 CPU plumbing case
  c2  6x34x60   (12,240 tokens) +-1 frame, ragged edge blocks (2-row, 4-col tails),
      Q and K rotated by the 3-D RoPE of their positions
  c3  6x45x80   (21,600 tokens) +-1 frame, ragged 5-row tail blocks
  c4  2 query frames of 45x80 against a 4-frame cache + the 2 current frames,
      the reference's streaming rule (one query run (0, 2, 0, 6))
  prod_* the refiner's shipped geometry: 4x4 blocks, radius 3, 3-frame chunks,
      streaming KV of up to 12 frames, optional LQ anchor

Inputs: ``torch.Generator("cpu").manual_seed(seed)``, fp32 draws in the order
Q, K, V (then K_cache, V_cache for c4), each ~ N(0,1) * 128^-1/2; for c2, Q and
K are then rotated by the 3-D RoPE of their (frame, row, column) positions
(models.py:173-214, theta 10000, 44/42/42 dims, frame offset 0); cast to the
run dtype; generated on the CPU so every consumer sees identical bits.
"""
from __future__ import annotations

import torch

from .attention import _BlockGridSpec
from . import blockgrid_hip as bgh

N_HEADS = 24
HEAD_DIM = 128

# name: (f_cur, f_cache, h, w, bh, bw, rh, rw, rule)
WINDOW_CONFIGS = {
    "c1": dict(f_cur=3, f_cache=0, h=16, w=16, bh=8, bw=8, rh=1, rw=1, rule="sym1"),
    "c2": dict(f_cur=6, f_cache=0, h=34, w=60, bh=8, bw=8, rh=1, rw=1, rule="sym1", rope=True),
    "c3": dict(f_cur=6, f_cache=0, h=45, w=80, bh=8, bw=8, rh=1, rw=1, rule="sym1"),
    "c4": dict(f_cur=2, f_cache=4, h=45, w=80, bh=8, bw=8, rh=1, rw=1, rule="stream"),
    "prod": dict(f_cur=3, f_cache=9, h=45, w=80, bh=4, bw=4, rh=3, rw=3, rule="stream"),
}


def window_spec(name: str, anchor_hw=None, streaming=None) -> _BlockGridSpec:
    c = WINDOW_CONFIGS[name]
    f_kv = c["f_cur"] + c["f_cache"]
    if c["rule"] == "sym1":
        return _BlockGridSpec(f_cur=c["f_cur"], f_kv=f_kv, h=c["h"], w=c["w"], block_t=1,
                              bh=c["bh"], bw=c["bw"], rh=c["rh"], rw=c["rw"],
                              streaming=bool(c["f_cache"]) if streaming is None else streaming,
                              sym_rt=1)
    # streaming rule: block_t = chunk (3), rt derived from the KV length
    # (attention.py:1598-1604)
    bt = 3
    return _BlockGridSpec(f_cur=c["f_cur"], f_kv=f_kv, h=c["h"], w=c["w"], block_t=bt,
                          bh=c["bh"], bw=c["bw"], rh=c["rh"], rw=c["rw"],
                          rt=max(0, f_kv // bt - 1), streaming=True, anchor_hw=anchor_hw)


def make_window_inputs(name: str, dtype=torch.bfloat16, device="cpu", seed=0, temperature=1.0):
    """Seeded ``(q, k, v, k_cache, v_cache)`` as ``[1, S, 24, 128]`` tensors.

    ``k_cache``/``v_cache`` are None without a cache.  ``temperature`` scales Q
    and K (1.0 is the benchmark distribution; larger values give peaky softmax).
    """
    c = WINDOW_CONFIGS[name]
    L = c["h"] * c["w"]
    s_cur, s_cache = c["f_cur"] * L, c["f_cache"] * L
    g = torch.Generator("cpu").manual_seed(seed)
    sc = HEAD_DIM ** -0.5

    def draw(s):
        return torch.randn(1, s, N_HEADS, HEAD_DIM, generator=g, dtype=torch.float32) * sc

    q, k, v = draw(s_cur), draw(s_cur), draw(s_cur)
    kc = vc = None
    if s_cache:
        kc, vc = draw(s_cache), draw(s_cache)
    if c.get("rope"):
        from .model import SRDiTConfig, rope_apply, rope_table
        tab = rope_table(SRDiTConfig(), c["f_cur"], c["h"], c["w"], 0, "cpu")
        q = rope_apply(q[0], tab).unsqueeze(0)
        k = rope_apply(k[0], tab).unsqueeze(0)
    if temperature != 1.0:
        q = q * temperature
        k = k * temperature
        if kc is not None:
            kc = kc * temperature
    cast = lambda t: None if t is None else t.to(dtype=dtype).to(device)
    return cast(q), cast(k), cast(v), cast(kc), cast(vc)


def plan_useful_flops(plan, n_heads=N_HEADS, head_dim=HEAD_DIM) -> int:
    """Sum over windows and heads of 4 * Lq * Lkv * d, read off a params table."""
    return int(bgh._window_cost(plan).sum()) * 4 * head_dim * n_heads


def plan_kv_bytes_streamed(plan, n_heads=N_HEADS, head_dim=HEAD_DIM, elem=2) -> int:
    """K+V bytes a per-window walk reads: sum over windows of Lkv * 2 * d * elem (x m-tiles)."""
    p = plan["params"].to(torch.int64)
    if plan["p_stride"] == bgh.P_FRAME:
        lkv = p[:, 5] * p[:, 7] * p[:, 9] + p[:, 10] * p[:, 12] * p[:, 14]
    else:
        lkv = p[:, 7] * p[:, 9] * p[:, 11] + p[:, 12] * p[:, 14] * p[:, 16]
    return int(lkv.sum()) * 2 * head_dim * elem * n_heads
