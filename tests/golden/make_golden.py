"""Write golden params tables from the reference's own planner.

Runs ONLY in the build container, where the reference is mounted at
/root/reference; the fixtures it writes (tests/golden/plans.json) are what the
tests read, so nothing reads the reference at test time.

It imports video_refiner/wan/modules/sr_dit/attention.py (for _BlockGridSpec,
attention.py:348-512) and blockgrid_triton.py (for build_plan,
blockgrid_triton.py:83-150) and records, per geometry, the temporal runs and
the full plan (params rows, block_m, m_tiles, block_n, hr_base, p_stride).
The params-row layout, the row order and the temporal rules are definitions,
so these vectors are what pins the planner bit for bit.

The benchmark geometries use a symmetric +-1 frame rule that the reference does
not define; for those the reference build_plan is driven through a duck-typed
spec whose temporal_runs() returns per-frame runs (the seam named at
blockgrid_triton.py:86-88, :153-154).

Usage: python tests/golden/make_golden.py
"""
from __future__ import annotations

import importlib.util
import json
import os
import sys

REF = "/root/reference/video_refiner/wan/modules/sr_dit"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "plans.json")


def _load(name, path):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


class SymSpec:
    """Duck-typed spec: the reference spec's geometry with per-frame +-r runs."""

    def __init__(self, base, r):
        self.base, self.r = base, r

    def __iter__(self):
        return iter(tuple(self.base) + (("sym", self.r),))

    def temporal_runs(self):
        f_cur, f_kv = self.base.f_cur, self.base.f_kv
        off = f_kv - f_cur
        return [(t, t + 1, max(0, t + off - self.r), min(f_kv, t + off + self.r + 1))
                for t in range(f_cur)]

    def __getattr__(self, item):
        return getattr(self.base, item)


def cases(Spec):
    c = []

    def add(name, anchor_mode=None, sym=None, **kw):
        c.append((name, kw, anchor_mode, sym))

    # benchmark geometries: 8x8 blocks, radius 1, +-1 frame
    for name, (f, h, w) in {"c1_3x16x16": (3, 16, 16), "c2_6x34x60": (6, 34, 60),
                            "c3_6x45x80": (6, 45, 80)}.items():
        add(name, sym=1, f_cur=f, f_kv=f, h=h, w=w, block_t=1, bh=8, bw=8, rh=1, rw=1)
    # AR chunk with cache: streaming rule, one query run (0, 2, 0, 6)
    add("c4_ar_2of6x45x80", f_cur=2, f_kv=6, h=45, w=80, block_t=3, bh=8, bw=8, rh=1, rw=1,
        rt=1, streaming=True)
    # production geometry 4x4 / r3, chunk 3, streaming ramp, legacy rule
    for fkv in (3, 6, 9, 12):
        add(f"prod_legacy_fkv{fkv}_45x80", f_cur=3, f_kv=fkv, h=45, w=80, block_t=3, bh=4,
            bw=4, rh=3, rw=3, rt=max(0, fkv // 3 - 1), streaming=True)
    # production with the LQ anchor, both aligns
    for mode in ("chunk", "frame"):
        add(f"prod_anchor_{mode}_fkv12_45x80", anchor_mode=mode, f_cur=3, f_kv=12, h=45, w=80,
            block_t=3, bh=4, bw=4, rh=3, rw=3, rt=3, streaming=True)
    # native (coarser) anchor grid, frame align
    add("prod_native_anchor_frame_44x80", anchor_mode="frame", f_cur=3, f_kv=9, h=44, w=80,
        block_t=3, bh=4, bw=4, rh=3, rw=3, rt=2, streaming=True, anchor_hw=(22, 40))
    add("native_anchor_chunk_12x16", anchor_mode="chunk", f_cur=2, f_kv=4, h=12, w=16,
        block_t=2, bh=4, bw=4, rh=1, rw=2, rt=1, streaming=True, anchor_hw=(6, 8))
    # 1-frame anchor harvest (sub-block query grid)
    add("harvest_1frame_45x80", f_cur=1, f_kv=1, h=45, w=80, block_t=3, bh=4, bw=4, rh=3,
        rw=3, rt=0, streaming=False)
    # chunk-anchored rule (block_radius_t given): parallel partition and streaming
    add("hist_parallel_6f_20x24", f_cur=6, f_kv=6, h=20, w=24, block_t=3, bh=4, bw=4, rh=2,
        rw=2, hist=3, chunk_frames=3, streaming=False)
    add("hist_stream_3of9_20x24", f_cur=3, f_kv=9, h=20, w=24, block_t=3, bh=4, bw=4, rh=2,
        rw=2, hist=9, chunk_frames=3, streaming=True)
    # legacy rule, parallel partition into query blocks
    add("legacy_parallel_6f_13x11", f_cur=6, f_kv=6, h=13, w=11, block_t=3, bh=4, bw=4, rh=1,
        rw=1, rt=1, streaming=False)
    # tiny ragged grids for brute force
    add("tiny_sym_4x13x11", sym=1, f_cur=4, f_kv=4, h=13, w=11, block_t=1, bh=4, bw=4, rh=1, rw=1)
    add("tiny_sym_r2_3x9x10", sym=2, f_cur=3, f_kv=3, h=9, w=10, block_t=1, bh=4, bw=3, rh=1, rw=2)
    add("tiny_anchor_frame_2of4x8x12", anchor_mode="frame", f_cur=2, f_kv=4, h=8, w=12,
        block_t=2, bh=4, bw=4, rh=1, rw=1, rt=1, streaming=True)
    add("tiny_anchor_chunk_2of4x8x12", anchor_mode="chunk", f_cur=2, f_kv=4, h=8, w=12,
        block_t=2, bh=4, bw=4, rh=1, rw=1, rt=1, streaming=True)
    add("tiny_cache_sym_2of4x9x9", sym=1, f_cur=2, f_kv=4, h=9, w=9, block_t=1, bh=4, bw=4,
        rh=1, rw=1, streaming=True)
    return c


def main():
    bgt = _load("_ref_blockgrid_triton", os.path.join(REF, "blockgrid_triton.py"))
    att = _load("_ref_attention", os.path.join(REF, "attention.py"))
    Spec = att._BlockGridSpec
    out = []
    for name, kw, anchor_mode, sym in cases(Spec):
        spec = Spec(**kw)
        if sym is not None:
            spec = SymSpec(spec, sym)
        runs = [list(r) for r in spec.temporal_runs()]
        plan = bgt.build_plan(spec, anchor_mode=anchor_mode)
        out.append({
            "name": name, "spec": kw, "sym_rt": sym, "anchor_mode": anchor_mode,
            "temporal_runs": runs,
            "params": plan["params"].tolist(), "n_w": plan["n_w"],
            "block_m": plan["block_m"], "m_tiles": plan["m_tiles"],
            "block_n": plan["block_n"], "hr_base": plan["hr_base"],
            "p_stride": plan["p_stride"],
        })
    with open(OUT, "w") as f:
        json.dump({"source": "reference build_plan / _BlockGridSpec (blockgrid_triton.py:83-150, "
                             "attention.py:348-512)", "cases": out}, f, separators=(",", ":"))
    print(f"wrote {len(out)} cases to {OUT}", file=sys.stderr)


if __name__ == "__main__":
    main()
