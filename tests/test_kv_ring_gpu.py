"""In-place streaming KV cache on the GPU: the window kernels reading a KVRing.

The ring only changes where the kernels fetch each logical KV frame, so every
output must be bit-identical to the same op on the reference's concatenated
cache (``pre_cache_k``/``pre_cache_v`` + ``kv_len``, attention.py:1506-1510,
:964-974) over chunk sequences that wrap the ring.  Covered: the grouped
kernel with two members per workgroup (two-m-tile windows) and with one (the
other plain plans), the single-window kernel (the anchored plans), the
per-frame and whole-chunk LQ anchor, the shipped 4x4/r3 geometry, and a launch
captured in a HIP graph that keeps following the ring as it advances.
"""
import pytest
import torch

from sr_dit import attention as att
from sr_dit import blockgrid_hip as bgh
from sr_dit.kv_ring import KVRing

pytestmark = pytest.mark.gpu

DEV = "cuda"
N, D = 24, 128


def _rand(shape, seed, scale=D ** -0.5):
    g = torch.Generator("cpu").manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16).to(DEV)


def _stream(h, w, f_cur, kv_len, bhw, rhw, chunks, anchor=None, seed=0):
    """Run the op chunk by chunk on the concatenated cache and on a ring; compare."""
    L = h * w
    a_tok = f_cur * L if anchor else 0
    ring = KVRing(1, kv_len, f_cur, L, N, D, anchor_tokens=a_tok, device=DEV)
    ck = torch.zeros(1, 0, N, D, dtype=torch.bfloat16, device=DEV)  # empty cache: streaming
    cv = ck.clone()
    grid = torch.tensor([[f_cur, h, w]])
    kw = dict(block_t=3, block_hw=bhw, block_radius_hw=rhw)
    for c in range(chunks):
        s = seed + 10 * c
        q, k, v = _rand((1, f_cur * L, N, D), s), _rand((1, f_cur * L, N, D), s + 1), \
            _rand((1, f_cur * L, N, D), s + 2, 1.0)
        akw = {}
        if anchor:
            akw = dict(anchor_k=_rand((1, a_tok, N, D), s + 3), anchor_v=_rand((1, a_tok, N, D), s + 4),
                       anchor_align=anchor)
        print(f"[case] ring h={h} w={w} f_cur={f_cur} kv_len={kv_len} chunk={c} "
              f"cached={ring.cached} head={ring.head} anchor={anchor}", flush=True)
        ref, ck, cv = att.mask_free_window_attention(q, k, v, grid, pre_cache_k=ck, pre_cache_v=cv,
                                                     kv_len=kv_len, **kw, **akw)
        out, r1, r2 = att.mask_free_window_attention(q, k, v, grid, kv_ring=ring, kv_commit=True,
                                                     **kw, **akw)
        torch.cuda.synchronize()
        assert r1 is ring and r2 is ring
        assert torch.equal(out, ref), f"chunk {c}: ring output differs from the concatenated cache"
        lk, lv = ring.logical(0)
        assert torch.equal(lk, ck[0]) and torch.equal(lv, cv[0]), f"chunk {c}: cache differs"
    return ring


def test_ring_grouped_kernel_two_frame_chunks():
    """8x8 blocks, 2-frame chunks (two 64-query m-tiles per window: grouped kernel),
    a 5-frame cache wrapped several times."""
    spec = att._BlockGridSpec(f_cur=2, f_kv=7, h=24, w=40, block_t=3, bh=8, bw=8, rh=1, rw=1,
                              rt=1, streaming=True)
    plan = bgh.build_plan(spec)
    assert bgh.groups_supported(plan)
    assert bgh.paired_fraction(bgh.build_groups(plan)) >= 0.75
    ring = _stream(24, 40, 2, 5, (8, 8), (1, 1), chunks=8)
    assert ring.head != 0


def test_ring_solo_kernel_three_frame_chunks():
    """3-frame chunks (three m-tiles that do not all pair: one member per workgroup),
    ragged 45x80-style edges."""
    _stream(21, 36, 3, 4, (8, 8), (1, 1), chunks=7, seed=100)


@pytest.mark.parametrize("anchor", ["frame", "chunk"])
def test_ring_with_lq_anchor(anchor):
    _stream(16, 24, 3, 6, (4, 4), (2, 2), chunks=6, anchor=anchor, seed=200)


def test_ring_production_geometry():
    """The shipped geometry: 45x80, 4x4 blocks, radius 3, 3-frame chunks, 9 cached frames."""
    _stream(45, 80, 3, 9, (4, 4), (3, 3), chunks=5, anchor="frame", seed=300)


@pytest.mark.parametrize("kernel", ["single", "grouped", "solo"])
def test_ring_launcher_both_kernels(kernel):
    """Launcher level: a full ring (head mid-way) against the same frames concatenated."""
    h, w, f_cur, R = 24, 40, 2, 5
    L = h * w
    ring = KVRing(1, R, f_cur, L, N, D, device=DEV)
    for c in range(4):  # fill and wrap: head ends at 3
        ring.write_current(0, _rand((f_cur * L, N, D), 50 + c), _rand((f_cur * L, N, D), 60 + c))
        ring.commit(f_cur)
    assert ring.cached == R and ring.head == 3
    q = _rand((f_cur * L, N, D), 70)
    ring.write_current(0, _rand((f_cur * L, N, D), 71), _rand((f_cur * L, N, D), 72, 1.0))
    lk, lv = ring.logical(0)
    k_cat = torch.cat([lk, ring.current_k(0)]).contiguous()
    v_cat = torch.cat([lv, ring.current_v(0)]).contiguous()
    spec = att._BlockGridSpec(f_cur=f_cur, f_kv=R + f_cur, h=h, w=w, block_t=3, bh=8, bw=8,
                              rh=1, rw=1, rt=(R + f_cur) // 3 - 1, streaming=True)
    plan = bgh.build_plan(spec)
    ref = torch.empty_like(q)
    out = torch.empty_like(q)
    print(f"[case] launcher ring kernel={kernel}", flush=True)
    bgh.run_blockgrid_hip(q, k_cat, v_cat, ref, plan=plan, f_cur=f_cur, h=h, w=w, n=N, d=D,
                          kernel=kernel)
    bgh.run_blockgrid_hip(q, ring.k[0], ring.v[0], out, plan=plan, f_cur=f_cur, h=h, w=w, n=N,
                          d=D, kernel=kernel, ring=ring.kernel_ring(), hr_base=0)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_ring_graph_follows_head():
    """One ring attention call captured in a HIP graph; the ring then advances (head in
    device memory changes) and every replay must equal the eager call on the new state."""
    h, w, f_cur, R = 24, 40, 2, 4
    L = h * w
    ring = KVRing(1, R, f_cur, L, N, D, device=DEV)
    for c in range(2):  # saturate: cached == R, so the plan stays fixed from here on
        ring.write_current(0, _rand((f_cur * L, N, D), 80 + c), _rand((f_cur * L, N, D), 90 + c))
        ring.commit(f_cur)
    grid = torch.tensor([[f_cur, h, w]])
    kw = dict(block_t=3, block_hw=(8, 8), block_radius_hw=(1, 1))
    q = _rand((1, f_cur * L, N, D), 100)
    k = _rand((1, f_cur * L, N, D), 101)
    v = _rand((1, f_cur * L, N, D), 102, 1.0)
    att.mask_free_window_attention(q, k, v, grid, kv_ring=ring, **kw)  # plan + tables built
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g_out, _, _ = att.mask_free_window_attention(q, k, v, grid, kv_ring=ring, **kw)
    for step in range(4):
        # advance: a new chunk into the ring (eager, outside the graph)
        ring.write_current(0, _rand((f_cur * L, N, D), 110 + step),
                           _rand((f_cur * L, N, D), 120 + step))
        ring.commit(f_cur)
        torch.cuda.synchronize()
        print(f"[case] graph replay {step} head={ring.head}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        eager, _, _ = att.mask_free_window_attention(q, k, v, grid, kv_ring=ring, **kw)
        torch.cuda.synchronize()
        assert torch.equal(g_out, eager), f"replay {step} (head {ring.head})"
