"""Window attention on the GPU through the C ABI, against the oracle.

Small grids: the float64 numpy oracle (oracle/blockgrid.py), anchors and every
temporal rule included.  Benchmark sizes (c1-c4 and the shipped 4x4/r3 anchor
geometry): the torch restatement of the reference gather backend in fp32 on the
GPU (oracle/gather_torch.py), at the benchmark input distribution and with
peaky (temperature 8) inputs that make softmax errors visible.  Plus mask
sensitivity, determinism and the raise paths.
"""
import numpy as np
import pytest
import torch

from sr_dit import attention as att
from sr_dit import blockgrid_hip as bgh
from sr_dit import workloads as wl
from oracle import blockgrid as obg
from oracle import gather_torch as ogt

from parity import check_attention, metrics

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _geom_of(spec):
    return obg.Geometry(**{f: getattr(spec, f) for f in obg.Geometry.__dataclass_fields__})


def _rand(shape, seed, scale, dtype=torch.bfloat16):
    g = torch.Generator("cpu").manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def _run_spec(spec, anchor_mode, q, k_ext, v_ext, kernel="auto"):
    plan = bgh.build_plan(spec, anchor_mode=anchor_mode)
    out = torch.empty_like(q)
    n, d = q.shape[1], q.shape[2]
    bgh.run_blockgrid_hip(q, k_ext, v_ext, out, plan=plan, f_cur=spec.f_cur, h=spec.h,
                          w=spec.w, n=n, d=d, anchor_mode=anchor_mode, kernel=kernel)
    torch.cuda.synchronize()
    return out


SMALL = [
    ("sym_3x16x16_8x8", att._BlockGridSpec(f_cur=3, f_kv=3, h=16, w=16, block_t=1, bh=8, bw=8,
                                           rh=1, rw=1, sym_rt=1), None),
    ("sym_ragged_4x13x11", att._BlockGridSpec(f_cur=4, f_kv=4, h=13, w=11, block_t=1, bh=4, bw=4,
                                              rh=1, rw=1, sym_rt=1), None),
    ("sym_r2_3x9x10", att._BlockGridSpec(f_cur=3, f_kv=3, h=9, w=10, block_t=1, bh=4, bw=3, rh=1,
                                         rw=2, sym_rt=2), None),
    ("stream_legacy_2of6_10x12", att._BlockGridSpec(f_cur=2, f_kv=6, h=10, w=12, block_t=3, bh=4,
                                                    bw=4, rh=1, rw=1, rt=1, streaming=True), None),
    ("legacy_parallel_6f_13x11", att._BlockGridSpec(f_cur=6, f_kv=6, h=13, w=11, block_t=3, bh=4,
                                                    bw=4, rh=1, rw=1, rt=1), None),
    ("hist_parallel_6f_12x16", att._BlockGridSpec(f_cur=6, f_kv=6, h=12, w=16, block_t=3, bh=4,
                                                  bw=4, rh=2, rw=2, hist=3, chunk_frames=3), None),
    ("big_window_2f_16x16_m2tiles", att._BlockGridSpec(f_cur=2, f_kv=4, h=16, w=16, block_t=3,
                                                       bh=8, bw=8, rh=1, rw=1, rt=1,
                                                       streaming=True), None),
    ("anchor_frame_2of4_8x12", att._BlockGridSpec(f_cur=2, f_kv=4, h=8, w=12, block_t=2, bh=4, bw=4,
                                                  rh=1, rw=1, rt=1, streaming=True), "frame"),
    ("anchor_chunk_2of4_8x12", att._BlockGridSpec(f_cur=2, f_kv=4, h=8, w=12, block_t=2, bh=4, bw=4,
                                                  rh=1, rw=1, rt=1, streaming=True), "chunk"),
    ("anchor_frame_3f_8x8_blk8_m_tiles3", att._BlockGridSpec(f_cur=3, f_kv=6, h=8, w=8, block_t=3,
                                                             bh=8, bw=8, rh=1, rw=1, rt=1,
                                                             streaming=True), "frame"),
    ("native_anchor_frame_12x16", att._BlockGridSpec(f_cur=2, f_kv=4, h=12, w=16, block_t=2, bh=4,
                                                     bw=4, rh=1, rw=2, rt=1, streaming=True,
                                                     anchor_hw=(6, 8)), "frame"),
    ("native_anchor_chunk_12x16", att._BlockGridSpec(f_cur=2, f_kv=4, h=12, w=16, block_t=2, bh=4,
                                                     bw=4, rh=1, rw=2, rt=1, streaming=True,
                                                     anchor_hw=(6, 8)), "chunk"),
]


@pytest.mark.parametrize("name,spec,mode", SMALL, ids=[s[0] for s in SMALL])
@pytest.mark.parametrize("temp", [1.0, 8.0])
def test_small_vs_float64_oracle(name, spec, mode, temp):
    n, d = 4, 128
    g = _geom_of(spec)
    L = spec.h * spec.w
    a_h, a_w = g.anchor_grid
    n_a = spec.f_cur * a_h * a_w if mode else 0
    sc = d ** -0.5
    q = _rand((spec.f_cur * L, n, d), 11, sc * temp)
    k = _rand((n_a + spec.f_kv * L, n, d), 12, sc * temp)
    v = _rand((n_a + spec.f_kv * L, n, d), 13, sc)
    print(f"[case] {name} temp={temp} tokens={q.shape[0]} kv={k.shape[0]}", flush=True)
    out = _run_spec(spec, mode, q.to(DEV), k.to(DEV), v.to(DEV))
    ref = obg.window_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), g, mode)
    check_attention(out, ref, label=name)


ANCHOR_CASES = [c for c in SMALL if c[2] is not None]


@pytest.mark.parametrize("name,spec,mode", ANCHOR_CASES, ids=[c[0] for c in ANCHOR_CASES])
@pytest.mark.parametrize("kernel", ["single", "solo"])
def test_anchor_plans_both_kernels_vs_float64_oracle(name, spec, mode, kernel):
    """Anchored plans on the single-window kernel and on the one-member grouped
    kernel (anchor frames walked after the HR frames), peaky inputs."""
    n, d = 4, 128
    g = _geom_of(spec)
    L = spec.h * spec.w
    a_h, a_w = g.anchor_grid
    n_a = spec.f_cur * a_h * a_w
    sc = d ** -0.5
    q = _rand((spec.f_cur * L, n, d), 41, sc * 8)
    k = _rand((n_a + spec.f_kv * L, n, d), 42, sc * 8)
    v = _rand((n_a + spec.f_kv * L, n, d), 43, sc)
    print(f"[case] {name} kernel={kernel}", flush=True)
    out = _run_spec(spec, mode, q.to(DEV), k.to(DEV), v.to(DEV), kernel=kernel)
    ref = obg.window_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), g, mode)
    check_attention(out, ref, label=f"{name}/{kernel}")


def _gather_ref(spec, mode, q, k_ext, v_ext):
    plan = ogt.GatherPlan(_geom_of(spec), mode, device=q.device)
    return ogt.gather_attend(plan, q.float(), k_ext.float(), v_ext.float(), win_chunk=48,
                             math_backend=True)


def test_gpu_gather_reference_matches_float64_on_c3_windows():
    """The full-size reference itself: the fp32 gather restatement on the GPU
    (SDPA on its math backend) against the float64 oracle on a sample of c3
    windows (corner, ragged last block row, interior, both edge columns, every
    frame run), all 24 heads, peaky inputs."""
    spec = wl.window_spec("c3")
    geo = _geom_of(spec)
    q, k, v, _, _ = wl.make_window_inputs("c3", torch.bfloat16, DEV, seed=11, temperature=8.0)
    q, k, v = q[0].contiguous(), k[0].contiguous(), v[0].contiguous()
    ref = _gather_ref(spec, None, q, k, v).double().cpu().numpy()
    qn, kn, vn = (t.double().cpu().numpy() for t in (q, k, v))
    wins = obg.windows(geo)
    pick = sorted({0, 9, 50, 59, 60 * 2 + 33, 60 * 3 + 10, 60 * 5 + 59, len(wins) - 1})
    worst = 0.0
    for i in pick:
        q_idx, kv_idx = wins[i]
        qs = qn[q_idx].transpose(1, 0, 2)
        ks = kn[kv_idx].transpose(1, 0, 2)
        vs = vn[kv_idx].transpose(1, 0, 2)
        sc = qs @ ks.transpose(0, 2, 1) * 128 ** -0.5
        p = np.exp(sc - sc.max(-1, keepdims=True))
        o = (p @ vs / p.sum(-1, keepdims=True)).transpose(1, 0, 2)
        err = np.abs(ref[q_idx] - o).max() / max(1e-30, np.abs(o).max())
        worst = max(worst, err)
    print(f"[metrics] gather reference vs float64 on {len(pick)} c3 windows: "
          f"max rel err {worst:.3e}", flush=True)
    # fp32 accumulation over at most 1728 keys
    assert worst < 1e-5, worst


@pytest.mark.parametrize("cfg", ["c1", "c2", "c3", "c4"])
@pytest.mark.parametrize("temp", [1.0, 8.0])
def test_benchmark_configs_vs_fp32_gather(cfg, temp):
    spec = wl.window_spec(cfg)
    q, k, v, kc, vc = wl.make_window_inputs(cfg, torch.bfloat16, DEV, seed=0, temperature=temp)
    q, k, v = q[0], k[0], v[0]
    if kc is not None:
        k = torch.cat([kc[0], k], 0)
        v = torch.cat([vc[0], v], 0)
    print(f"[case] {cfg} temp={temp} q={tuple(q.shape)} kv={tuple(k.shape)}", flush=True)
    out = _run_spec(spec, None, q.contiguous(), k.contiguous(), v.contiguous())
    ref = _gather_ref(spec, None, q, k, v)
    m = check_attention(out, ref, label=cfg)
    print(f"[metrics] {cfg} temp={temp} {m}", flush=True)


@pytest.mark.parametrize("mode", ["frame", "chunk"])
@pytest.mark.parametrize("kernel", ["auto", "single"])
def test_production_anchor_geometry(mode, kernel):
    """Shipped geometry: 4x4 blocks, radius 3, f_cur 3, 12-frame KV, LQ anchor."""
    spec = att._BlockGridSpec(f_cur=3, f_kv=12, h=45, w=80, block_t=3, bh=4, bw=4, rh=3, rw=3,
                              rt=3, streaming=True)
    n, d = 24, 128
    L = 45 * 80
    sc = d ** -0.5
    q = _rand((3 * L, n, d), 21, sc * 4).to(DEV)
    k = _rand((3 * L + 12 * L, n, d), 22, sc * 4).to(DEV)
    v = _rand((3 * L + 12 * L, n, d), 23, sc).to(DEV)
    print(f"[case] prod anchor={mode} kernel={kernel}", flush=True)
    out = _run_spec(spec, mode, q, k, v, kernel=kernel)
    ref = _gather_ref(spec, mode, q, k, v)
    check_attention(out, ref, label=f"prod_{mode}")


def test_op_entry_streaming_cache_and_truncation():
    """mask_free_window_attention with a KV cache: output and returned cache (c4)."""
    q, k, v, kc, vc = wl.make_window_inputs("c4", torch.bfloat16, DEV, seed=3)
    grid = torch.tensor([[2, 45, 80]])
    out, ck, cv = att.mask_free_window_attention(
        q, k, v, grid, pre_cache_k=kc, pre_cache_v=vc, kv_len=3, attn_impl="hip",
        block_t=3, block_hw=(8, 8), block_radius_hw=(1, 1))
    torch.cuda.synchronize()
    full_k = torch.cat([kc[0], k[0]], 0)
    full_v = torch.cat([vc[0], v[0]], 0)
    assert torch.equal(ck[0], full_k[-3 * 3600:]) and torch.equal(cv[0], full_v[-3 * 3600:])
    ref = _gather_ref(wl.window_spec("c4"), None, q[0], full_k, full_v)
    check_attention(out[0], ref, label="c4 op")


def test_op_entry_symmetric_rule_batch2():
    q1, k1, v1, _, _ = wl.make_window_inputs("c1", torch.bfloat16, DEV, seed=4)
    q2, k2, v2, _, _ = wl.make_window_inputs("c1", torch.bfloat16, DEV, seed=5)
    q, k, v = torch.cat([q1, q2]), torch.cat([k1, k2]), torch.cat([v1, v2])
    grid = torch.tensor([[3, 16, 16], [3, 16, 16]])
    out, ck, cv = att.mask_free_window_attention(q, k, v, grid, block_t=1, block_hw=(8, 8),
                                                 block_radius_hw=(1, 1), sym_radius_t=1)
    torch.cuda.synchronize()
    assert out.shape == q.shape and torch.equal(ck, k)
    spec = wl.window_spec("c1")
    for i in range(2):
        check_attention(out[i], _gather_ref(spec, None, q[i], k[i], v[i]), label=f"batch{i}")


def test_mask_sensitivity():
    """Changing K/V outside a query's window leaves its output bit-identical;
    changing one visible token changes it."""
    spec = att._BlockGridSpec(f_cur=3, f_kv=3, h=24, w=24, block_t=1, bh=8, bw=8, rh=1, rw=1,
                              sym_rt=1)
    n, d = 2, 128
    L = 24 * 24
    q = _rand((3 * L, n, d), 31, 0.3).to(DEV)
    k = _rand((3 * L, n, d), 32, 0.3).to(DEV)
    v = _rand((3 * L, n, d), 33, 1.0).to(DEV)
    base = _run_spec(spec, None, q, k, v)
    # query token: frame 0, row 0, col 0 -> sees frames 0-1, rows/cols 0..15
    k2, v2 = k.clone(), v.clone()
    outside = [2 * L + 0, 0 * L + 16 * 24 + 0, 1 * L + 0 * 24 + 16, 0 * L + 23 * 24 + 23]
    for t in outside:
        k2[t] += 5.0
        v2[t] -= 5.0
    o2 = _run_spec(spec, None, q, k2, v2)
    assert torch.equal(o2[0], base[0])
    inside = 1 * L + 15 * 24 + 15
    k3, v3 = k.clone(), v.clone()
    v3[inside] += 1.0
    o3 = _run_spec(spec, None, q, k3, v3)
    assert not torch.equal(o3[0], base[0])


def test_deterministic():
    spec = wl.window_spec("c2")
    q, k, v, _, _ = wl.make_window_inputs("c2", torch.bfloat16, DEV, seed=7)
    a = _run_spec(spec, None, q[0], k[0], v[0])
    b = _run_spec(spec, None, q[0], k[0], v[0])
    assert torch.equal(a, b)


@pytest.mark.parametrize("kernel", ["single", "solo", "grouped"])
def test_fp16_and_head_dim_64(kernel):
    spec = att._BlockGridSpec(f_cur=3, f_kv=3, h=16, w=16, block_t=1, bh=8, bw=8, rh=1, rw=1,
                              sym_rt=1)
    g = _geom_of(spec)
    for dtype, d in ((torch.float16, 128), (torch.bfloat16, 64), (torch.float16, 64)):
        print(f"[case] {kernel} {dtype} d={d}", flush=True)
        q = _rand((3 * 256, 3, d), 41, d ** -0.5 * 4, dtype)
        k = _rand((3 * 256, 3, d), 42, d ** -0.5 * 4, dtype)
        v = _rand((3 * 256, 3, d), 43, 1.0, dtype)
        out = _run_spec(spec, None, q.to(DEV), k.to(DEV), v.to(DEV), kernel=kernel)
        ref = obg.window_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), g)
        rel = metrics(out, ref)["rel_l2"]
        assert rel < 4e-3, (dtype, d, rel)


@pytest.mark.parametrize("mode", ["frame", "chunk"])
@pytest.mark.parametrize("kernel", ["single", "solo"])
def test_anchor_fp16_and_head_dim_64(mode, kernel):
    """The anchored forms in fp16 and at head_dim 64: 4x4 blocks, radius 2, 3 query
    frames against 6 KV frames (streaming rule) with the LQ anchor."""
    spec = att._BlockGridSpec(f_cur=3, f_kv=6, h=16, w=24, block_t=3, bh=4, bw=4, rh=2, rw=2,
                              rt=1, streaming=True)
    g = _geom_of(spec)
    L = 16 * 24
    for dtype, d in ((torch.float16, 128), (torch.bfloat16, 64), (torch.float16, 64)):
        print(f"[case] anchor {mode} {kernel} {dtype} d={d}", flush=True)
        q = _rand((3 * L, 3, d), 51, d ** -0.5 * 4, dtype)
        k = _rand((3 * L + 6 * L, 3, d), 52, d ** -0.5 * 4, dtype)
        v = _rand((3 * L + 6 * L, 3, d), 53, 1.0, dtype)
        out = _run_spec(spec, mode, q.to(DEV), k.to(DEV), v.to(DEV), kernel=kernel)
        ref = obg.window_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), g, mode)
        rel = metrics(out, ref)["rel_l2"]
        assert rel < 4e-3, (mode, kernel, dtype, d, rel)


def test_raise_paths():
    spec_kw = dict(block_t=1, block_hw=(8, 8), block_radius_hw=(1, 1), sym_radius_t=1)
    q = torch.zeros(1, 768, 2, 128, dtype=torch.bfloat16)
    grid = torch.tensor([[3, 16, 16]])
    with pytest.raises(RuntimeError):
        att.mask_free_window_attention(q, q, q, grid, **spec_kw)            # CPU tensors
    with pytest.raises(ValueError):
        att.mask_free_window_attention(q, q, q, grid, attn_impl="triton", **spec_kw)
    qg = q.to(DEV).requires_grad_(True)
    with pytest.raises(RuntimeError):
        att.mask_free_window_attention(qg, qg, qg, grid, **spec_kw)         # autograd
    with pytest.raises(ValueError):
        att.mask_free_window_attention(q.to(DEV).float(), q.to(DEV).float(), q.to(DEV).float(),
                                       grid, **spec_kw)                    # fp32


KERNEL_CASES = [c for c in SMALL if c[2] is None]


@pytest.mark.parametrize("name,spec,mode", KERNEL_CASES, ids=[c[0] for c in KERNEL_CASES])
@pytest.mark.parametrize("kernel", ["single", "grouped", "solo"])
def test_both_kernels_vs_float64_oracle(name, spec, mode, kernel):
    """The single-window kernel and the grouped kernel (two members or one per
    workgroup) each against the oracle, peaky inputs."""
    n, d = 4, 128
    g = _geom_of(spec)
    L = spec.h * spec.w
    sc = d ** -0.5
    q = _rand((spec.f_cur * L, n, d), 31, sc * 8).to(DEV)
    k = _rand((spec.f_kv * L, n, d), 32, sc * 8).to(DEV)
    v = _rand((spec.f_kv * L, n, d), 33, sc).to(DEV)
    print(f"[case] {name} kernel={kernel}", flush=True)
    plan = bgh.build_plan(spec)
    out = torch.empty_like(q)
    bgh.run_blockgrid_hip(q, k, v, out, plan=plan, f_cur=spec.f_cur, h=spec.h, w=spec.w, n=n,
                          d=d, kernel=kernel)
    torch.cuda.synchronize()
    ref = obg.window_attention(q.float().cpu().numpy(), k.float().cpu().numpy(),
                               v.float().cpu().numpy(), g)
    check_attention(out, ref, label=f"{name}/{kernel}")


@pytest.mark.parametrize("cfg,kernel", [("c3", "single"), ("c4", "single"), ("c3", "grouped"),
                                        ("c4", "solo")])
def test_forced_kernels_on_benchmark_configs(cfg, kernel):
    """Each kernel stays correct on the benchmark sizes where "auto" picks another one."""
    spec = wl.window_spec(cfg)
    q, k, v, kc, vc = wl.make_window_inputs(cfg, torch.bfloat16, DEV, seed=1, temperature=8.0)
    q, k, v = q[0].contiguous(), k[0], v[0]
    if kc is not None:
        k, v = torch.cat([kc[0], k], 0), torch.cat([vc[0], v], 0)
    k, v = k.contiguous(), v.contiguous()
    plan = bgh.build_plan(spec)
    out = torch.empty_like(q)
    bgh.run_blockgrid_hip(q, k, v, out, plan=plan, f_cur=spec.f_cur, h=spec.h, w=spec.w,
                          n=wl.N_HEADS, d=wl.HEAD_DIM, kernel=kernel)
    torch.cuda.synchronize()
    check_attention(out, _gather_ref(spec, None, q, k, v), label=f"{cfg}/{kernel}")


def test_grouped_kernel_limits():
    """Two members per workgroup: plain rows only; one member: at most 16 HR frames."""
    spec = att._BlockGridSpec(f_cur=2, f_kv=4, h=8, w=12, block_t=2, bh=4, bw=4, rh=1, rw=1,
                              rt=1, streaming=True)
    plan = bgh.build_plan(spec, anchor_mode="chunk")
    q = torch.zeros(2 * 96, 2, 128, dtype=torch.bfloat16, device=DEV)
    kv = torch.zeros(2 * 96 + 4 * 96, 2, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="grouped"):
        bgh.run_blockgrid_hip(q, kv, kv, torch.empty_like(q), plan=plan, f_cur=2, h=8, w=12,
                              n=2, d=128, anchor_mode="chunk", kernel="grouped")
    long = att._BlockGridSpec(f_cur=3, f_kv=21, h=8, w=12, block_t=3, bh=4, bw=4, rh=1, rw=1,
                              rt=6, streaming=True)
    plan = bgh.build_plan(long)
    assert not bgh.solo_supported(plan)
    q = torch.zeros(3 * 96, 2, 128, dtype=torch.bfloat16, device=DEV)
    kv = torch.zeros(21 * 96, 2, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="16 HR frames"):
        bgh.run_blockgrid_hip(q, kv, kv, torch.empty_like(q), plan=plan, f_cur=3, h=8, w=12,
                              n=2, d=128, kernel="solo")


@pytest.mark.parametrize("cfg,anchor,kernel", [("c3", None, "auto"), ("c2", None, "single"),
                                               ("c4", None, "grouped"), ("prod", "frame", "auto")])
def test_output_amax_word(cfg, anchor, kernel):
    """amax_out receives the fp32 bits of max |out| (the first pass of the output
    projection's per-tensor quantiser), and asking for it leaves out unchanged."""
    if cfg == "prod":
        spec = att._BlockGridSpec(f_cur=3, f_kv=12, h=45, w=80, block_t=3, bh=4, bw=4, rh=3,
                                  rw=3, rt=3, streaming=True)
        L = 45 * 80
        q = _rand((3 * L, 24, 128), 31, 128 ** -0.5).to(DEV)
        k = _rand((15 * L, 24, 128), 32, 128 ** -0.5).to(DEV)
        v = _rand((15 * L, 24, 128), 33, 1.0).to(DEV)
    else:
        spec = wl.window_spec(cfg)
        q, k, v, _, _ = wl.make_window_inputs(cfg, torch.bfloat16, DEV, seed=9)
        q, k, v = q[0].contiguous(), k[0].contiguous(), v[0].contiguous()
    plan = bgh.build_plan(spec, anchor_mode=anchor)
    ref = torch.empty_like(q)
    out = torch.empty_like(q)
    kw = dict(plan=plan, f_cur=spec.f_cur, h=spec.h, w=spec.w, n=24, d=128, anchor_mode=anchor,
              kernel=kernel)
    print(f"[case] amax {cfg} anchor={anchor} kernel={kernel}", flush=True)
    bgh.run_blockgrid_hip(q, k, v, ref, **kw)
    word = torch.full((1,), -1, dtype=torch.int32, device=DEV)  # cleared by the launch
    bgh.run_blockgrid_hip(q, k, v, out, amax_out=word, **kw)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    want = out.float().abs().max().view(torch.int32)
    assert int(word) == int(want)


PAR_CASES = {
    # name: (f_cur, extra op kwargs, expected spec fields as the reference derives them,
    #        attention.py:1583-1604: no cache and no anchor -> not streaming)
    "chunk_causal": (9, dict(causal_chunk_frames=3, causal_kv_span=6),
                     dict(hist=None, rt=1, chunk_frames=3)),          # rt = span // bt - 1
    "radius_t": (9, dict(causal_chunk_frames=3, block_radius_t=1),
                 dict(hist=9, rt=2, chunk_frames=3)),                 # hist = (2 r_t + 1) bt
    "legacy_rt": (9, dict(), dict(hist=None, rt=2, chunk_frames=None)),  # rt = f_kv // bt - 1
}


@pytest.mark.parametrize("case", sorted(PAR_CASES))
def test_op_entry_parallel_forward_rules(case):
    """The op's own derivation of the temporal rule for a forward without a cache:
    the chunk-causal span of the parallel forward (models.py:647-650), the
    chunk-anchored history of block_radius_t, and the legacy rt rule; the output
    matches the oracle on the spec the reference derives."""
    f, h, w, n, d = PAR_CASES[case][0], 16, 24, 4, 128
    L = h * w
    sc = d ** -0.5
    q = _rand((1, f * L, n, d), 61, sc * 4).to(DEV)
    k = _rand((1, f * L, n, d), 62, sc * 4).to(DEV)
    v = _rand((1, f * L, n, d), 63, sc).to(DEV)
    grid = torch.tensor([[f, h, w]])
    print(f"[case] op parallel rule {case}", flush=True)
    out, _, _ = att.mask_free_window_attention(q, k, v, grid, attn_impl="hip", block_t=3,
                                               block_hw=(4, 4), block_radius_hw=(2, 2),
                                               **PAR_CASES[case][1])
    torch.cuda.synchronize()
    spec = att._BlockGridSpec(f_cur=f, f_kv=f, h=h, w=w, block_t=3, bh=4, bw=4, rh=2, rw=2,
                              streaming=False, **PAR_CASES[case][2])
    ref = _gather_ref(spec, None, q[0], k[0], v[0])
    check_attention(out[0], ref, label=f"op {case}")


def test_op_entry_anchor_keep():
    """anchor_keep False drops a sample's anchor (attention.py:1560-1565): the output
    equals the call without an anchor; True keeps it and changes the output."""
    h, w, n, d = 16, 24, 4, 128
    L = h * w
    sc = d ** -0.5
    q = _rand((1, 3 * L, n, d), 71, sc * 4).to(DEV)
    k = _rand((1, 3 * L, n, d), 72, sc * 4).to(DEV)
    v = _rand((1, 3 * L, n, d), 73, sc).to(DEV)
    ak = _rand((1, 3 * L, n, d), 74, sc * 4).to(DEV)
    av = _rand((1, 3 * L, n, d), 75, sc).to(DEV)
    grid = torch.tensor([[3, h, w]])
    kw = dict(attn_impl="hip", block_t=3, block_hw=(4, 4), block_radius_hw=(2, 2))
    print("[case] op anchor_keep", flush=True)
    plain, _, _ = att.mask_free_window_attention(q, k, v, grid, **kw)
    dropped, _, _ = att.mask_free_window_attention(q, k, v, grid, anchor_k=ak, anchor_v=av,
                                                   anchor_keep=[False], **kw)
    kept, _, _ = att.mask_free_window_attention(q, k, v, grid, anchor_k=ak, anchor_v=av,
                                                anchor_keep=[True], **kw)
    torch.cuda.synchronize()
    assert torch.equal(dropped, plain)
    assert not torch.equal(kept, plain)
