"""The shared-fetch window kernel (csrc/window_share.hip) on the GPU, through
the C ABI, against the float64 oracle (small grids) and the fp32 gather
restatement of the reference's CPU path (benchmark configs).

Covers ragged grid edges in both directions (units with fewer valid rows or
columns), workgroups with fewer than four members, two m-tiles per window, a
streaming cache and fp16, at the benchmark distribution and with peaky
(temperature 8) inputs.
"""
import pytest
import torch

from sr_dit import attention as att
from sr_dit import blockgrid_hip as bgh
from sr_dit import workloads as wl
from oracle import blockgrid as obg
from oracle import gather_torch as ogt

from parity import check_attention

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _geom_of(spec):
    return obg.Geometry(**{f: getattr(spec, f) for f in obg.Geometry.__dataclass_fields__})


def _rand(shape, seed, scale, dtype=torch.bfloat16):
    g = torch.Generator("cpu").manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def _sym(f, h, w, bh=8, bw=8, rh=1, rw=1, rt=1):
    return att._BlockGridSpec(f_cur=f, f_kv=f, h=h, w=w, block_t=1, bh=bh, bw=bw, rh=rh, rw=rw,
                              sym_rt=rt)


SMALL = [
    ("sym_3x16x16", _sym(3, 16, 16)),
    ("ragged_3x13x21", _sym(3, 13, 21)),
    ("one_frame_8x40_partial_group", _sym(1, 8, 40)),
    ("radius2_3x24x32", _sym(3, 24, 32, rh=2, rw=2)),
    ("stream_2of4_16x16_m2tiles", att._BlockGridSpec(f_cur=2, f_kv=4, h=16, w=16, block_t=3,
                                                     bh=8, bw=8, rh=1, rw=1, rt=1,
                                                     streaming=True)),
]


def _run(spec, q, k, v, kernel):
    plan = bgh.build_plan(spec)
    out = torch.empty_like(q)
    bgh.run_blockgrid_hip(q, k, v, out, plan=plan, f_cur=spec.f_cur, h=spec.h, w=spec.w,
                          n=q.shape[1], d=q.shape[2], kernel=kernel)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("name,spec", SMALL, ids=[s[0] for s in SMALL])
@pytest.mark.parametrize("temp", [1.0, 8.0])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("kernel", ["shared", "shared2"])
def test_small_vs_float64_oracle(name, spec, temp, dtype, kernel):
    n, d = 3, 128
    L = spec.h * spec.w
    sc = d ** -0.5
    q = _rand((spec.f_cur * L, n, d), 51, sc * temp, dtype)
    k = _rand((spec.f_kv * L, n, d), 52, sc * temp, dtype)
    v = _rand((spec.f_kv * L, n, d), 53, sc, dtype)
    print(f"[case] {kernel} {name} temp={temp} {dtype}", flush=True)
    out = _run(spec, q.to(DEV), k.to(DEV), v.to(DEV), kernel)
    ref = obg.window_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                               _geom_of(spec), None)
    check_attention(out, ref, label=f"shared/{name}")


@pytest.mark.parametrize("cfg", ["c1", "c2", "c3", "c4"])
@pytest.mark.parametrize("temp", [1.0, 8.0])
@pytest.mark.parametrize("kernel", ["shared", "shared2"])
def test_benchmark_configs_vs_fp32_gather(cfg, temp, kernel):
    spec = wl.window_spec(cfg)
    q, k, v, kc, vc = wl.make_window_inputs(cfg, torch.bfloat16, DEV, seed=0, temperature=temp)
    q, k, v = q[0], k[0], v[0]
    if kc is not None:
        k = torch.cat([kc[0], k], 0)
        v = torch.cat([vc[0], v], 0)
    print(f"[case] {kernel} {cfg} temp={temp}", flush=True)
    out = _run(spec, q.contiguous(), k.contiguous(), v.contiguous(), kernel)
    gp = ogt.GatherPlan(_geom_of(spec), None, device=q.device)
    ref = ogt.gather_attend(gp, q.float(), k.float(), v.float(), win_chunk=48)
    m = check_attention(out, ref, label=f"{kernel}/{cfg}")
    print(f"[metrics] {kernel} {cfg} temp={temp} {m}", flush=True)


def test_matches_solo_kernel_and_is_deterministic():
    """c3 on the shared kernel twice (bit-identical) and against the one-member
    grouped kernel (same arithmetic per key, different key order: within
    the bf16 rounding of O)."""
    spec = wl.window_spec("c3")
    q, k, v, _, _ = wl.make_window_inputs("c3", torch.bfloat16, DEV, seed=5, temperature=4.0)
    q, k, v = q[0].contiguous(), k[0].contiguous(), v[0].contiguous()
    a = _run(spec, q, k, v, "shared")
    b = _run(spec, q, k, v, "shared")
    assert torch.equal(a, b)
    s = _run(spec, q, k, v, "solo")
    check_attention(a, s.float(), label="shared vs solo")


def test_ring_cache_equals_concatenation():
    """c4 through the in-place ring layout (cached frames rotated in the ring)
    equals the concatenated cache, bit for bit."""
    spec = wl.window_spec("c4")
    q, k, v, kc, vc = wl.make_window_inputs("c4", torch.bfloat16, DEV, seed=7, temperature=4.0)
    q, k, v, kc, vc = q[0], k[0], v[0], kc[0], vc[0]
    L = spec.h * spec.w
    R, head = 4, 3
    kcat, vcat = torch.cat([kc, k]).contiguous(), torch.cat([vc, v]).contiguous()
    ref = _run(spec, q.contiguous(), kcat, vcat, "shared")
    kr = torch.empty_like(kcat)
    vr = torch.empty_like(vcat)
    for f in range(4):  # cached logical frame f lives in slot (head + f) % R
        s = (head + f) % R
        kr[s * L:(s + 1) * L] = kc[f * L:(f + 1) * L]
        vr[s * L:(s + 1) * L] = vc[f * L:(f + 1) * L]
    kr[R * L:] = k
    vr[R * L:] = v
    plan = bgh.build_plan(spec)
    out = torch.empty_like(q)
    hd = torch.tensor([head], dtype=torch.int32, device=DEV)
    bgh.run_blockgrid_hip(q.contiguous(), kr, vr, out, plan=plan, f_cur=spec.f_cur, h=spec.h,
                          w=spec.w, n=q.shape[1], d=q.shape[2], kernel="shared", ring=(R, 4, hd))
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_amax_out():
    spec = wl.window_spec("c1")
    q, k, v, _, _ = wl.make_window_inputs("c1", torch.bfloat16, DEV, seed=2, temperature=4.0)
    q, k, v = q[0].contiguous(), k[0].contiguous(), v[0].contiguous()
    plan = bgh.build_plan(spec)
    out = torch.empty_like(q)
    word = torch.full((1,), 12345, dtype=torch.int32, device=DEV)
    bgh.run_blockgrid_hip(q, k, v, out, plan=plan, f_cur=3, h=16, w=16, n=24, d=128,
                          kernel="shared", amax_out=word)
    torch.cuda.synchronize()
    got = word.view(torch.float32).item()
    assert got == out.float().abs().max().item()
