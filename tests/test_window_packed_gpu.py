"""Packed window tiles on the GPU through the C ABI (srdit_window_attn_packed_fwd).

4x4-token blocks over three frames make 48-query windows; the packed launch
puts the end of one window and the start of its right neighbour in one 64-row
tile, walks their 32-column KV union and drops each query's outside columns.
Checked against the float64 oracle on small grids of that geometry (bf16,
fp16, head_dim 64), against the fp32 gather restatement at the shipped
45x80 / 12-frame size, against the one-window-per-tile launch on a ring cache
that wraps, for the amax word, and that the launcher's automatic choice is the
packed launch on this geometry.
"""
import pytest
import torch

from sr_dit import attention as att
from sr_dit import blockgrid_hip as bgh
from sr_dit.kv_ring import KVRing
from oracle import blockgrid as obg
from oracle import gather_torch as ogt

from parity import check_attention, metrics

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _spec(f_cur, f_kv, h, w, r=3):
    return att._BlockGridSpec(f_cur=f_cur, f_kv=f_kv, h=h, w=w, block_t=3, bh=4, bw=4, rh=r,
                              rw=r, rt=f_kv // 3 - 1, streaming=True)


def _geom_of(spec):
    return obg.Geometry(**{f: getattr(spec, f) for f in obg.Geometry.__dataclass_fields__})


def _rand(shape, seed, scale, dtype=torch.bfloat16):
    g = torch.Generator("cpu").manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def _launch(spec, q, k, v, kernel, **kw):
    plan = kw.pop("plan", None) or bgh.build_plan(spec)
    out = torch.empty_like(q)
    bgh.run_blockgrid_hip(q, k, v, out, plan=plan, f_cur=spec.f_cur, h=spec.h, w=spec.w,
                          n=q.shape[1], d=q.shape[2], kernel=kernel, **kw)
    torch.cuda.synchronize()
    return out


SMALL = [
    ("3of6_24x40", _spec(3, 6, 24, 40)),
    ("3of3_20x36", _spec(3, 3, 20, 36)),
    ("3of9_17x44_ragged", _spec(3, 9, 17, 44)),
    ("3of12_21x52", _spec(3, 12, 21, 52)),
]


@pytest.mark.parametrize("name,spec", SMALL, ids=[c[0] for c in SMALL])
@pytest.mark.parametrize("temp", [1.0, 8.0])
def test_packed_vs_float64_oracle(name, spec, temp):
    plan = bgh.build_plan(spec)
    tiles = bgh.build_packed(plan)
    assert tiles is not None and int((tiles[:, 3] >= 0).sum()) > 0, "geometry does not pack"
    n, d = 4, 128
    L = spec.h * spec.w
    sc = d ** -0.5
    q = _rand((spec.f_cur * L, n, d), 31, sc * temp)
    k = _rand((spec.f_kv * L, n, d), 32, sc * temp)
    v = _rand((spec.f_kv * L, n, d), 33, 1.0)
    print(f"[case] packed {name} temp={temp} tiles={tiles.shape[0]}", flush=True)
    out = _launch(spec, q.to(DEV), k.to(DEV), v.to(DEV), "packed", plan=plan)
    ref = obg.window_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                               _geom_of(spec))
    check_attention(out, ref, label=f"packed/{name}")


def test_packed_fp16_and_head_dim_64():
    spec = _spec(3, 6, 24, 40)
    L = spec.h * spec.w
    for dtype, d in ((torch.float16, 128), (torch.bfloat16, 64), (torch.float16, 64)):
        print(f"[case] packed {dtype} d={d}", flush=True)
        q = _rand((3 * L, 3, d), 41, d ** -0.5 * 4, dtype)
        k = _rand((6 * L, 3, d), 42, d ** -0.5 * 4, dtype)
        v = _rand((6 * L, 3, d), 43, 1.0, dtype)
        out = _launch(spec, q.to(DEV), k.to(DEV), v.to(DEV), "packed")
        ref = obg.window_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                   _geom_of(spec))
        rel = metrics(out, ref)["rel_l2"]
        assert rel < 4e-3, (dtype, d, rel)


@pytest.mark.parametrize("temp", [1.0, 8.0])
def test_packed_shipped_geometry_vs_fp32_gather(temp):
    """45x80, 4x4 blocks, radius 3, a 3-frame chunk against 12 KV frames, 24 heads x 128."""
    spec = _spec(3, 12, 45, 80)
    L = 45 * 80
    sc = 128 ** -0.5
    q = _rand((3 * L, 24, 128), 21, sc * temp).to(DEV)
    k = _rand((12 * L, 24, 128), 22, sc * temp).to(DEV)
    v = _rand((12 * L, 24, 128), 23, 1.0).to(DEV)
    print(f"[case] packed shipped temp={temp}", flush=True)
    out = _launch(spec, q, k, v, "packed")
    ref = ogt.gather_attend(ogt.GatherPlan(_geom_of(spec), None, device=q.device), q.float(),
                            k.float(), v.float(), win_chunk=48, math_backend=True)
    check_attention(out, ref, label=f"packed_shipped_t{temp}")


def test_auto_is_packed_and_amax_word():
    """The launcher picks the packed launch for the shipped geometry (bit-equal
    outputs), and the amax word is the fp32 bits of max |out|."""
    spec = _spec(3, 12, 45, 80)
    L = 45 * 80
    q = _rand((3 * L, 24, 128), 61, 128 ** -0.5).to(DEV)
    k = _rand((12 * L, 24, 128), 62, 128 ** -0.5).to(DEV)
    v = _rand((12 * L, 24, 128), 63, 1.0).to(DEV)
    plan = bgh.build_plan(spec)
    print("[case] packed auto + amax", flush=True)
    packed = _launch(spec, q, k, v, "packed", plan=plan)
    auto = _launch(spec, q, k, v, "auto", plan=plan)
    assert torch.equal(auto, packed)
    word = torch.full((1,), -1, dtype=torch.int32, device=DEV)  # cleared by the launch
    out = _launch(spec, q, k, v, "packed", plan=plan, amax_out=word)
    assert torch.equal(out, packed)
    assert int(word) == int(out.float().abs().max().view(torch.int32))
    # the one-window-per-tile launch agrees to a rounding of the output
    solo = _launch(spec, q, k, v, "solo", plan=plan)
    assert (solo.float() - packed.float()).abs().max().item() <= 2e-3


def test_packed_ring_matches_concatenated_frames():
    """A full ring with its head mid-way against the same frames concatenated:
    the ring only moves where frames are fetched, so outputs are bit-identical."""
    h, w, f_cur, R, n, d = 24, 40, 3, 6, 8, 128
    L = h * w
    ring = KVRing(1, R, f_cur, L, n, d, device=DEV)
    for c in range(3):  # fill and wrap: head ends at 3
        ring.write_current(0, _rand((f_cur * L, n, d), 50 + c, d ** -0.5).to(DEV),
                           _rand((f_cur * L, n, d), 60 + c, 1.0).to(DEV))
        ring.commit(f_cur)
    assert ring.cached == R and ring.head == 3
    q = _rand((f_cur * L, n, d), 70, d ** -0.5).to(DEV)
    ring.write_current(0, _rand((f_cur * L, n, d), 71, d ** -0.5).to(DEV),
                       _rand((f_cur * L, n, d), 72, 1.0).to(DEV))
    lk, lv = ring.logical(0)
    k_cat = torch.cat([lk, ring.current_k(0)]).contiguous()
    v_cat = torch.cat([lv, ring.current_v(0)]).contiguous()
    spec = _spec(f_cur, R + f_cur, h, w)
    plan = bgh.build_plan(spec)
    print("[case] packed ring", flush=True)
    ref = _launch(spec, q, k_cat, v_cat, "packed", plan=plan)
    out = _launch(spec, q, ring.k[0], ring.v[0], "packed", plan=plan, ring=ring.kernel_ring(),
                  hr_base=0)
    assert torch.equal(out, ref)


def test_packed_raise_paths():
    """Plans that do not pack are refused by name, not launched."""
    spec = att._BlockGridSpec(f_cur=3, f_kv=3, h=16, w=16, block_t=1, bh=8, bw=8, rh=1, rw=1,
                              sym_rt=1)
    q = torch.zeros(3 * 256, 2, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="pack"):
        _launch(spec, q, q, q, "packed")
    anchored = _spec(3, 6, 16, 24, r=2)
    plan = bgh.build_plan(anchored, anchor_mode="frame")
    q = torch.zeros(3 * 384, 2, 128, dtype=torch.bfloat16, device=DEV)
    kv = torch.zeros(9 * 384, 2, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        _launch(anchored, q, kv, kv, "packed", plan=plan, anchor_mode="frame")
