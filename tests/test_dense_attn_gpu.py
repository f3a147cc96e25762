"""Dense attention (srdit_dense_attn_fwd, the cross-attention of the refiner
over its text context) on the GPU through the C ABI.

Against the float64 oracle (oracle/blockgrid.dense_attention with every key
visible) at small ragged shapes and two temperatures; against the window
kernel's dense plan (the path it replaces) at the refiner's full size, where
both walk the keys in the same order with the same arithmetic; the amax word;
graph replays against eager calls.
"""
import numpy as np
import pytest
import torch

from oracle import blockgrid as obg
from parity import check_attention

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _rand(shape, seed, scale, dtype=torch.bfloat16):
    g = torch.Generator("cpu").manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def _dense(q, k, v, amax=None):
    from sr_dit import _lib
    out = torch.full_like(q, float("nan"))
    _lib.dense_attn_fwd(q, k, v, out, q.shape[2] ** -0.5, amax)
    return out


CASES = [
    # Lq, Lkv, heads, head_dim, dtype: ragged query tiles (not multiples of
    # 128), key counts that leave a partial block, an odd number of blocks
    # (one fully masked padding step) and a single key
    (300, 512, 4, 128, torch.bfloat16),
    (129, 77, 3, 128, torch.bfloat16),
    (257, 96, 5, 64, torch.bfloat16),
    (1000, 33, 2, 64, torch.float16),
    (64, 1, 2, 128, torch.bfloat16),
    (5000, 512, 6, 128, torch.float16),
]


@pytest.mark.parametrize("lq,lkv,n,d,dt", CASES, ids=lambda v: str(v))
@pytest.mark.parametrize("temp", [1.0, 8.0])
def test_dense_attention_vs_float64_oracle(lq, lkv, n, d, dt, temp):
    print(f"[case] dense attention lq={lq} lkv={lkv} heads={n} d={d} {dt} temp={temp}",
          flush=True)
    sc = d ** -0.5
    q = _rand((lq, n, d), 1, sc * temp, dt)
    k = _rand((lkv, n, d), 2, sc * temp, dt)
    v = _rand((lkv, n, d), 3, sc, dt)
    amax = torch.full((1,), 12345, dtype=torch.int32, device=DEV)
    out = _dense(q.to(DEV), k.to(DEV), v.to(DEV), amax)
    torch.cuda.synchronize()
    ref = obg.dense_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                              np.ones((lq, lkv), dtype=bool))
    check_attention(out, ref, label=f"dense {lq}x{lkv}")
    assert amax.item() == out.float().abs().max().view(torch.int32).item()


def test_dense_attention_equals_the_window_kernel_at_full_size():
    """21,600 video queries over 512 context tokens, 24 heads x 128: the dense
    kernel against the window kernel's dense plan (CrossAttentionPlan on the
    window path), which walks the same keys in the same 32-key steps with the
    same arithmetic: bit for bit, the amax words too."""
    from sr_dit import model as mdl
    print("[case] dense attention 21600 x 512 x 24 x 128 against the window kernel", flush=True)
    lq, lc, n, d = 21600, 512, 24, 128
    q = _rand((lq, n, d), 5, 1.0).to(DEV)
    k = _rand((lc, n, d), 6, 1.0).to(DEV)
    v = _rand((lc, n, d), 7, 1.0).to(DEV)
    plan = mdl.CrossAttentionPlan(lq, lc)
    a1 = torch.zeros(1, dtype=torch.int32, device=DEV)
    a2 = torch.zeros(1, dtype=torch.int32, device=DEV)
    got = plan.run(q, k, v, torch.empty_like(q), amax_out=a1)
    old = mdl.DENSE_CROSS
    try:
        mdl.DENSE_CROSS = False
        want = plan.run(q, k, v, torch.empty_like(q), amax_out=a2)
    finally:
        mdl.DENSE_CROSS = old
    torch.cuda.synchronize()
    diff = (got.float() - want.float()).abs().max().item()
    print(f"[metrics] max |dense - window| = {diff:.3e}", flush=True)
    assert torch.equal(got, want)
    assert torch.equal(a1, a2)


def test_dense_attention_graph_replays_equal_eager():
    """Captured once, replayed on changing queries with eager work between the
    replays; every replay bit for bit the eager call."""
    from sr_dit import _lib
    lq, lc, n, d = 3000, 512, 8, 128
    q = _rand((lq, n, d), 8, 1.0).to(DEV)
    k = _rand((lc, n, d), 9, 1.0).to(DEV)
    v = _rand((lc, n, d), 10, 1.0).to(DEV)
    out = torch.empty_like(q)
    amax = torch.zeros(1, dtype=torch.int32, device=DEV)
    _lib.dense_attn_fwd(q, k, v, out, d ** -0.5, amax)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _lib.dense_attn_fwd(q, k, v, out, d ** -0.5, amax)
    for it in range(3):
        q.copy_(_rand((lq, n, d), 20 + it, 1.0 + it).to(DEV))
        g.replay()
        want = torch.empty_like(q)
        a2 = torch.zeros(1, dtype=torch.int32, device=DEV)
        _lib.dense_attn_fwd(q, k, v, want, d ** -0.5, a2)
        torch.cuda.synchronize()
        assert torch.equal(out, want), it
        assert torch.equal(amax, a2), it
