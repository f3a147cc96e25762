"""Prewarm contracts on the GPU (attention.py:883-961, fp8_linear.py:191-211):
the variants / shapes warmed are returned, their tables are built and
uploaded, a rejected variant is skipped with a warning, and fp8 buffers keep
their dtypes across module conversions (fp8_linear.py:260-280)."""
import warnings

import pytest
import torch

from sr_dit import attention as att
from sr_dit import blockgrid_hip as bgh
from sr_dit import fp8_linear as fl

pytestmark = pytest.mark.gpu


def test_prewarm_blockgrid_returns_variants_and_uploads_tables():
    bgh.clear_plan_cache()
    geo = dict(h=16, w=24, bt=3, bh=4, bw=4, rh=3, rw=3, n=4, d=128)
    variants = [(3, "frame"), (1, None), (3, None)]
    print("[case] prewarm 3 variants", flush=True)
    got = att.prewarm_blockgrid_hip(variants=variants, **geo)
    assert got == variants
    dev_keys = [k for plan in bgh.HIP_PLAN_CACHE.values() for k in plan
                if isinstance(k, tuple) and k and k[0] == "dev"]
    assert len(bgh.HIP_PLAN_CACHE) == 3 and len(dev_keys) == 3


def test_prewarm_blockgrid_skips_rejected_variant_with_warning():
    geo = dict(h=16, w=24, bt=3, bh=4, bw=4, rh=3, rw=3, n=4, d=128)
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        got = att.prewarm_blockgrid_hip(variants=[(3, "sideways"), (3, "chunk")], **geo)
    assert got == [(3, "chunk")]
    assert any("sideways" in str(x.message) for x in w)


def test_prewarm_blockgrid_native_anchor_grid():
    geo = dict(h=16, w=24, bt=3, bh=4, bw=4, rh=3, rw=3, n=4, d=128)
    assert att.prewarm_blockgrid_hip(variants=[(3, "frame")], anchor_hw=(8, 12), **geo) == [
        (3, "frame")]


def test_prewarm_quantizer_runs_each_shape():
    fl.reset_quantizer_state()
    shapes = fl.quantizer_shapes([640, 384], 256, 1024, [77 * 8])
    print(f"[case] prewarm quantiser {shapes}", flush=True)
    got = fl.prewarm_quantizer(shapes)
    assert got == shapes
    assert set(fl.quantizer_stats()["shapes"]) == set(shapes)
    # a shape the quantiser cannot take (K % 8 != 0) is left out
    assert fl.prewarm_quantizer([(16, 100), (16, 128)]) == [(16, 128)]


def test_fp8_linear_conversions_keep_codes():
    torch.manual_seed(3)
    lin = torch.nn.Linear(256, 128, bias=True).to(torch.bfloat16).cuda()
    m = fl.Fp8Linear.from_linear(lin)
    x = torch.randn(64, 256, dtype=torch.bfloat16, device="cuda")
    y0 = m(x)
    codes = m.weight_fp8.clone()
    for conv in (lambda mod: mod.to(torch.float32), lambda mod: mod.half(),
                 lambda mod: mod.to("cuda", torch.bfloat16), lambda mod: mod.cuda()):
        m = conv(m)
        assert m.weight_fp8.dtype == torch.float8_e4m3fn and torch.equal(m.weight_fp8, codes)
        assert m.weight_scale.dtype == torch.float32
        assert m.bias.dtype == torch.bfloat16
    m = m.to(torch.bfloat16)
    assert torch.equal(m(x), y0)
