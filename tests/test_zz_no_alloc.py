"""srdit_fp8_linear_tensor_static (the per-tensor fp8 Linear that allocates
nothing, its activation amax, scale and codes in the library's static
per-device scratch) against the existing entry points it restates:
srdit_fp8_quant_tensor with caller buffers, then srdit_fp8_gemm_ex on the MFMA
kernel.  Bit-identical outputs, on two calls in a row, the second smaller (the
scratch keeps the first call's contents), and with per-tensor and per-channel
weight scales."""
import pytest
import torch

from sr_dit import _lib

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _case(M, K, N, seed, per_channel, bias):
    g = torch.Generator("cpu").manual_seed(seed)
    x = (torch.randn(M, K, generator=g) * 3).to(torch.bfloat16).to(DEV)
    w = (torch.randn(N, K, generator=g) * 40).clamp(-448, 448).to(torch.float8_e4m3fn).to(DEV)
    ws = (torch.rand(N if per_channel else 1, generator=g) * 0.01 + 1e-3).to(DEV)
    b = (torch.randn(N, generator=g) * 0.1).to(torch.bfloat16).to(DEV) if bias else None
    return x, w, ws, b


def _existing(x, w, ws, b):
    M, K = x.shape
    xq = torch.empty(M, K, dtype=torch.float8_e4m3fn, device=DEV)
    scale = torch.empty(1, dtype=torch.float32, device=DEV)
    amax = torch.zeros(1, dtype=torch.int32, device=DEV)
    _lib.fp8_quant_tensor(x, xq, scale, amax)
    out = torch.empty(M, w.shape[0], dtype=torch.bfloat16, device=DEV)
    _lib.fp8_gemm_ex(xq, w, scale, ws, b, out)
    return out


def _static(x, w, ws, b):
    out = torch.full((x.shape[0], w.shape[0]), float("nan"), dtype=torch.bfloat16, device=DEV)
    _lib.fp8_linear_tensor_static(x, w, ws, b, out)
    return out


def test_static_linear_equals_existing_entry_points_twice():
    cases = [(777, 1024, 512, 1, False, True),    # first call: larger
             (300, 512, 256, 2, True, False)]     # second call: smaller, new amax
    for M, K, N, seed, per_channel, bias in cases:
        print(f"[case] static linear M={M} K={K} N={N} per_channel={per_channel} bias={bias}",
              flush=True)
        x, w, ws, b = _case(M, K, N, seed, per_channel, bias)
        got = _static(x, w, ws, b)
        want = _existing(x, w, ws, b)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got, want), (M, K, N)


def test_static_linear_second_call_does_not_see_the_first():
    """A small-amplitude input after a large one: the amax word is cleared by each
    call, so the scale follows the second input."""
    x1, w, ws, b = _case(256, 512, 256, 3, False, True)
    _static(x1 * 100, w, ws, b)
    x2 = x1 * 0.01
    got = _static(x2, w, ws, b)
    torch.cuda.synchronize()
    assert torch.equal(got, _existing(x2, w, ws, b))


def test_static_linear_rejects_more_than_the_scratch():
    M, K = (_lib.LINEAR_SCRATCH_CODES // 1024) + 1, 1024
    x = torch.empty(M, K, dtype=torch.bfloat16, device=DEV)
    w = torch.empty(128, K, dtype=torch.float8_e4m3fn, device=DEV)
    ws = torch.ones(1, dtype=torch.float32, device=DEV)
    out = torch.empty(M, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="exceeds the static scratch"):
        _lib.fp8_linear_tensor_static(x, w, ws, None, out)
