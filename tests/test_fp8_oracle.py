"""The fp8 oracle pinned against torch's float8_e4m3fn cast, brute force and invariants (CPU)."""
import numpy as np
import pytest
import torch

from oracle import fp8 as of


def _torch_cast(x32: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_decode_table_known_codes():
    t = of.e4m3_decode_table()
    assert t[0x00] == 0.0 and t[0x80] == 0.0
    assert t[0x01] == 2.0 ** -9            # smallest subnormal
    assert t[0x07] == 7 * 2.0 ** -9        # largest subnormal
    assert t[0x08] == 2.0 ** -6            # smallest normal
    assert t[0x38] == 1.0
    assert t[0x7E] == 448.0 and t[0xFE] == -448.0
    assert np.isnan(t[0x7F]) and np.isnan(t[0xFF])
    # the decode table agrees with torch's own fp8 -> fp32 conversion
    codes = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    fin = ~np.isnan(t)
    assert np.array_equal(codes[fin], t[fin].astype(np.float32))


def test_encode_every_bf16_value_matches_torch_cast():
    vals = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    v = vals[np.isfinite(vals) & (np.abs(vals) <= 448)]
    assert np.array_equal(of.e4m3_encode(v), _torch_cast(v))


def test_encode_random_fp32_and_ties_match_torch_cast():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(100000) * np.exp(rng.uniform(-16, 6, 100000))).astype(np.float32)
    x = np.clip(x, -448, 448)
    # exact midpoints between neighbouring codes (ties go to the even mantissa)
    t = of.e4m3_decode_table()
    pos = np.sort(t[:0x7F])
    mids = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)
    x = np.concatenate([x, mids, -mids, np.float32([0.0, -0.0, 448.0, -448.0])])
    assert np.array_equal(of.e4m3_encode(x), _torch_cast(x))


def test_encode_is_nearest_value_brute_force():
    """Every code is the nearest representable value; ties pick the even code."""
    t = of.e4m3_decode_table()
    cand = np.arange(0x7F)                    # non-negative finite codes
    rng = np.random.default_rng(2)
    x = np.abs(rng.standard_normal(4000) * np.exp(rng.uniform(-12, 6, 4000))).astype(np.float32)
    x = np.minimum(x, 448)
    got = of.e4m3_encode(x)
    for xi, gi in zip(x.astype(np.float64), got):
        d = np.abs(t[cand] - xi)
        best = cand[d == d.min()]
        want = best[0] if len(best) == 1 else best[(best & 1) == 0][0]
        assert gi == want, (xi, gi, best)


def test_encode_rejects_out_of_range():
    with pytest.raises(ValueError):
        of.e4m3_encode(np.float32([449.0]))
    with pytest.raises(ValueError):
        of.e4m3_encode(np.float32([np.nan]))


def test_quantize_rowwise_invariants():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((33, 256)) * np.exp(rng.uniform(-8, 8, (33, 1)))).astype(np.float32)
    x[5] = 0.0                                          # all-zero row -> floor scale
    q, s = of.quantize_rowwise(x)
    t = of.e4m3_decode_table()
    deq = t[q]
    assert s.dtype == np.float32 and s.shape == (33,)
    assert s[5] == np.float32(1e-12) and np.all(deq[5] == 0)
    for r in range(33):
        if r == 5:
            continue
        # the row's largest |x| maps onto the largest code
        assert np.max(np.abs(deq[r])) == 448.0
        assert s[r] == np.float32(np.max(np.abs(x[r])) * (np.float32(1) / np.float32(448)))
        # dequantisation error is within half an e4m3 step (relative 2^-4 for normals,
        # absolute 2^-10 * scale in the subnormal range)
        err = np.abs(deq[r] * s[r] - x[r])
        bound = np.maximum(np.abs(x[r]) * 2.0 ** -4, 2.0 ** -10 * s[r]) * (1 + 1e-6)
        assert np.all(err <= bound)


def test_quantize_tensor_single_scale():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((17, 64)).astype(np.float32)
    x[3, 7] = 1000.0
    q, s = of.quantize_tensor(x)
    assert s.shape == (1,) and s[0] == np.float32(1000.0) * (np.float32(1) / np.float32(448))
    assert of.e4m3_decode_table()[q[3, 7]] == 448.0


def test_gemm_dequant_matches_explicit_sum():
    rng = np.random.default_rng(5)
    a = rng.integers(0, 0x7F, (3, 8)).astype(np.uint8) | (rng.integers(0, 2, (3, 8)) << 7).astype(np.uint8)
    b = rng.integers(0, 0x7F, (4, 8)).astype(np.uint8)
    sa = np.float32([0.5, 2.0, 0.25])
    sb = np.float32([1.0, 3.0, 0.5, 4.0])
    bias = np.float32([0.1, -0.2, 0.3, 0.0])
    t = of.e4m3_decode_table()
    got = of.gemm_dequant(a, b, sa, sb, bias)
    for m in range(3):
        for n in range(4):
            ref = sum(t[a[m, k]] * t[b[n, k]] for k in range(8)) * sa[m] * sb[n] + bias[n]
            assert abs(got[m, n] - ref) <= 1e-12 * max(1.0, abs(ref))
    # per-tensor scales broadcast
    got1 = of.gemm_dequant(a, b, sa[:1], sb[:1])
    assert np.allclose(got1, (t[a] @ t[b].T) * sa[0] * sb[0])


def test_scale_is_reciprocal_multiply_as_on_the_gpu():
    """amax / 448.0 on a GPU tensor is amax * fl32(1/448): find amax values where that
    differs from the exact quotient, and check the oracle takes the multiply."""
    rng = np.random.default_rng(6)
    amax = rng.uniform(1e-3, 1e3, 20000).astype(np.float32)
    mul = amax * (np.float32(1) / np.float32(448))
    div = amax / np.float32(448)
    differ = amax[mul != div]
    assert differ.size > 0
    x = np.zeros((differ.size, 8), dtype=np.float32)
    x[:, 0] = differ
    _, s = of.quantize_rowwise(x)
    assert np.array_equal(s, differ * (np.float32(1) / np.float32(448)))
