"""fp8 e4m3 oracle: quantisers and the dequantised GEMM, numpy.  TEST INFRASTRUCTURE ONLY.

Restates video_refiner/wan/modules/sr_dit/fp8_linear.py:93-103
(``_quantize_rowwise_impl``) and the ``torch._scaled_mm`` call of
``Fp8Linear.forward`` (:282-297):

    amax  = max |x| over the row (or the whole tensor), fp32
    scale = max(amax * fl32(1/448), 1e-12)         fp32 multiply
    q     = e4m3(clamp(x / scale, -448, 448))      fp32 division, RNE
    out   = bf16(sum_k qa qb * sa * sb + bias)

``amax / 448.0`` is written as a multiply by the fp32 reciprocal because that
is what it computes where the reference runs (a GPU): torch divides a GPU
tensor by a Python scalar as ``a * (1/b)`` in fp32 (ATen's true-divide GPU
kernel), and inductor lowers a division by a constant to a multiply by its
reciprocal.  ``x / scale`` has a tensor divisor and is a true division.  On the
CPU torch divides exactly, which can differ in the scale's last bit.

The e4m3 encoder is written from the OCP e4m3fn format (bias 7, 3 mantissa
bits, no infinities, max normal 448, subnormals m * 2^-9); it is pinned by
the tests against torch's ``float8_e4m3fn`` cast (the reference's cast) over
every bf16 value and against a brute-force nearest-value search.
"""
from __future__ import annotations

import numpy as np

FP8_MAX = np.float32(448.0)
INV_FP8_MAX = np.float32(1.0) / np.float32(448.0)     # fl32(1/448)
SCALE_FLOOR = np.float32(1e-12)


def e4m3_decode_table() -> np.ndarray:
    """float64 value of each of the 256 e4m3fn codes (NaN for 0x7f / 0xff)."""
    vals = np.empty(256, dtype=np.float64)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        e, m = (code >> 3) & 0xF, code & 7
        if e == 0xF and m == 7:
            vals[code] = np.nan
        elif e == 0:
            vals[code] = sign * m * 2.0 ** -9
        else:
            vals[code] = sign * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return vals


def e4m3_encode(x) -> np.ndarray:
    """float32 array (finite, |x| <= 448) -> uint8 e4m3fn codes, round to nearest even."""
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x).astype(np.float64)
    if np.any(~np.isfinite(a)) or np.any(a > 448.0):
        raise ValueError("e4m3_encode: inputs must be finite with |x| <= 448")
    code = np.zeros(a.shape, dtype=np.int64)
    normal = a >= 2.0 ** -6
    # normals: a = 2^e * (1 + f), 0 <= f < 1; round f*8 half to even
    mant, exp = np.frexp(np.where(normal, a, 1.0))    # a = mant * 2^exp, mant in [0.5, 1)
    e = exp - 1
    frac8 = (mant * 2.0 - 1.0) * 8.0                  # exact in float64
    q = np.round(frac8).astype(np.int64)              # numpy rounds half to even
    carry = q == 8
    e = np.where(carry, e + 1, e)
    q = np.where(carry, 0, q)
    code_n = ((e + 7) << 3) | q
    # subnormals (and zero): a = m * 2^-9, m rounded half to even; m == 8 is 2^-6
    code_s = np.round(a * 2.0 ** 9).astype(np.int64)
    code = np.where(normal, code_n, code_s)
    sign = np.signbit(x).astype(np.int64) << 7
    return (code | sign).astype(np.uint8)


def _to_f32(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32)


def quantize_rowwise(x):
    """x [M, K] (float32 values of the input) -> (codes uint8 [M, K], scale float32 [M])."""
    x = _to_f32(x)
    amax = np.max(np.abs(x), axis=-1)
    scale = np.maximum(amax * INV_FP8_MAX, SCALE_FLOOR).astype(np.float32)
    q = np.clip(x / scale[:, None], -FP8_MAX, FP8_MAX).astype(np.float32)
    return e4m3_encode(q), scale


def quantize_tensor(x):
    """x [M, K] -> (codes uint8 [M, K], scale float32 [1])."""
    x = _to_f32(x)
    amax = np.max(np.abs(x))
    scale = np.float32(max(np.float32(amax * INV_FP8_MAX), SCALE_FLOOR))
    q = np.clip(x / scale, -FP8_MAX, FP8_MAX).astype(np.float32)
    return e4m3_encode(q), np.array([scale], dtype=np.float32)


def gemm_dequant(a_codes, b_codes, sa, sb, bias=None) -> np.ndarray:
    """float64 reference of out[m, n] = sum_k a[m,k] b[n,k] * sa * sb + bias (before bf16)."""
    table = e4m3_decode_table()
    A = table[np.asarray(a_codes)]
    B = table[np.asarray(b_codes)]
    out = A @ B.T
    sa = np.asarray(sa, dtype=np.float64).reshape(-1)
    sb = np.asarray(sb, dtype=np.float64).reshape(-1)
    out = out * (sa[:, None] if sa.size > 1 else sa[0]) * (sb[None, :] if sb.size > 1 else sb[0])
    if bias is not None:
        out = out + np.asarray(bias, dtype=np.float64)[None, :]
    return out
