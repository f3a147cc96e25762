// e4m3 quantiser arithmetic shared by the quantisers (fp8.hip) and the fused
// LayerNorm kernels that quantise their own output (fused.hip), so both write
// the same codes for the same values.
#pragma once

#include "common.h"

namespace srdit {
namespace q8 {

inline constexpr float kFp8Max = 448.f;
inline constexpr float kInvFp8Max = 1.0f / 448.0f;   // fl32(1/448), folded at compile time
inline constexpr float kScaleFloor = 1e-12f;

// scale = max(amax * fl32(1/448), 1e-12); a NaN amax stays NaN as torch's clamp_min keeps it.
static __device__ __forceinline__ float scale_from_amax_bits(uint32_t bits) {
  const float s = __uint_as_float(bits) * kInvFp8Max;
  return s < kScaleFloor ? kScaleFloor : s;
}

static __device__ __forceinline__ float clamp_fp8(float q) {
  return q > kFp8Max ? kFp8Max : (q < -kFp8Max ? -kFp8Max : q);
}

// x / s correctly rounded, for one divisor s shared by many quotients: with
// r = RN(1/s) (one IEEE division per thread) and q0 = RN(x * r), within one
// ulp of x / s, the residual x - q0 * s is exact in one FMA and
// RN(q0 + residual * r) is the correctly rounded quotient (Markstein, IBM J.
// Res. Dev. 34(1), 1990; Muller et al., Handbook of Floating-Point Arithmetic,
// section 4.9), barring underflow and overflow.  Here s = max(amax / 448, 1e-12)
// with |x| <= amax, so no quotient overflows, and an underflowing residual
// needs |x| < 2^-100, i.e. |x / s| < 2^-60: far below the e4m3 grid, where
// both quotients encode to a zero of x's sign.  A divisor whose reciprocal is
// not a normal float, or an infinite or NaN one (an inf or NaN in the
// tensor), takes the IEEE division.  A zero residual keeps q0, so -0 / s stays -0.
struct SharedDivisor {
  float s, r;
  bool fast;
  __device__ __forceinline__ explicit SharedDivisor(float s_) : s(s_) {
    r = 1.0f / s_;
    fast = r >= 1.17549435e-38f && r < 3.40282347e38f && s_ < 3.40282347e38f;
  }
  __device__ __forceinline__ float div(float x) const {
    if (!fast) return x / s;
    return div_fast(x);
  }
  // The quotient when `fast` holds (callers that test it once for many values).
  __device__ __forceinline__ float div_fast(float x) const {
    const float q0 = x * r;
    const float e = __builtin_fmaf(-q0, s, x);
    return e == 0.f ? q0 : __builtin_fmaf(e, r, q0);
  }
};

// Eight values -> eight e4m3 bytes of clamp(x / s, +-448) (round to nearest even).
// FAST: the caller has checked d.fast once for all its values.
template <bool FAST = false>
static __device__ __forceinline__ uint2 to_e4m3x8(const float f[8], const SharedDivisor& d) {
  float q[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) q[i] = clamp_fp8(FAST ? d.div_fast(f[i]) : d.div(f[i]));
  int lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
  lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], lo, true);
  int hi = __builtin_amdgcn_cvt_pk_fp8_f32(q[4], q[5], 0, false);
  hi = __builtin_amdgcn_cvt_pk_fp8_f32(q[6], q[7], hi, true);
  return make_uint2((uint32_t)lo, (uint32_t)hi);
}

}  // namespace q8
}  // namespace srdit
