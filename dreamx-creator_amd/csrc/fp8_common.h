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

// Eight values -> eight e4m3 bytes (round to nearest even).
static __device__ __forceinline__ uint2 to_e4m3x8(const float f[8], float s) {
  float q[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) q[i] = clamp_fp8(f[i] / s);
  int lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
  lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], lo, true);
  int hi = __builtin_amdgcn_cvt_pk_fp8_f32(q[4], q[5], 0, false);
  hi = __builtin_amdgcn_cvt_pk_fp8_f32(q[6], q[7], hi, true);
  return make_uint2((uint32_t)lo, (uint32_t)hi);
}

}  // namespace q8
}  // namespace srdit
