// fp8 e4m3 quantisers and scaled GEMM for gfx950 (placeholder entry points;
// the kernels land in the next change).
#include "common.h"

extern "C" int srdit_fp8_quant_rowwise(const void*, int64_t, int64_t, int64_t, void*, float*, void*) {
  srdit::set_error("srdit_fp8_quant_rowwise: not implemented yet");
  return SRDIT_EUNSUPPORTED;
}
extern "C" int srdit_fp8_quant_tensor(const void*, int64_t, int64_t, int64_t, void*, float*, float*, void*) {
  srdit::set_error("srdit_fp8_quant_tensor: not implemented yet");
  return SRDIT_EUNSUPPORTED;
}
extern "C" int srdit_fp8_gemm(const void*, const void*, const float*, int64_t, const float*, int64_t,
                              const void*, void*, int64_t, int64_t, int64_t, int64_t, void*) {
  srdit::set_error("srdit_fp8_gemm: not implemented yet");
  return SRDIT_EUNSUPPORTED;
}
