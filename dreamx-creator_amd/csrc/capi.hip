// C ABI plumbing of libsrdit_hip: error reporting, version, calibration copy.
#include "common.h"

#include <string.h>

namespace srdit {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

namespace {
__global__ __launch_bounds__(256) void copy16_kernel(const uint4* __restrict__ src,
                                                     uint4* __restrict__ dst, int64_t n) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (; i < n; i += stride) dst[i] = src[i];
}
}  // namespace

}  // namespace srdit

extern "C" int srdit_last_error(char* buf, int len) {
  const int n = static_cast<int>(strlen(srdit::g_last_error));
  if (buf && len > 0) {
    const int m = n < len - 1 ? n : len - 1;
    memcpy(buf, srdit::g_last_error, m);
    buf[m] = '\0';
  }
  return n;
}

extern "C" int srdit_version(void) { return 100; }

extern "C" int srdit_copy_bytes(const void* src, void* dst, int64_t bytes, void* stream) {
  using namespace srdit;
  SRDIT_REQUIRE(src && dst, "srdit_copy_bytes: null pointer");
  SRDIT_REQUIRE(aligned16(src) && aligned16(dst), "srdit_copy_bytes: pointers must be 16-byte aligned");
  SRDIT_REQUIRE(bytes >= 0 && bytes % 16 == 0, "srdit_copy_bytes: bytes must be a non-negative multiple of 16");
  if (bytes == 0) return SRDIT_OK;
  const int64_t n = bytes / 16;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 256 * 32) blocks = 256 * 32;
  hipLaunchKernelGGL(copy16_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), reinterpret_cast<const uint4*>(src),
                     reinterpret_cast<uint4*>(dst), n);
  SRDIT_LAUNCH_CHECK("copy16_kernel");
  return SRDIT_OK;
}
