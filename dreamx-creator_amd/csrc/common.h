// Shared helpers for the libsrdit_hip kernels: status reporting, vector types,
// alignment checks.  gfx950 only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "srdit_hip.h"

namespace srdit {

// Per-thread message of the last failure, read back by srdit_last_error().
void set_error(const char* fmt, ...);

// The persistent MFMA GEMM of fp8.hip on bf16 operands: out [M, N] (row
// stride ldo) = bf16(a [M, K] w [N, K]^T + bias), then bf16(gelu_tanh(.)) when
// gelu; contiguous rows, K % 64 == 0, N % 16 == 0, 16-byte aligned pointers.
int bf16_gemm_persistent(const void* a, const void* w, const void* bias, void* out, int64_t M,
                         int64_t N, int64_t K, int64_t ldo, int gelu, void* stream,
                         const char* who);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

#define SRDIT_REQUIRE(cond, ...)           \
  do {                                     \
    if (!(cond)) {                         \
      ::srdit::set_error(__VA_ARGS__);     \
      return SRDIT_EINVAL;                 \
    }                                      \
  } while (0)

#define SRDIT_HIP_CHECK(expr)                                                        \
  do {                                                                               \
    hipError_t e_ = (expr);                                                          \
    if (e_ != hipSuccess) {                                                          \
      ::srdit::set_error("%s failed: %s", #expr, hipGetErrorString(e_));             \
      return SRDIT_EHIP;                                                             \
    }                                                                                \
  } while (0)

// Launch-error check after <<<>>>: reports configuration errors synchronously.
#define SRDIT_LAUNCH_CHECK(what)                                                     \
  do {                                                                               \
    hipError_t e_ = hipGetLastError();                                               \
    if (e_ != hipSuccess) {                                                          \
      ::srdit::set_error("%s launch failed: %s", what, hipGetErrorString(e_));       \
      return SRDIT_EHIP;                                                             \
    }                                                                                \
  } while (0)

typedef __bf16 bf16x8_t __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef _Float16 f16x8_t __attribute__((__vector_size__(8 * sizeof(_Float16))));
typedef short s16x4_t __attribute__((__vector_size__(4 * sizeof(short))));
typedef float f32x16_t __attribute__((__vector_size__(16 * sizeof(float))));
typedef float f32x4_t __attribute__((__vector_size__(4 * sizeof(float))));
typedef int i32x8_t __attribute__((__vector_size__(8 * sizeof(int))));
typedef int i32x4_t __attribute__((__vector_size__(4 * sizeof(int))));
typedef int i32x2_t __attribute__((__vector_size__(2 * sizeof(int))));

// GELU with the tanh approximation, as torch evaluates it in fp32:
// 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))).
__device__ __forceinline__ float gelu_tanh(float x) {
  const float kBeta = 0.7978845608028654f;  // sqrt(2 / pi)
  const float kKappa = 0.044715f;
  const float x3 = x * x * x;
  const float inner = kBeta * (x + kKappa * x3);
  return 0.5f * x * (1.0f + tanhf(inner));
}

// bf16 round trip (nearest even): the value torch holds after .to(bf16).
__device__ __forceinline__ float bf16_rt(float x) {
  typedef float f32x2v __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
  const uint32_t b = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2v{x, 0.f}, bf16x2v));
  return __uint_as_float(b << 16);
}

// Raise an amax word to at least m (the float bits of a non-negative
// maximum, so unsigned order is float order and a NaN wins): the word is read
// from L2 first and the atomic issued only when m is larger.  The word only
// grows, so a skipped atomic could not have changed it, and most callers end
// without one: thousands of atomics on one word otherwise serialise at its L2
// channel (dense attention over 512 keys with its output amax: 248 -> 176 us).
__device__ __forceinline__ void raise_max_word(uint32_t* word, uint32_t m) {
  const uint32_t cur = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (m > cur) atomicMax(word, m);
}

// XCD-contiguous task index.  Workgroups are dispatched round-robin over the
// 8 XCDs (workgroup b runs on XCD b % 8); this bijection on [0, n) gives each
// XCD one contiguous range of tasks so neighbouring tasks share that XCD's L2.
__device__ __forceinline__ uint32_t xcd_task(uint32_t bid, uint32_t n) {
  const uint32_t x = bid & 7u, slot = bid >> 3;
  return x * (n >> 3) + (x < (n & 7u) ? x : (n & 7u)) + slot;
}

}  // namespace srdit
