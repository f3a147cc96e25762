// Device helpers shared by the window-attention kernels (gfx950).
#pragma once

#include "common.h"

#include <utility>

namespace srdit {
namespace win {

// Unrolled loop with a compile-time index (DPP controls must be immediates).
template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

// Eight fp32 values -> one 8-element MFMA operand, converted two at a time
// (v_cvt_pk_*) and assembled as whole 32-bit registers.
template <typename H2, typename V8>
__device__ __forceinline__ V8 pack8_impl(const float* x) {
  i32x4_t w;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const f32x2_t f = {x[2 * j], x[2 * j + 1]};
    w[j] = __builtin_bit_cast(int, __builtin_convertvector(f, H2));
  }
  return __builtin_bit_cast(V8, w);
}

template <typename T> struct Elem;
template <> struct Elem<__bf16> {
  typedef bf16x8_t v8;
  typedef bf16x2_t h2;
  static __device__ __forceinline__ f32x16_t mma(v8 a, v8 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ v8 pack8(const float* x) { return pack8_impl<h2, v8>(x); }
  // a.x*b.x + a.y*b.y + c in fp32 (v_dot2_f32_bf16)
  static __device__ __forceinline__ float dot2(h2 a, h2 b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(a, b, c, false);
  }
};
template <> struct Elem<_Float16> {
  typedef f16x8_t v8;
  typedef f16x2_t h2;
  static __device__ __forceinline__ f32x16_t mma(v8 a, v8 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ v8 pack8(const float* x) { return pack8_impl<h2, v8>(x); }
  // a.x*b.x + a.y*b.y + c in fp32 (v_dot2_f32_f16)
  static __device__ __forceinline__ float dot2(h2 a, h2 b, float c) {
    return __builtin_amdgcn_fdot2(a, b, c, false);
  }
};

// Largest growth (log2 units) of a query's running max tolerated before the
// accumulator is rescaled.  Between rescales P = exp2(s - m_used) <= 2^TAU,
// which the final O = acc / l normalisation cancels exactly; it only bounds
// the range (2^8 fits bf16 and fp16 P with room to spare).
constexpr float TAU = 8.0f;

// n / d for 0 <= n < 2^22, d > 0, rd = 1/d: float estimate plus one correction
// (the estimate is within one of n / d, so qv * d stays below 2^23 and fits the
// 24-bit multiply).
__device__ __forceinline__ int fdiv(int n, int d, float rd) {
  int qv = static_cast<int>(static_cast<float>(n) * rd);
  const int r = n - __mul24(qv, d);
  qv += (r >= d) - (r < 0);
  return qv;
}

__device__ __forceinline__ float other_half_max(float x) {
  i32x2_t s = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
  return fmaxf(__int_as_float(s[0]), __int_as_float(s[1]));
}
__device__ __forceinline__ float half_sum(float x) {
  i32x2_t s = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
  return __int_as_float(s[0]) + __int_as_float(s[1]);
}

// 16 bytes per lane from record `index`, byte `offset` of a structured buffer
// straight into LDS at lds + 16 * lane (buffer_load_dwordx4 ... idxen offen lds).
// A plain device function: the builtin is a device-only one, and a template
// instantiated in the host pass must not name it.
__device__ __forceinline__ void buffer_load_lds_x4(__amdgpu_buffer_rsrc_t rsrc, void* lds, int index,
                                                   int offset) {
  __builtin_amdgcn_struct_ptr_buffer_load_lds(
      rsrc, (__attribute__((address_space(3))) void*)lds, 16, index, offset, 0, 0, 0);
}

// 16 bytes per lane from record `index`, byte `offset` of the structured
// buffer `rsrc` straight into LDS at byte address lds + 16 * lane
// (buffer_load_dwordx4 ... idxen offen lds).  Written as inline asm so the
// compiler does not treat it as an LDS store: it would otherwise wait for
// every outstanding fill before any later LDS read.  Callers fill only LDS
// that no wavefront is reading, and order the fills before the reads of the
// data with explicit waits and a barrier.
__device__ __forceinline__ void dma_x4(i32x4_t rsrc, uint32_t lds, int index, int offset) {
  const i32x2_t va = {index, offset};
  asm volatile("buffer_load_dwordx4 %0, %1, 0 idxen offen lds" ::"v"(va), "s"(rsrc), "{m0}"(lds)
               : "memory");
}

// Compiler-only fence: keeps LDS/DMA accesses on their side of a wait or a
// barrier without emitting any wait of its own.
__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }

// All of this wavefront's memory operations (the DMA fills, the LDS reads)
// retired, then a workgroup barrier: after it every fill issued before it by
// either wavefront is in LDS, and every LDS read issued before it has returned.
__device__ __forceinline__ void fill_barrier() {
  compiler_fence();
  __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0) expcnt(0) lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  compiler_fence();
}

// As fill_barrier, but the last `keep` vector-memory operations this wavefront
// issued may still be in flight (vmcnt(keep)); LDS reads are all retired.
template <int N>
__device__ __forceinline__ void waitcnt_vm_keep() {
  static_assert(N >= 0 && N < 64, "vmcnt out of range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));  // lgkmcnt(0)
}
__device__ __forceinline__ void fill_barrier_keep(int keep) {
  compiler_fence();
  switch (keep) {  // s_waitcnt takes an immediate; keep counts whole load groups
    case 0: waitcnt_vm_keep<0>(); break;
    case 4: waitcnt_vm_keep<4>(); break;
    case 8: waitcnt_vm_keep<8>(); break;
    case 12: waitcnt_vm_keep<12>(); break;
    case 16: waitcnt_vm_keep<16>(); break;
    case 24: waitcnt_vm_keep<24>(); break;
    case 32: waitcnt_vm_keep<32>(); break;
    case 40: waitcnt_vm_keep<40>(); break;
    case 48: waitcnt_vm_keep<48>(); break;
    case 56: waitcnt_vm_keep<56>(); break;
    default: waitcnt_vm_keep<0>(); break;  // any other count: wait for everything
  }
  __builtin_amdgcn_s_barrier();
  compiler_fence();
}

// Per-lane LDS byte offsets, loop-invariant: the K A-operand reads, the V^T
// transposing reads (lane part; the key-block part is a compile-time constant)
// and the 16-byte chunk each fill load of this wavefront reads from its key's
// head row (K swizzle for wavefront 0, V swizzle for wavefront 1).
template <int D>
struct LaneOff {
  static constexpr int KS = D / 16, DT = D / 32, NL = D / 16;
  int k[KS];
  int v[DT];
  int fill[NL];
};

// LDS tiles: 32 keys x D, one row of CPK 16-byte slots per key (chunk L = 8
// head dims), row-major with an XOR swizzle of the slot within its row:
//   slot(key, L) = key*CPK + (L ^ swz(key)).
// Fill load q writes slots [64q, 64q + 64): lane l covers key 64q+l / CPK at
// row position l % CPK, i.e. CPK consecutive lanes read one key's whole
// contiguous head row (chunk (l % CPK) ^ swz(key)), so each load touches
// 64/CPK full rows.  The swizzles (K: (key*CPK/16) % CPK; V: for D=128
// 4(key%4) ^ 8((key>>2)&1), for D=64 key%8) make the K A-operand reads and the
// V transposing reads hit every bank group equally often.
template <int D> __device__ __forceinline__ int swz_k(int key) { return (key * (D / 8) / 16) % (D / 8); }
template <int D> __device__ __forceinline__ int swz_v(int key) {
  return D == 128 ? ((4 * (key & 3)) ^ (8 * ((key >> 2) & 1))) : (key % (D / 8));
}

template <int D>
__device__ __forceinline__ LaneOff<D> make_lane_offsets(int wave) {
  constexpr int CPK = D / 8, LPK = CPK, KPI = 64 / CPK;
  LaneOff<D> o;
  const int lane = threadIdx.x & 63;
  const int c = lane & 31, hf = lane >> 5;
  const int g = lane >> 4, i16 = lane & 15;
#pragma unroll
  for (int ks = 0; ks < LaneOff<D>::KS; ++ks)
    o.k[ks] = (c * CPK + ((hf * LaneOff<D>::KS + ks) ^ swz_k<D>(c))) * 16;
  // V^T read of (kk, dt, h2): key = 16kk + 8h2 + kl with kl = 4hf + i16/4; the
  // swizzle of such a key depends on kl only, so the lane part is
  // (kl*CPK + (Lc ^ swz_v(kl)))*16 + 8*(i16&1) and 16kk + 8h2 adds rows.
  const int kl = 4 * hf + (i16 >> 2);
#pragma unroll
  for (int dt = 0; dt < LaneOff<D>::DT; ++dt) {
    const int Lc = 4 * dt + 2 * (g & 1) + ((i16 & 3) >> 1);
    o.v[dt] = (kl * CPK + (Lc ^ swz_v<D>(kl))) * 16 + 8 * (i16 & 1);
  }
  const int sub = (lane & 15) / LPK, pos = lane % CPK;
#pragma unroll
  for (int q = 0; q < LaneOff<D>::NL; ++q) {
    const int key = q * KPI + (lane >> 4) * (16 / LPK) + sub;
    o.fill[q] = (pos ^ (wave == 0 ? swz_k<D>(key) : swz_v<D>(key))) * 16;
  }
  return o;
}

// One contiguous run of keys with a common decode:
//   token = base + (t0 + j/sp)*frame_len + (r0 + (j%sp)/cols)*Wg + c0 + (j%sp)%cols
// The HR cuboid, the anchor prefix of the plain kernel and an anchor segment of
// the frame kernel are all this formula with their own grid.
// Max |value| of the output, as fp32 bits (non-negative floats order like their
// bits; a NaN sorts above infinity, so it wins as in torch's amax): the
// wavefront's maximum goes to *amax from lane 0 (raise_max_word).
template <typename H2>
__device__ __forceinline__ uint32_t abs_bits2(H2 v) {
  const f32x2_t f = __builtin_convertvector(v, f32x2_t);
  return max(__float_as_uint(f[0]) & 0x7fffffffu, __float_as_uint(f[1]) & 0x7fffffffu);
}

__device__ __forceinline__ void wave_amax_out(uint32_t* amax, uint32_t m) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = max(m, static_cast<uint32_t>(__shfl_xor(static_cast<int>(m), o)));
  if ((threadIdx.x & 63) == 0) raise_max_word(amax, m);
}

// Frame layout of a streaming KV cache kept in place: R ring slots holding the
// nc cached frames (oldest first, cached frame f in slot (head + f) mod R),
// followed by the current chunk's frames (logical frame nc + i at R + i).
// R == 0 is the plain layout, logical frame f at f.
struct KvRing {
  int R, nc, head;  // 0 <= head < R, 0 <= nc <= R
};

__device__ __forceinline__ int ring_frame(const KvRing& r, int f) {
  if (r.R <= 0) return f;
  if (f < r.nc) {
    const int s = r.head + f;  // < 2R
    return s >= r.R ? s - r.R : s;
  }
  return r.R + (f - r.nc);
}

// The ring of a launch: R and nc by value, head from device memory (so one
// captured launch stays valid while the ring advances), clamped into range.
__device__ __forceinline__ KvRing load_ring(int R, int nc, const int32_t* head) {
  KvRing r;
  r.R = R > 0 ? R : 0;
  r.nc = nc < 0 ? 0 : (nc > r.R ? r.R : nc);
  int h = (r.R > 0 && head != nullptr) ? __builtin_amdgcn_readfirstlane(head[0]) : 0;
  r.head = (h < 0 || h >= r.R) ? 0 : h;
  return r;
}

struct KeyRun {
  int n;          // keys in the run
  int base;       // token offset of frame 0 of the run
  int frame_len;  // tokens per frame of the grid the run lives on
  int t0, r0, c0; // first frame / row / column
  int rows, cols; // cuboid rows / columns per frame
  int Wg;         // grid width (row stride in tokens)
  float r_sp, r_cols;
  KvRing ring;    // logical -> physical frame (R == 0: identity)
};

__device__ __forceinline__ KeyRun make_run(int n, int base, int frame_len, int t0, int r0,
                                           int c0, int rows, int cols, int Wg,
                                           KvRing ring = KvRing{0, 0, 0}) {
  KeyRun k;
  k.n = n; k.base = base; k.frame_len = frame_len; k.t0 = t0; k.r0 = r0; k.c0 = c0;
  k.rows = rows; k.cols = cols; k.Wg = Wg;
  k.r_sp = 1.0f / static_cast<float>(rows * cols);
  k.r_cols = 1.0f / static_cast<float>(cols);
  k.ring = ring;
  return k;
}

}  // namespace win
}  // namespace srdit
