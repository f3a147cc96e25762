// Dense Linears at the two ends of the refiner forward, for gfx950.
//
//   bf16_linear   out = bf16(A W^T + b) [then bf16(gelu_tanh(out))]: the patch
//                 embedding (the Conv3d with kernel = stride = patch, as a
//                 GEMM, models.py:1551-1552) and the text embedding's two
//                 Linears and their tanh GELU (models.py:1860-1866)
//   linear_f32_modulated
//                 out = xin W^T + b in fp32, xin = f32(A) * s1 + m0: the head's
//                 modulation of its bf16 LayerNorm output and its fp32 Linear
//                 (models.py:1372-1384)
//   gemv_f32      out = x W^T + b in fp32: the time embedding and projection
//                 MLPs (models.py:1845-1849), whose input is one row
//
// Every product is exact and every accumulator is fp32, as torch's GEMMs on
// these dtypes; only the summation order differs.  Epilogues round where
// torch's separate ops round: the bias is added to the fp32 accumulator, the
// result rounds once to the output dtype, and the GELU acts on the rounded
// bf16 value and rounds again.
//
// The MFMA operands are read straight from global memory (L2), without LDS
// staging: these GEMMs are either bound by their output stores (patch
// embedding: K = 64) or are small (text embedding: 512 rows; head: 64 output
// columns), and one wave's 32-row operand slice is re-read by at most two
// waves of its workgroup.  Lanes 0-31 of an MFMA operand hold rows 0-31 of
// k-slice [k0, k0+8), lanes 32-63 the same rows at [k0+8, k0+16): a k index is
// paired the same way in A and W, so the sum over k is the GEMM's.
#include "common.h"

namespace srdit {
namespace {

typedef float f32x8v __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float x) {
  typedef float f32x2v __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
  return (uint16_t)__builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2v{x, 0.f}, bf16x2v));
}

template <typename T>
__device__ __forceinline__ f32x8v load8_f32(const T* p);

template <>
__device__ __forceinline__ f32x8v load8_f32<float>(const float* p) {
  const f32x4_t lo = *reinterpret_cast<const f32x4_t*>(p);
  const f32x4_t hi = *reinterpret_cast<const f32x4_t*>(p + 4);
  return f32x8v{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

__device__ __forceinline__ f32x8v unpack_bf16x8(const uint4 v) {
  const uint32_t u[4] = {v.x, v.y, v.z, v.w};
  f32x8v f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(u[i] << 16);
    f[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
  }
  return f;
}

template <>
__device__ __forceinline__ f32x8v load8_f32<uint16_t>(const uint16_t* p) {
  return unpack_bf16x8(*reinterpret_cast<const uint4*>(p));
}

template <typename WT>
__device__ __forceinline__ float load1_f32(const WT* p, int i);
template <>
__device__ __forceinline__ float load1_f32<float>(const float* p, int i) { return p[i]; }
template <>
__device__ __forceinline__ float load1_f32<uint16_t>(const uint16_t* p, int i) {
  return bf16_bits_to_f32(p[i]);
}

// ---------------------------------------------------------------------------
// Tiling shared by the two GEMMs.  A wave owns a 32-row x 64-column output
// tile as two 32x32 MFMA accumulators (columns 0-31 and 32-63).  The MFMAs take
// W as their first operand and the activations as their second, so register v
// of lane l holds row l%32, column 32 t + 8 (v/4) + 4 (l/32) + v%4: four
// consecutive columns per register group.  A workgroup is 4 waves: with KS = 1
// they stack along rows (a 128 x 64 tile); with KS = 4 they share one 32 x 64
// tile and each sums a quarter of the k-steps (for grids too small to fill the
// chip, e.g. 512-row GEMMs).  The epilogue goes through LDS: each wave writes
// its accumulators as an fp32 tile, and the rows are read back 8 columns per
// lane (the KS partials summed in wave order, so results do not depend on
// timing) and stored as 16-byte pieces.
constexpr int WT_M = 32, WT_N = 64;
constexpr int EPI_LD = WT_N + 4;   // fp32 row stride of an LDS tile: rows start 4 banks apart
constexpr int EPI_TILE = WT_M * EPI_LD;
constexpr int RING = 4;            // k-steps of operands in flight per wave

__device__ __forceinline__ void acc_to_lds(float* tile, const f32x16_t& c0, const f32x16_t& c1,
                                           int lane) {
  float* row = tile + (lane & 31) * EPI_LD + 4 * (lane >> 5);
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    *reinterpret_cast<f32x4_t*>(row + 8 * g) = f32x4_t{c0[4 * g], c0[4 * g + 1], c0[4 * g + 2], c0[4 * g + 3]};
    *reinterpret_cast<f32x4_t*>(row + 32 + 8 * g) =
        f32x4_t{c1[4 * g], c1[4 * g + 1], c1[4 * g + 2], c1[4 * g + 3]};
  }
}

template <typename OT>
__device__ __forceinline__ void store8(OT* p, const float v[8]);

template <>
__device__ __forceinline__ void store8<uint16_t>(uint16_t* p, const float v[8]) {
  uint32_t u[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    u[i] = (uint32_t)f32_to_bf16_bits(v[2 * i]) | ((uint32_t)f32_to_bf16_bits(v[2 * i + 1]) << 16);
  *reinterpret_cast<uint4*>(p) = make_uint4(u[0], u[1], u[2], u[3]);
}

template <>
__device__ __forceinline__ void store8<float>(float* p, const float v[8]) {
  *reinterpret_cast<f32x4_t*>(p) = f32x4_t{v[0], v[1], v[2], v[3]};
  *reinterpret_cast<f32x4_t*>(p + 4) = f32x4_t{v[4], v[5], v[6], v[7]};
}

// The first nv (< 8, or rows not 16-byte aligned) values one at a time.
__device__ __forceinline__ void store1(uint16_t* p, float v) { *p = f32_to_bf16_bits(v); }
__device__ __forceinline__ void store1(float* p, float v) { *p = v; }

// After the LDS tiles are written and a barrier: wave w stores its own tile's
// 32 rows (KS = 1) or rows 8w..8w+7 of the shared tile (KS = 4).  Lane l takes
// row l/8 of each 8-row group, columns 8 (l%8) .. +8, as one 16-byte store
// where the piece is whole and the rows are 16-byte aligned (vec_out), else
// value by value (the last piece of a row whose length is not a multiple of 8).
template <int KS, int GELU, typename OT, typename BT>
__device__ __forceinline__ void epilogue(const float* lds, int wave, int lane, int m_tile, int n0,
                                         int M, int N, const BT* __restrict__ bias,
                                         OT* __restrict__ out, int64_t ldo, bool vec_out) {
  const int c = lane & 7, rr = lane >> 3;
  const int n = n0 + 8 * c;
  if (n >= N) return;
  const int nv = N - n < 8 ? N - n : 8;  // columns of this piece inside the matrix
  f32x8v b = {};
  if (bias) {
    if (nv == 8 && (reinterpret_cast<uintptr_t>(bias) & 15) == 0) {  // uniform
      b = load8_f32<BT>(bias + n);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) b[i] = i < nv ? load1_f32<BT>(bias, n + i) : 0.f;
    }
  }
#pragma unroll
  for (int q = 0; q < (KS == 1 ? 4 : 1); ++q) {
    const int r = KS == 1 ? 8 * q + rr : 8 * wave + rr;
    const int m = m_tile + r;
    if (m >= M) break;   // rows only grow with q
    const float* src = lds + (KS == 1 ? wave : 0) * EPI_TILE + r * EPI_LD + 8 * c;
    f32x4_t lo = *reinterpret_cast<const f32x4_t*>(src);
    f32x4_t hi = *reinterpret_cast<const f32x4_t*>(src + 4);
#pragma unroll
    for (int p = 1; p < KS; ++p) {
      lo += *reinterpret_cast<const f32x4_t*>(src + p * EPI_TILE);
      hi += *reinterpret_cast<const f32x4_t*>(src + p * EPI_TILE + 4);
    }
    float v[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v[i] += b[i];
      if (GELU) v[i] = gelu_tanh(bf16_rt(v[i]));
    }
    OT* dst = out + (int64_t)m * ldo + n;
    if (vec_out && nv == 8) {
      store8<OT>(dst, v);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (i < nv) store1(dst + i, v[i]);
    }
  }
}

// ---------------------------------------------------------------------------
// bf16 x bf16 -> fp32 accumulators -> bf16 (32x32x16 bf16 MFMAs).
template <int GELU, int KS>
__global__ __launch_bounds__(256) void bf16_linear_kernel(
    const uint16_t* __restrict__ a, int64_t lda, const uint16_t* __restrict__ w, int64_t ldw,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ out, int64_t ldo, int M, int N,
    int K, bool vec_out) {
  __shared__ __attribute__((aligned(16))) float lds[4 * EPI_TILE];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m_tile = blockIdx.y * (KS == 1 ? 4 * WT_M : WT_M) + (KS == 1 ? WT_M * wave : 0);
  const int n0 = blockIdx.x * WT_N;
  const int r = lane & 31, kh = (lane >> 5) * 8;
  // rows past the end read the last row (in bounds); their results are not stored
  const bf16x8_t* pa = reinterpret_cast<const bf16x8_t*>(a + (int64_t)min(m_tile + r, M - 1) * lda + kh);
  const bf16x8_t* pw0 = reinterpret_cast<const bf16x8_t*>(w + (int64_t)min(n0 + r, N - 1) * ldw + kh);
  const bf16x8_t* pw1 =
      reinterpret_cast<const bf16x8_t*>(w + (int64_t)min(n0 + 32 + r, N - 1) * ldw + kh);
  const int steps = K / 16;
  const int s_begin = KS == 1 ? 0 : wave * (steps / KS);
  const int s_end = KS == 1 ? steps : s_begin + steps / KS;
  const int groups = (s_end - s_begin) / RING;
  f32x16_t c0 = {}, c1 = {};
  bf16x8_t ra[RING], rw0[RING], rw1[RING];
  if (groups > 0) {
#pragma unroll
    for (int j = 0; j < RING; ++j) {
      const int s = s_begin + j;
      ra[j] = pa[2 * s]; rw0[j] = pw0[2 * s]; rw1[j] = pw1[2 * s];
      __builtin_amdgcn_sched_barrier(0);   // slot by slot, as the refills
    }
    for (int g = 0; g < groups; ++g) {
#pragma unroll
      for (int j = 0; j < RING; ++j) {
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(rw0[j], ra[j], c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(rw1[j], ra[j], c1, 0, 0, 0);
        const int s = min(s_begin + (g + 1) * RING + j, s_end - 1);   // past the end: reload
        ra[j] = pa[2 * s]; rw0[j] = pw0[2 * s]; rw1[j] = pw1[2 * s];
        // keep the refill here: clustered at the end of the group, the loads
        // would be waited for a few MFMAs after their issue
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  for (int s = s_begin + groups * RING; s < s_end; ++s) {
    const bf16x8_t va = pa[2 * s];
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pw0[2 * s], va, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pw1[2 * s], va, c1, 0, 0, 0);
  }
  acc_to_lds(lds + wave * EPI_TILE, c0, c1, lane);
  __syncthreads();
  epilogue<KS, GELU, uint16_t, uint16_t>(lds, wave, lane, m_tile, n0, M, N, bias, out, ldo,
                                         vec_out);
}

// ---------------------------------------------------------------------------
// fp32 GEMM with the head's modulation applied to its bf16 input as it is
// read: xin = (f32(a) * s1[k]) + m0[k], rounded after the product and after the
// sum (torch's two elementwise kernels), as 32x32x2 fp32 MFMAs.
__device__ __forceinline__ float modulate(float x, float s1, float m0) {
#pragma clang fp contract(off)
  return x * s1 + m0;
}

template <typename WT>
struct WChunk;  // the raw 8 weights of one lane's k-slice
template <>
struct WChunk<uint16_t> {
  uint4 v;
  __device__ __forceinline__ void load(const uint16_t* p) { v = *reinterpret_cast<const uint4*>(p); }
  __device__ __forceinline__ f32x8v get() const { return unpack_bf16x8(v); }
};
template <>
struct WChunk<float> {
  f32x4_t lo, hi;
  __device__ __forceinline__ void load(const float* p) {
    lo = *reinterpret_cast<const f32x4_t*>(p);
    hi = *reinterpret_cast<const f32x4_t*>(p + 4);
  }
  __device__ __forceinline__ f32x8v get() const {
    return f32x8v{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
};

struct ModChunk {
  uint4 a;
  f32x4_t s_lo, s_hi, m_lo, m_hi;
  __device__ __forceinline__ void load(const uint16_t* pa, const float* s1, const float* m0) {
    a = *reinterpret_cast<const uint4*>(pa);
    s_lo = *reinterpret_cast<const f32x4_t*>(s1);
    s_hi = *reinterpret_cast<const f32x4_t*>(s1 + 4);
    m_lo = *reinterpret_cast<const f32x4_t*>(m0);
    m_hi = *reinterpret_cast<const f32x4_t*>(m0 + 4);
  }
};

template <typename WT>
__device__ __forceinline__ void mod_step(f32x16_t& c0, f32x16_t& c1, const ModChunk& x,
                                         const WChunk<WT>& w0, const WChunk<WT>& w1) {
  const f32x8v xa = unpack_bf16x8(x.a);
  const float sv[8] = {x.s_lo[0], x.s_lo[1], x.s_lo[2], x.s_lo[3], x.s_hi[0], x.s_hi[1], x.s_hi[2], x.s_hi[3]};
  const float mv[8] = {x.m_lo[0], x.m_lo[1], x.m_lo[2], x.m_lo[3], x.m_hi[0], x.m_hi[1], x.m_hi[2], x.m_hi[3]};
  const f32x8v b0 = w0.get(), b1 = w1.get();
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float xin = modulate(xa[i], sv[i], mv[i]);
    c0 = __builtin_amdgcn_mfma_f32_32x32x2f32(b0[i], xin, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x2f32(b1[i], xin, c1, 0, 0, 0);
  }
}

template <typename WT, int KS>
__global__ __launch_bounds__(256) void linear_f32_modulated_kernel(
    const uint16_t* __restrict__ a, int64_t lda, const float* __restrict__ s1,
    const float* __restrict__ m0, const WT* __restrict__ w, int64_t ldw,
    const WT* __restrict__ bias, float* __restrict__ out, int64_t ldo, int M, int N, int K,
    bool vec_out) {
  __shared__ __attribute__((aligned(16))) float lds[4 * EPI_TILE];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m_tile = blockIdx.y * (KS == 1 ? 4 * WT_M : WT_M) + (KS == 1 ? WT_M * wave : 0);
  const int n0 = blockIdx.x * WT_N;
  const int r = lane & 31, kh = (lane >> 5) * 8;
  const uint16_t* pa = a + (int64_t)min(m_tile + r, M - 1) * lda + kh;
  const WT* pw0 = w + (int64_t)min(n0 + r, N - 1) * ldw + kh;
  const WT* pw1 = w + (int64_t)min(n0 + 32 + r, N - 1) * ldw + kh;
  const float* ps = s1 + kh;
  const float* pm = m0 + kh;
  const int steps = K / 16;
  const int s_begin = KS == 1 ? 0 : wave * (steps / KS);
  const int s_end = KS == 1 ? steps : s_begin + steps / KS;
  const int groups = (s_end - s_begin) / RING;
  f32x16_t c0 = {}, c1 = {};
  ModChunk rx[RING];
  WChunk<WT> rw0[RING], rw1[RING];
  if (groups > 0) {
#pragma unroll
    for (int j = 0; j < RING; ++j) {
      const int k = 16 * (s_begin + j);
      rx[j].load(pa + k, ps + k, pm + k);
      rw0[j].load(pw0 + k);
      rw1[j].load(pw1 + k);
      __builtin_amdgcn_sched_barrier(0);   // slot by slot, as the refills
    }
    for (int g = 0; g < groups; ++g) {
#pragma unroll
      for (int j = 0; j < RING; ++j) {
        mod_step<WT>(c0, c1, rx[j], rw0[j], rw1[j]);
        const int k = 16 * min(s_begin + (g + 1) * RING + j, s_end - 1);
        rx[j].load(pa + k, ps + k, pm + k);
        rw0[j].load(pw0 + k);
        rw1[j].load(pw1 + k);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  for (int s = s_begin + groups * RING; s < s_end; ++s) {
    ModChunk x;
    WChunk<WT> w0, w1;
    x.load(pa + 16 * s, ps + 16 * s, pm + 16 * s);
    w0.load(pw0 + 16 * s);
    w1.load(pw1 + 16 * s);
    mod_step<WT>(c0, c1, x, w0, w1);
  }
  acc_to_lds(lds + wave * EPI_TILE, c0, c1, lane);
  __syncthreads();
  epilogue<KS, 0, float, WT>(lds, wave, lane, m_tile, n0, M, N, bias, out, ldo, vec_out);
}

// ---------------------------------------------------------------------------
// fp32 GEMV rows: out[m, n] = sum_k x[m, k] w[n, k] + b[n].  One wave per
// output (4 per workgroup); the lanes stride the row 8 elements at a time and
// the 64 partial sums reduce across the wave.
template <typename WT>
__global__ __launch_bounds__(256) void gemv_f32_kernel(const float* __restrict__ x, int64_t ldx,
                                                       const WT* __restrict__ w, int64_t ldw,
                                                       const WT* __restrict__ bias,
                                                       float* __restrict__ out, int64_t ldo,
                                                       int N, int K) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;  // whole waves: no barrier follows
  const int m = blockIdx.y;
  const float* xr = x + (int64_t)m * ldx;
  const WT* wr = w + (int64_t)n * ldw;
  float acc = 0.f;
  for (int k = lane * 8; k < K; k += 512) {
    const f32x8v xv = load8_f32<float>(xr + k);
    const f32x8v wv = load8_f32<WT>(wr + k);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc = __builtin_fmaf(xv[i], wv[i], acc);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off);
  if (lane == 0) out[(int64_t)m * ldo + n] = acc + (bias ? load1_f32<WT>(bias, n) : 0.f);
}

bool aligned_rows16(const void* p, int64_t ld, int elem) {
  return aligned16(p) && (ld * elem) % 16 == 0;
}

}  // namespace
}  // namespace srdit

using namespace srdit;

namespace srdit {
namespace {

// Split k over the workgroup's 4 waves when 128 x 64 tiles would leave the
// grid under two workgroups per CU and every wave gets whole groups of steps.
int pick_ks(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = ((M + 4 * WT_M - 1) / (4 * WT_M)) * ((N + WT_N - 1) / WT_N);
  const int64_t steps = K / 16;
  return (steps % 4 == 0 && steps >= 16 && tiles < 512) ? 4 : 1;
}

dim3 dense_grid(int64_t M, int64_t N, int ks) {
  const int64_t rows = ks == 1 ? 4 * WT_M : WT_M;
  return dim3((unsigned)((N + WT_N - 1) / WT_N), (unsigned)((M + rows - 1) / rows));
}

}  // namespace
}  // namespace srdit

extern "C" int srdit_bf16_linear(const void* a, int64_t lda, const void* w, int64_t ldw,
                                 const void* bias, void* out, int64_t ldo, int64_t M, int64_t N,
                                 int64_t K, int epilogue, void* stream) {
  const char* fn = "srdit_bf16_linear";
  SRDIT_REQUIRE(a && w && out, "%s: null operand", fn);
  SRDIT_REQUIRE(M > 0 && N > 0 && K > 0 && M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 31),
                "%s: bad sizes M=%lld N=%lld K=%lld", fn, (long long)M, (long long)N,
                (long long)K);
  SRDIT_REQUIRE(K % 16 == 0, "%s: K=%lld must be a multiple of 16", fn, (long long)K);
  SRDIT_REQUIRE(lda >= K && ldw >= K && ldo >= N, "%s: leading dimensions below the row length",
                fn);
  SRDIT_REQUIRE(aligned_rows16(a, lda, 2) && aligned_rows16(w, ldw, 2),
                "%s: A and W rows must be 16-byte aligned", fn);
  SRDIT_REQUIRE((reinterpret_cast<uintptr_t>(out) & 1) == 0 &&
                    (!bias || (reinterpret_cast<uintptr_t>(bias) & 1) == 0),
                "%s: misaligned bf16 output or bias", fn);
  const bool vec_out = aligned_rows16(out, ldo, 2);
  SRDIT_REQUIRE(epilogue == 0 || epilogue == 1, "%s: epilogue %d is not 0 (none) or 1 (gelu)", fn,
                epilogue);
  // Grids of at least 128 256x256 tiles with contiguous rows take the
  // persistent LDS-pipelined GEMM (fp8.hip, bf16 operands); the rest (few
  // rows, like the 512-token text embedding, or odd layouts) the kernels here.
  const int64_t big_tiles = ((M + 255) / 256) * ((N + 255) / 256);
  if (big_tiles >= 128 && K % 64 == 0 && N % 16 == 0 && lda == K && ldw == K && aligned16(bias) &&
      aligned_rows16(out, ldo, 2) &&
      M * K * 2 < (1LL << 31) && N * K * 2 < (1LL << 31) && (255 * ldo + N) * 2 + 16 < (1LL << 31))
    return bf16_gemm_persistent(a, w, bias, out, M, N, K, ldo, epilogue, stream, fn);
  const int ks = pick_ks(M, N, K);
  const dim3 grid = dense_grid(M, N, ks);
  SRDIT_REQUIRE(grid.y < 65536u * 16, "%s: M=%lld too large", fn, (long long)M);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* ap = static_cast<const uint16_t*>(a);
  const uint16_t* wp = static_cast<const uint16_t*>(w);
  const uint16_t* bp = static_cast<const uint16_t*>(bias);
  uint16_t* op = static_cast<uint16_t*>(out);
#define SRDIT_BL(G, KS)                                                                      \
  bf16_linear_kernel<G, KS><<<grid, 256, 0, s>>>(ap, lda, wp, ldw, bp, op, ldo, (int)M, (int)N, \
                                                 (int)K, vec_out)
  if (epilogue && ks == 4) SRDIT_BL(1, 4);
  else if (epilogue) SRDIT_BL(1, 1);
  else if (ks == 4) SRDIT_BL(0, 4);
  else SRDIT_BL(0, 1);
#undef SRDIT_BL
  SRDIT_LAUNCH_CHECK("bf16_linear_kernel");
  return SRDIT_OK;
}

extern "C" int srdit_linear_f32_modulated(const void* a, int64_t lda, const float* s1,
                                          const float* m0, const void* w, int64_t ldw,
                                          const void* bias, int w_dtype, float* out, int64_t ldo,
                                          int64_t M, int64_t N, int64_t K, void* stream) {
  const char* fn = "srdit_linear_f32_modulated";
  SRDIT_REQUIRE(a && s1 && m0 && w && out, "%s: null operand", fn);
  SRDIT_REQUIRE(w_dtype == SRDIT_DTYPE_BF16 || w_dtype == SRDIT_DTYPE_FP32,
                "%s: w_dtype %d is not bf16 (0) or fp32 (2)", fn, w_dtype);
  SRDIT_REQUIRE(M > 0 && N > 0 && K > 0 && M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 31),
                "%s: bad sizes M=%lld N=%lld K=%lld", fn, (long long)M, (long long)N,
                (long long)K);
  SRDIT_REQUIRE(K % 16 == 0, "%s: K=%lld must be a multiple of 16", fn, (long long)K);
  SRDIT_REQUIRE(lda >= K && ldw >= K && ldo >= N, "%s: leading dimensions below the row length",
                fn);
  const int welem = w_dtype == SRDIT_DTYPE_FP32 ? 4 : 2;
  SRDIT_REQUIRE(aligned_rows16(a, lda, 2) && aligned_rows16(w, ldw, welem) && aligned16(s1) &&
                    aligned16(m0),
                "%s: A, W, s1 and m0 must be 16-byte aligned (rows included)", fn);
  SRDIT_REQUIRE((reinterpret_cast<uintptr_t>(out) & 3) == 0 &&
                    (!bias || (reinterpret_cast<uintptr_t>(bias) & (welem - 1)) == 0),
                "%s: misaligned output or bias", fn);
  const bool vec_out = aligned_rows16(out, ldo, 4);
  const int ks = pick_ks(M, N, K);
  const dim3 grid = dense_grid(M, N, ks);
  SRDIT_REQUIRE(grid.y < 65536u * 16, "%s: M=%lld too large", fn, (long long)M);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* ap = static_cast<const uint16_t*>(a);
#define SRDIT_LF(WT, KS)                                                                        \
  linear_f32_modulated_kernel<WT, KS><<<grid, 256, 0, s>>>(ap, lda, s1, m0,                     \
                                                           static_cast<const WT*>(w), ldw,      \
                                                           static_cast<const WT*>(bias), out,   \
                                                           ldo, (int)M, (int)N, (int)K, vec_out)
  if (w_dtype == SRDIT_DTYPE_FP32 && ks == 4) SRDIT_LF(float, 4);
  else if (w_dtype == SRDIT_DTYPE_FP32) SRDIT_LF(float, 1);
  else if (ks == 4) SRDIT_LF(uint16_t, 4);
  else SRDIT_LF(uint16_t, 1);
#undef SRDIT_LF
  SRDIT_LAUNCH_CHECK("linear_f32_modulated_kernel");
  return SRDIT_OK;
}

extern "C" int srdit_gemv_f32(const float* x, int64_t ldx, const void* w, int64_t ldw,
                              const void* bias, int w_dtype, float* out, int64_t ldo, int64_t M,
                              int64_t N, int64_t K, void* stream) {
  const char* fn = "srdit_gemv_f32";
  SRDIT_REQUIRE(x && w && out, "%s: null operand", fn);
  SRDIT_REQUIRE(w_dtype == SRDIT_DTYPE_BF16 || w_dtype == SRDIT_DTYPE_FP32,
                "%s: w_dtype %d is not bf16 (0) or fp32 (2)", fn, w_dtype);
  SRDIT_REQUIRE(M > 0 && M < 65536 && N > 0 && N < (1LL << 31) && K > 0 && K < (1LL << 31),
                "%s: bad sizes M=%lld N=%lld K=%lld", fn, (long long)M, (long long)N,
                (long long)K);
  SRDIT_REQUIRE(K % 8 == 0, "%s: K=%lld must be a multiple of 8", fn, (long long)K);
  SRDIT_REQUIRE(ldx >= K && ldw >= K && ldo >= N, "%s: leading dimensions below the row length",
                fn);
  const int welem = w_dtype == SRDIT_DTYPE_FP32 ? 4 : 2;
  SRDIT_REQUIRE(aligned_rows16(x, ldx, 4) && aligned_rows16(w, ldw, welem),
                "%s: x and W rows must be 16-byte aligned", fn);
  SRDIT_REQUIRE((reinterpret_cast<uintptr_t>(out) & 3) == 0 &&
                    (!bias || (reinterpret_cast<uintptr_t>(bias) & (welem - 1)) == 0),
                "%s: misaligned output or bias", fn);
  const dim3 grid((unsigned)((N + 3) / 4), (unsigned)M);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (w_dtype == SRDIT_DTYPE_FP32)
    gemv_f32_kernel<float><<<grid, 256, 0, s>>>(x, ldx, static_cast<const float*>(w), ldw,
                                                static_cast<const float*>(bias), out, ldo, (int)N,
                                                (int)K);
  else
    gemv_f32_kernel<uint16_t><<<grid, 256, 0, s>>>(x, ldx, static_cast<const uint16_t*>(w), ldw,
                                                   static_cast<const uint16_t*>(bias), out, ldo,
                                                   (int)N, (int)K);
  SRDIT_LAUNCH_CHECK("gemv_f32_kernel");
  return SRDIT_OK;
}
