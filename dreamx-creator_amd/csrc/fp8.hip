// fp8 e4m3 quantisers and the scaled fp8 GEMM for gfx950.
//
// Quantisers (fp8_linear.py:93-103): scale = max(amax * fl32(1/448), 1e-12),
// q = e4m3(clamp(x / scale, +-448)) with the IEEE quotient (formed from the
// shared scale's reciprocal and one FMA correction, SharedDivisor in
// fp8_common.h) and round-to-nearest-even conversion (v_cvt_pk_fp8_f32 writes
// OCP e4m3fn on gfx950).  The scale is a
// multiply by the fp32 reciprocal because that is what `amax / 448.0` computes
// on the GPU: torch divides a GPU tensor by a Python scalar as a multiply by
// the scalar's fp32 reciprocal (and inductor lowers division by a constant the
// same way); `x / scale`, with a tensor divisor, is a true division.  The row-wise
// kernel is one wavefront per row; the per-tensor one is an amax pass
// (integer max over the float bits of |x|, so a NaN wins as in torch's amax)
// followed by a quantise pass that reads the amax from device memory.
//
// GEMM: out = bf16(a . b^T * sa * sb + bias) on v_mfma_f32_32x32x64_f8f6f4.
// A workgroup of four wavefronts computes a 256 x 256 output tile; each
// wavefront owns 128 x 128 (sixteen 32 x 32 accumulators).  K advances 128
// bytes at a time through a two-stage LDS ring filled by buffer_load ... lds
// (16 bytes per lane straight into LDS); rows past M or N read as zero through
// the buffer descriptor's range check.  LDS rows are 128 bytes; 16-byte chunk c
// of row r sits at chunk position c ^ ((r >> 1) & 7), which makes every
// operand read (32 rows x 16 bytes per half-wave) conflict-free.  The MFMA's A
// operand is the weight tile and its B operand the activation tile, so the
// accumulator holds out^T: each lane owns one output row and runs of four
// consecutive columns, stored as 8-byte bf16 quads.
#include "common.h"
#include "fp8_common.h"

#include <mutex>
#include <type_traits>
#include <utility>

namespace srdit {
namespace {

using namespace q8;

// ---------------------------------------------------------------- quantisers

// Eight consecutive elements of a row as float, plus the max of their |x|
// bit patterns (non-negative floats order like their bits; NaN sorts last).
template <typename T> struct Load8;

template <> struct Load8<uint16_t> {  // bf16
  static __device__ __forceinline__ void get(const void* row, int64_t c, float f[8]) {
    const uint4 v = reinterpret_cast<const uint4*>(row)[c];
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(w[i] << 16);
      f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
};

template <> struct Load8<_Float16> {
  static __device__ __forceinline__ void get(const void* row, int64_t c, float f[8]) {
    const f16x8_t v = reinterpret_cast<const f16x8_t*>(row)[c];
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (float)v[i];
  }
};

template <> struct Load8<float> {
  static __device__ __forceinline__ void get(const void* row, int64_t c, float f[8]) {
    const float4 a = reinterpret_cast<const float4*>(row)[2 * c];
    const float4 b = reinterpret_cast<const float4*>(row)[2 * c + 1];
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
  }
};

__device__ __forceinline__ uint32_t abs_bits_max8(const float f[8], uint32_t m) {
#pragma unroll
  for (int i = 0; i < 8; ++i) m = max(m, __float_as_uint(f[i]) & 0x7fffffffu);
  return m;
}

__device__ __forceinline__ uint32_t wave_umax(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o));
  return v;
}


// One wavefront per row, four rows per workgroup.  The second pass re-reads
// the row, which is still in the L1/L2 after the first.
template <typename T>
__global__ __launch_bounds__(256) void quant_rowwise_kernel(const T* __restrict__ x, int64_t M,
                                                            int64_t K, int64_t ldx,
                                                            uint8_t* __restrict__ xq,
                                                            float* __restrict__ scale) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const T* xr = x + row * ldx;
  const int64_t nchunk = K >> 3;
  uint32_t amax = 0;
  for (int64_t c = lane; c < nchunk; c += 64) {
    float f[8];
    Load8<T>::get(xr, c, f);
    amax = abs_bits_max8(f, amax);
  }
  amax = wave_umax(amax);
  const float s = scale_from_amax_bits(amax);
  if (lane == 0) scale[row] = s;
  const SharedDivisor sd(s);
  uint2* qr = reinterpret_cast<uint2*>(xq + row * K);
  for (int64_t c = lane; c < nchunk; c += 64) {
    float f[8];
    Load8<T>::get(xr, c, f);
    qr[c] = to_e4m3x8(f, sd);
  }
}

__global__ void clear_u32_kernel(uint32_t* p) { *p = 0u; }

// Grid-stride amax: each wavefront walks rows wave_id, wave_id + n_waves, ...
template <typename T>
__global__ __launch_bounds__(256) void amax_kernel(const T* __restrict__ x, int64_t M, int64_t K,
                                                   int64_t ldx, uint32_t* __restrict__ amax_ws) {
  __shared__ uint32_t part[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t nchunk = K >> 3;
  uint32_t amax = 0;
  for (int64_t row = (int64_t)blockIdx.x * 4 + wave; row < M; row += (int64_t)gridDim.x * 4) {
    const T* xr = x + row * ldx;
    // four chunks per lane in flight; a clamped index re-reads a chunk already
    // counted, which leaves the max unchanged
    for (int64_t c0 = lane; c0 < nchunk; c0 += 256) {
      float f[4][8];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t c = c0 + 64 * u;
        Load8<T>::get(xr, c < nchunk ? c : nchunk - 1, f[u]);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) amax = abs_bits_max8(f[u], amax);
    }
  }
  amax = wave_umax(amax);
  if (lane == 0) part[wave] = amax;
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t m = max(max(part[0], part[1]), max(part[2], part[3]));
    raise_max_word(amax_ws, m);
  }
}

constexpr int QU = 4;  // 16-byte chunks per lane in flight in the quantise pass

template <typename T>
__global__ __launch_bounds__(256) void quant_tensor_kernel(const T* __restrict__ x, int64_t M,
                                                           int64_t K, int64_t ldx,
                                                           uint8_t* __restrict__ xq,
                                                           float* __restrict__ scale,
                                                           const uint32_t* __restrict__ amax_ws) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const float s = scale_from_amax_bits(*amax_ws);
  const SharedDivisor sd(s);
  if (blockIdx.x == 0 && threadIdx.x == 0) scale[0] = s;
  const int64_t nchunk = K >> 3;
  for (int64_t row = (int64_t)blockIdx.x * 4 + wave; row < M; row += (int64_t)gridDim.x * 4) {
    const T* xr = x + row * ldx;
    uint2* qr = reinterpret_cast<uint2*>(xq + row * K);
    // QU chunks per lane in flight: the loads (indices clamped into the row, so
    // they need no branch) all issue before the first conversion.
    for (int64_t c0 = lane; c0 < nchunk; c0 += 64 * QU) {
      float f[QU][8];
#pragma unroll
      for (int u = 0; u < QU; ++u) {
        const int64_t c = c0 + 64 * u;
        Load8<T>::get(xr, c < nchunk ? c : nchunk - 1, f[u]);
      }
#pragma unroll
      for (int u = 0; u < QU; ++u) {
        const int64_t c = c0 + 64 * u;
        if (c < nchunk) qr[c] = to_e4m3x8(f[u], sd);
      }
    }
  }
}

// ---------------------------------------------------------------------- GEMM

constexpr int GT = 256;                       // tile rows (M) and columns (N)
constexpr int G_GROUP_M = 4;                  // M tiles per raster group

struct GemmArgs {
  const uint8_t* a;      // [M, K]
  const uint8_t* b;      // [N, K]
  const float* sa;       // [1] or [M]
  const float* sb;       // [1] or [N]
  const uint16_t* bias;  // [N] bf16 or null
  uint16_t* out;         // [M, ldo] bf16
  int M, N, K;
  int64_t ldo;
  int sa_per_row, sb_per_col;
  int tiles_m, tiles_n;
  uint32_t* amax_out;  // AMAX epilogue only
  // Split output (0: none): columns [j split_n, (j + 1) split_n) are stored at
  // out + j split_stride as a block of rows of stride ldo.
  int64_t split_n, split_stride;
  // This launch's tiles: [task_base, task_base + n_tasks) of the raster order.
  int task_base, n_tasks;
  // split_k > 0: each of those tiles is split over split_k workgroups along K.
  // Workgroup u takes tile task_base + u / split_k and the K stages
  // [c nks / split_k, (c + 1) nks / split_k), c = u % split_k, and writes its fp32
  // partial to ws_part; the last of a tile's workgroups to arrive (ws_cnt, one
  // word per tile, left 0) sums the partials in chunk order and stores the tile.
  int split_k;
  float* ws_part;
  uint32_t* ws_cnt;
};

// Bytes of one split-K partial, a 256 x 256 fp32 tile: 8 wavefronts x 8 accumulator
// blocks x 16 registers x 64 lanes.
constexpr int64_t G_PART_BYTES = 8 * 8 * 16 * 64 * 4;

__device__ __forceinline__ void compiler_fence_gemm() { asm volatile("" ::: "memory"); }

// Wait until at most N vector-memory operations of this wavefront are in
// flight (its newest ones), and for all its LDS reads (lgkmcnt(0)).
template <int N>
__device__ __forceinline__ void waitcnt_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt out of range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

__device__ __forceinline__ i32x8_t read_frag(const uint8_t* lds, int off_lo, int off_hi) {
  const i32x4_t lo = *reinterpret_cast<const i32x4_t*>(lds + off_lo);
  const i32x4_t hi = *reinterpret_cast<const i32x4_t*>(lds + off_hi);
  return i32x8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// GELU through a table.  The FFN's hidden activation h = bf16(gelu_tanh(x)) is
// a function of the 16 bits of a bf16 x, so the per-tensor GELU quantiser looks
// h up in a 65,536-entry table instead of evaluating tanhf per element (the
// passes were bound by tanhf).  gelu_lut_build_kernel writes the table (one
// entry per thread, the same gelu_tanh and bf16 rounding as the GEMM epilogue).
// Pass 1 copies it into LDS (128 KB: one workgroup per CU), looks every element
// up there and reduces max |h| (and stores h when asked); pass 2 turns it into
// a table of codes at the scale of that amax and looks the codes up.
constexpr int LUT_N = 65536;
constexpr int LUT_WAVES = 16;  // wavefronts per workgroup of the table passes

__global__ __launch_bounds__(256) void gelu_lut_build_kernel(uint16_t* __restrict__ lut,
                                                             uint32_t* __restrict__ amax_ws) {
  const int i = blockIdx.x * 256 + threadIdx.x;  // < LUT_N / 2: entries 2i, 2i + 1
  typedef float f32x2v __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
  const float x0 = __uint_as_float(static_cast<uint32_t>(2 * i) << 16);
  const float x1 = __uint_as_float(static_cast<uint32_t>(2 * i + 1) << 16);
  reinterpret_cast<uint32_t*>(lut)[i] =
      __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2v{gelu_tanh(x0), gelu_tanh(x1)},
                                                           bf16x2v));
  if (i == 0) *amax_ws = 0u;
}

__device__ __forceinline__ void load_lut_to_lds(uint16_t* lds, const uint16_t* __restrict__ lut) {
  const uint4* src = reinterpret_cast<const uint4*>(lut);
  uint4* dst = reinterpret_cast<uint4*>(lds);
  for (int i = threadIdx.x; i < LUT_N / 8; i += blockDim.x) dst[i] = src[i];
  __syncthreads();
}

// h for the 8 bf16 of one 16-byte chunk: four words of two table entries each.
__device__ __forceinline__ uint4 lut8(const uint16_t* lds, uint4 v) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    o[i] = static_cast<uint32_t>(lds[w[i] & 0xffffu]) | (static_cast<uint32_t>(lds[w[i] >> 16]) << 16);
  return make_uint4(o[0], o[1], o[2], o[3]);
}

__device__ __forceinline__ uint32_t abs_bits_max_bf16x8(uint4 h, uint32_t m) {
  const uint32_t w[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) m = max(m, max((w[i] & 0x7fffu) << 16, w[i] & 0x7fff0000u));
  return m;
}

// Inputs whose largest positive value is at least this (0.375) have
// max |h| = |h(that value)|: h is non-decreasing over x >= 0 and |h| <= 0.1700
// below 0, while h(0.375) = 0.2373.
constexpr uint32_t GELU_AMAX_SHORTCUT = 0x3ec00000u;

__global__ __launch_bounds__(64 * LUT_WAVES) void gelu_lut_amax_kernel(
    const uint16_t* __restrict__ x, int64_t M, int64_t K, int64_t ldx, uint16_t* __restrict__ h,
    int64_t ldh, const uint16_t* __restrict__ lut, uint32_t* __restrict__ amax_ws,
    const uint32_t* __restrict__ xmax_pos) {
  if (xmax_pos) {  // the producer's largest positive value decides the amax on its own
    const uint32_t key = *xmax_pos;
    if (key >= GELU_AMAX_SHORTCUT) {
      if (blockIdx.x == 0 && threadIdx.x == 0)
        *amax_ws = static_cast<uint32_t>(lut[key >> 16] & 0x7fffu) << 16;
      return;
    }
  }
  __shared__ __attribute__((aligned(16))) uint16_t tab[LUT_N];
  __shared__ uint32_t part[LUT_WAVES];
  load_lut_to_lds(tab, lut);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t nchunk = K >> 3;
  uint32_t amax = 0;
  for (int64_t row = (int64_t)blockIdx.x * LUT_WAVES + wave; row < M;
       row += (int64_t)gridDim.x * LUT_WAVES) {
    const uint4* xr = reinterpret_cast<const uint4*>(x + row * ldx);
    uint4* hr = h ? reinterpret_cast<uint4*>(h + row * ldh) : nullptr;
    // QU chunks per lane in flight; a clamped index re-reads a chunk already
    // counted, which leaves the max unchanged
    for (int64_t c0 = lane; c0 < nchunk; c0 += 64 * QU) {
      uint4 v[QU];
#pragma unroll
      for (int u = 0; u < QU; ++u) {
        const int64_t c = c0 + 64 * u;
        v[u] = xr[c < nchunk ? c : nchunk - 1];
      }
#pragma unroll
      for (int u = 0; u < QU; ++u) {
        const uint4 hv = lut8(tab, v[u]);
        amax = abs_bits_max_bf16x8(hv, amax);
        const int64_t c = c0 + 64 * u;
        if (hr && c < nchunk) hr[c] = hv;
      }
    }
  }
  amax = wave_umax(amax);
  if (lane == 0) part[wave] = amax;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t m = part[0];
#pragma unroll
    for (int w = 1; w < LUT_WAVES; ++w) m = max(m, part[w]);
    raise_max_word(amax_ws, m);
  }
}

// The quantise pass's walk for one wavefront takes groups of 64 GQ chunks,
// (row, base) with base a multiple of 64 GQ, row by row.  Two register sets
// alternate, so the loads of the next group are in flight while the current
// one is looked up and stored, across row ends too.  A clamped index re-reads
// a chunk of the row; it is not stored.
constexpr int GQ = 8;  // chunks per lane per group

// The quantise pass through a table of codes: every workgroup first writes the
// e4m3 code of each of the 65,536 bf16 inputs at this call's scale into LDS
// (64 KB, from the h table and the same conversion the per-element pass makes,
// so the codes are the same), then each element of x is one byte lookup.
__device__ __forceinline__ void code_walk(const uint16_t* __restrict__ x, int64_t M, int64_t K,
                                          int64_t ldx, const uint8_t* codes,
                                          uint8_t* __restrict__ xq, int64_t first_row,
                                          int64_t row_step, int lane) {
  const int64_t nchunk = K >> 3;
  struct Pos {
    int64_t row, base;
  };
  auto advance = [&](Pos p) -> Pos {
    p.base += 64 * GQ;
    if (p.base >= nchunk) { p.base = 0; p.row += row_step; }
    return p;
  };
  auto load = [&](Pos p, uint4 (&v)[GQ]) __attribute__((always_inline)) {
    const uint4* xr = reinterpret_cast<const uint4*>(x + p.row * ldx);
#pragma unroll
    for (int u = 0; u < GQ; ++u) {
      const int64_t c = p.base + lane + 64 * u;
      v[u] = xr[c < nchunk ? c : nchunk - 1];
    }
  };
  auto look = [&](uint32_t w) __attribute__((always_inline)) -> uint32_t {
    return static_cast<uint32_t>(codes[w & 0xffffu]) |
           (static_cast<uint32_t>(codes[w >> 16]) << 8);
  };
  auto quant = [&](Pos p, const uint4 (&v)[GQ]) __attribute__((always_inline)) {
    uint2* qr = reinterpret_cast<uint2*>(xq + p.row * K);
#pragma unroll
    for (int u = 0; u < GQ; ++u) {
      const uint2 q = make_uint2(look(v[u].x) | (look(v[u].y) << 16),
                                 look(v[u].z) | (look(v[u].w) << 16));
      const int64_t c = p.base + lane + 64 * u;
      if (c < nchunk) qr[c] = q;
    }
  };
  Pos pa{first_row, 0};
  if (pa.row >= M) return;
  uint4 va[GQ], vb[GQ];
  load(pa, va);
  Pos pb = advance(pa);
  if (pb.row < M) load(pb, vb);
  while (true) {
    quant(pa, va);
    pa = advance(pb);
    if (pa.row < M) load(pa, va);
    if (pb.row >= M) break;
    quant(pb, vb);
    pb = advance(pa);
    if (pb.row < M) load(pb, vb);
    if (pa.row >= M) break;
  }
}

__global__ __launch_bounds__(64 * LUT_WAVES) void gelu_code_quant_kernel(
    const uint16_t* __restrict__ x, int64_t M, int64_t K, int64_t ldx,
    const uint16_t* __restrict__ lut, uint8_t* __restrict__ xq, float* __restrict__ scale,
    const uint32_t* __restrict__ amax_ws) {
  __shared__ __attribute__((aligned(16))) uint8_t codes[LUT_N];
  const float s = scale_from_amax_bits(*amax_ws);
  const SharedDivisor sd(s);
  if (blockIdx.x == 0 && threadIdx.x == 0) scale[0] = s;
  // the code of input bits i: e4m3(h(i) / s), eight entries per 16-byte read of h
  const uint4* src = reinterpret_cast<const uint4*>(lut);
  for (int i = threadIdx.x; i < LUT_N / 8; i += blockDim.x) {
    const uint4 hv = src[i];
    const uint32_t w[4] = {hv.x, hv.y, hv.z, hv.w};
    float f[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      f[2 * k] = __uint_as_float(w[k] << 16);
      f[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
    }
    reinterpret_cast<uint2*>(codes)[i] = sd.fast ? to_e4m3x8<true>(f, sd) : to_e4m3x8<false>(f, sd);
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t first = (int64_t)blockIdx.x * LUT_WAVES + wave;
  const int64_t step = (int64_t)gridDim.x * LUT_WAVES;
  code_walk(x, M, K, ldx, codes, xq, first, step, lane);
}

// ------------------------------------------------------------------ the GEMM
//
// One persistent workgroup of eight wavefronts per CU.  Workgroup b runs on
// XCD b % 8; each XCD owns one contiguous range of 256 x 256 output tiles
// (rastered in groups of G_GROUP_M tile rows, column by column, so the
// workgroups of one XCD share operand rows in its L2), and workgroup slot
// b / 8 walks that range with a stride of the XCD's workgroup count.
//
// Operands reach LDS by buffer_load_dwordx4 ... lds, one 128-byte K stage of
// both 256-row tiles at a time (whole 128-byte lines: the L2 -> LDS path is
// limited by lines, not bytes) through two 64 KB slots.  Each stage is computed
// as two 64-byte sub-steps of v_mfma_f32_32x32x64_f8f6f4 with double-buffered
// fragments: the MFMAs of one sub-step run while the fragments of the next are
// read, so the only barrier is once per stage, where the stage after next is
// filled into the slot the current stage has just left (its fragments are in
// registers by then).  The K loop is one stream of stages across tile
// boundaries, so the next tile's first stages are in flight while a tile
// finishes.  Wave (wm, wn) = (w & 1, w >> 1) owns activation rows
// [128 wm, +128) and weight rows [64 wn, +64): 2 x 4 blocks, 128 accumulators,
// which hold out^T (the weight is the MFMA's A operand).
//
// vmcnt is counted exactly, since the fills are inline asm the compiler cannot
// see: each wavefront issues 8 fill DMAs per stage, one epilogue-data DMA per
// tile (wavefronts 0-2, just before the tile's last stage), and EPI_STORES
// stores per tile; at the barrier before stage S + 1 is read, only the stores
// of a tile that ended right before stage S can be newer than fill S + 1.
//
// Epilogue data (per-row activation scales, per-column weight scales, bias)
// is DMA'd into one of three 3 KB LDS regions per tile, so no epilogue load
// touches vmcnt.  Each 32 x 32 output block is transposed through a 2 KB
// per-wavefront LDS buffer and stored as 16 rows x 64 bytes per instruction;
// rows past M and columns past N fall outside the store descriptor.
//
// Measured on one MI355X (per-tensor scales, bias, random operands): 21600 x
// 3072 x 3072 in 163-168 us (2.43-2.51 PFLOP/s), 21600 x 14336 x 3072 in
// 795-799 us (2.38-2.39), 21600 x 3072 x 14336 in 762-763 us (2.49-2.50);
// without its fills the same loop runs 2.85-3.3 PFLOP/s, where core-clock
// counters show the MFMA pipe ~99% busy at the ~1.57 GHz the chip sustains
// under that load.

// Order key of the largest positive value: the float bits of a non-negative
// x (so +inf and larger values win), 0 for negative x, and 0x7fffffff for any
// NaN, so a NaN anywhere makes the reduced key a NaN.
__device__ __forceinline__ uint32_t pos_key(uint32_t bits) {
  if ((bits & 0x7fffffffu) > 0x7f800000u) return 0x7fffffffu;
  return (bits & 0x80000000u) ? 0u : bits;
}

constexpr int G_FK = 128;                      // K bytes per fill stage
constexpr int G_OPB = GT * G_FK;               // one operand tile of a stage: 32 KB
constexpr int G_SLOT = 2 * G_OPB;              // 64 KB
constexpr int G_NI = 2, G_NJ = 4;              // 32 x 32 blocks per wavefront (weight, act)
constexpr int EPI_STORES = G_NI * G_NJ * 2;    // epilogue stores per wavefront per tile
constexpr int G_EPI_OFF = 2 * G_SLOT;          // three epilogue-data regions
constexpr int G_EPI_REG = 3 * 1024;            // sa[256] f32, sb[256] f32, bias[256] bf16 (+pad)
constexpr int G_STG_OFF = G_EPI_OFF + 3 * G_EPI_REG;
constexpr int G_LDS = G_STG_OFF + 8 * 2048;    // + 2 KB transpose buffer per wavefront

struct GemmFrags {
  i32x8_t w[G_NI], x[G_NJ];
};

// AMAX 0: none; 1: max |out| (float bits) into *g.amax_out; 2: the largest
// positive output instead (0 if none, and the bits of a NaN when there is one),
// which bounds the GELU of the output (srdit_fp8_quant_tensor_gelu_ex).
//
// BF 1: the operands are bf16 (g.K counts bytes, two per element) and the
// scales are 1: each 32-byte fragment feeds two 32x32x16 bf16 MFMAs (its two
// 16-byte chunks, paired the same way in both operands), which take the 64
// cycles of the one fp8 MFMA they replace, so the data movement is unchanged.
template <int EPI, int AMAX, int BF = 0, bool SPLIT = false>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void fp8_gemm_kernel(const GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[G_LDS];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave & 1, wn = wave >> 1;

  const uint32_t n_tasks = (uint32_t)g.n_tasks;
  constexpr bool splitk = SPLIT;  // the split launch: one K chunk of one tile per workgroup
  const uint32_t xcd = blockIdx.x & 7u, wslot = blockIdx.x >> 3, per = gridDim.x >> 3;
  const uint32_t r0 = xcd * (n_tasks >> 3) + min(xcd, n_tasks & 7u);
  const uint32_t r1 = r0 + (n_tasks >> 3) + (xcd < (n_tasks & 7u) ? 1u : 0u);
  // split-K: one unit per workgroup (tile sk_tile of the launch, K chunk sk_c)
  const int unit = (int)blockIdx.x;
  const int sk_tile = splitk ? unit / g.split_k : 0, sk_c = splitk ? unit % g.split_k : 0;
  const int my_tiles = splitk ? (sk_tile < (int)n_tasks ? 1 : 0)
                              : ((r0 + wslot < r1) ? (int)((r1 - r0 - wslot + per - 1) / per) : 0);
  if (my_tiles == 0) return;
  const int nks_tile = g.K / G_FK;  // stages of a whole tile
  const int k_first = splitk ? sk_c * nks_tile / g.split_k : 0;
  const int nks = splitk ? (sk_c + 1) * nks_tile / g.split_k - k_first : nks_tile;  // per task
  const int n_total = my_tiles * nks;
  const int width = G_GROUP_M * g.tiles_n;
  auto coords = [&](int t, int& m0, int& n0) __attribute__((always_inline)) {
    const uint32_t task = (uint32_t)g.task_base +
                          (splitk ? (uint32_t)sk_tile : r0 + wslot + per * (uint32_t)t);
    const int group = task / width;
    const int first_m = group * G_GROUP_M;
    const int gsize = min(g.tiles_m - first_m, G_GROUP_M);
    m0 = (first_m + (int)(task % width) % gsize) * GT;
    n0 = ((int)(task % width) / gsize) * GT;
  };
  auto rsrc_of = [](const void* p, int64_t bytes) __attribute__((always_inline)) -> i32x4_t {
    const uint64_t a = reinterpret_cast<uint64_t>(p);
    return i32x4_t{static_cast<int>(static_cast<uint32_t>(a)),
                   static_cast<int>(static_cast<uint32_t>(a >> 32)), static_cast<int>(bytes),
                   0x00020000};
  };

  // Fill: wavefront w writes rows [32 w, +32) of both tiles in four 1 KB DMAs
  // each (8 rows of 128 bytes); lane l -> row 8 q + l/8, position l%8 holding
  // source chunk (l%8) ^ ((row >> 1) & 7).  Rows past M or N read as zero
  // through the descriptor's range check.
  const int fpos = lane & 7;
  const int fbase = (wave * 32 + (lane >> 3)) * g.K;
  const int fv_even = fbase + ((fpos ^ ((lane >> 4) & 7)) * 16);
  const int fv_odd = fbase + ((fpos ^ ((4 + (lane >> 4)) & 7)) * 16);
  const int frow8 = 8 * g.K;
  const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem));
  const uint32_t lds_w = lds_base + wave * 32 * G_FK;
  auto dma = [](i32x4_t rsrc, int voff, int soff, uint32_t lds) __attribute__((always_inline)) {
    asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(rsrc), "s"(soff),
                 "{m0}"(lds)
                 : "memory");
  };
  int f_t = 0, f_kt = 0, f_slot = 0;  // fill cursor: tile, stage in tile, slot
  int f_m0 = 0, f_n0 = 0;             // the cursor tile's first row and column
  i32x4_t f_ra = {}, f_rb = {};
  auto fill_next = [&]() __attribute__((always_inline)) {
    // The tile's coordinates, once per tile (its integer divisions would
    // otherwise run after every stage's barrier).
    if (f_kt == 0) {
      coords(f_t, f_m0, f_n0);
      f_ra = rsrc_of(g.a + (int64_t)f_m0 * g.K, (int64_t)(g.M - f_m0) * g.K);
      f_rb = rsrc_of(g.b + (int64_t)f_n0 * g.K, (int64_t)(g.N - f_n0) * g.K);
    }
    if (f_kt == nks - 1 && wave < 3) {  // the tile's epilogue data, ahead of its last stage
      const int m0 = f_m0, n0 = f_n0;
      i32x4_t r;
      if (wave == 0) r = rsrc_of(g.sa + m0, g.sa_per_row ? (int64_t)(g.M - m0) * 4 : 0);
      else if (wave == 1) r = rsrc_of(g.sb + n0, g.sb_per_col ? (int64_t)(g.N - n0) * 4 : 0);
      else r = rsrc_of(g.bias ? (const void*)(g.bias + n0) : (const void*)g.b,
                       g.bias ? (int64_t)(g.N - n0) * 2 : 0);
      dma(r, 16 * lane, 0, lds_base + G_EPI_OFF + (f_t % 3) * G_EPI_REG + wave * 1024);
    }
    const uint32_t base = lds_w + f_slot * G_SLOT;
    const int koff = (k_first + f_kt) * G_FK;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      dma(f_ra, ((q & 1) ? fv_odd : fv_even) + q * frow8, koff, base + q * 1024);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      dma(f_rb, ((q & 1) ? fv_odd : fv_even) + q * frow8, koff, base + G_OPB + q * 1024);
    if (++f_kt == nks) { f_kt = 0; ++f_t; }
    f_slot ^= 1;
  };

  // Fragment reads: lane l reads row l & 31, bytes [64 kk + 32 (l >> 5), +32)
  // of the stage: two 16-byte chunks at their swizzled positions, which makes
  // the reads of 16 lanes cover all 64 banks.
  const int rrow = lane & 31;
  const int rswz = (rrow >> 1) & 7;
  const int h2 = 2 * (lane >> 5);
  int roff[2][2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int h = 0; h < 2; ++h) roff[kk][h] = rrow * G_FK + (((kk * 4 + h2 + h) ^ rswz) * 16);

  f32x16_t acc[G_NI][G_NJ];
#pragma unroll
  for (int i = 0; i < G_NI; ++i)
#pragma unroll
    for (int j = 0; j < G_NJ; ++j) acc[i][j] = f32x16_t{};
  auto mma_j = [&](const GemmFrags& f, int j) __attribute__((always_inline)) {
    if constexpr (BF) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < G_NI; ++i) {
          const i32x4_t wv = h ? __builtin_shufflevector(f.w[i], f.w[i], 4, 5, 6, 7)
                               : __builtin_shufflevector(f.w[i], f.w[i], 0, 1, 2, 3);
          const i32x4_t xv = h ? __builtin_shufflevector(f.x[j], f.x[j], 4, 5, 6, 7)
                               : __builtin_shufflevector(f.x[j], f.x[j], 0, 1, 2, 3);
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(bf16x8_t, wv), __builtin_bit_cast(bf16x8_t, xv), acc[i][j], 0,
              0, 0);
        }
    } else {
#pragma unroll
      for (int i = 0; i < G_NI; ++i)
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.w[i], f.x[j], acc[i][j], 0,
                                                                    0, 0, 0, 0, 0);
    }
  };
  // The MFMAs of fc, with the reads of sub-step kk of `slot` into fn between
  // them (the scheduling barriers keep that order).
  auto compute = [&](const GemmFrags& fc, GemmFrags& fn, int slot, auto kk_c)
                     __attribute__((always_inline)) {
    constexpr int kk = decltype(kk_c)::value;
    const uint8_t* ta = smem + slot * G_SLOT + wm * 128 * G_FK;
    const uint8_t* tb = smem + slot * G_SLOT + G_OPB + wn * 64 * G_FK;
    mma_j(fc, 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < G_NI; ++i) fn.w[i] = read_frag(tb + i * 32 * G_FK, roff[kk][0], roff[kk][1]);
    __builtin_amdgcn_sched_barrier(0);
    mma_j(fc, 1);
    __builtin_amdgcn_sched_barrier(0);
    fn.x[0] = read_frag(ta + 0 * 32 * G_FK, roff[kk][0], roff[kk][1]);
    fn.x[1] = read_frag(ta + 1 * 32 * G_FK, roff[kk][0], roff[kk][1]);
    __builtin_amdgcn_sched_barrier(0);
    mma_j(fc, 2);
    __builtin_amdgcn_sched_barrier(0);
    fn.x[2] = read_frag(ta + 2 * 32 * G_FK, roff[kk][0], roff[kk][1]);
    fn.x[3] = read_frag(ta + 3 * 32 * G_FK, roff[kk][0], roff[kk][1]);
    __builtin_amdgcn_sched_barrier(0);
    mma_j(fc, 3);
  };

  // Prologue: stages 0 and 1 in flight; wait for stage 0.
  fill_next();
  int pro_newer = 0;
  if (n_total > 1) {
    pro_newer = 8 + ((nks <= 2 && wave < 3) ? 1 : 0);  // stage 1 (and its tile's epilogue data)
    fill_next();
  }
  compiler_fence_gemm();
  if (pro_newer == 0) waitcnt_vm<0>();
  else if (pro_newer == 8) waitcnt_vm<8>();
  else waitcnt_vm<9>();
  __builtin_amdgcn_s_barrier();
  compiler_fence_gemm();
  GemmFrags F0, F1;
  {
    const uint8_t* ta = smem + wm * 128 * G_FK;
    const uint8_t* tb = smem + G_OPB + wn * 64 * G_FK;
#pragma unroll
    for (int i = 0; i < G_NI; ++i) F0.w[i] = read_frag(tb + i * 32 * G_FK, roff[0][0], roff[0][1]);
#pragma unroll
    for (int j = 0; j < G_NJ; ++j) F0.x[j] = read_frag(ta + j * 32 * G_FK, roff[0][0], roff[0][1]);
  }

  const float sa_t = BF ? 1.f : g.sa[0], sb_t = BF ? 1.f : g.sb[0];  // per-tensor scales
  int S = 0;
  for (int t = 0; t < my_tiles; ++t) {
    for (int sl = 0; sl < nks; ++sl, ++S) {
      // sub-step (S, 0): MFMAs of F0, reads of (S, 1) from this stage's slot
      compute(F0, F1, S & 1, std::integral_constant<int, 1>{});
      // sub-step (S, 1): stage S + 1 landed (this wavefront's fills, and after
      // the barrier everyone's); this stage's slot is free for stage S + 2
      compiler_fence_gemm();
      if (sl == 0 && t > 0) waitcnt_vm<EPI_STORES>();  // the previous tile's stores are newer
      else waitcnt_vm<0>();
      __builtin_amdgcn_s_barrier();
      compiler_fence_gemm();
      if (S + 2 < n_total) fill_next();
      compute(F1, F0, (S + 1) & 1, std::integral_constant<int, 0>{});
    }

    // ---- epilogue of tile t
    if constexpr (SPLIT) {  // publish this K chunk; the tile's last arrival stores it
      waitcnt_vm<0>();
      // accumulator register 4 r4 + e of block (i, j), lane l: float
      // (((w 8 + i G_NJ + j) 4 + r4) 64 + l) 4 + e of the unit's partial
      auto part_of = [&](int u) __attribute__((always_inline)) {
        return g.ws_part + (int64_t)u * (G_PART_BYTES / 4) + (int64_t)wave * (8 * 16 * 64);
      };
      float* wp = part_of(unit);
#pragma unroll
      for (int i = 0; i < G_NI; ++i)
#pragma unroll
        for (int j = 0; j < G_NJ; ++j)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4)
            *reinterpret_cast<f32x4_t*>(wp + (((i * G_NJ + j) * 4 + r4) * 64 + lane) * 4) =
                f32x4_t{acc[i][j][4 * r4], acc[i][j][4 * r4 + 1], acc[i][j][4 * r4 + 2],
                        acc[i][j][4 * r4 + 3]};
      __threadfence();  // release: the partial is visible to every XCD
      __syncthreads();
      // epilogue-data region 1 is unused with one task per workgroup
      uint32_t* arrivals = reinterpret_cast<uint32_t*>(smem + G_EPI_OFF + G_EPI_REG);
      if (threadIdx.x == 0) *arrivals = atomicAdd(g.ws_cnt + sk_tile, 1u);
      __syncthreads();
      if (*arrivals != (uint32_t)(g.split_k - 1)) return;  // uniform: not the last arrival
      __threadfence();  // acquire: the other chunks' partials
      // the tile's sum, chunk by chunk in K order (this chunk's own partial
      // included), so the result does not depend on the order of arrival
      for (int c = 0; c < g.split_k; ++c) {
        const float* rp = part_of(sk_tile * g.split_k + c);
#pragma unroll
        for (int i = 0; i < G_NI; ++i) {
          // one accumulator row of blocks at a time (32 registers of loads in
          // flight, not the whole partial's 128)
          f32x4_t v[G_NJ][4];
#pragma unroll
          for (int j = 0; j < G_NJ; ++j)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4)
              v[j][r4] = *reinterpret_cast<const f32x4_t*>(
                  rp + (((i * G_NJ + j) * 4 + r4) * 64 + lane) * 4);
#pragma unroll
          for (int j = 0; j < G_NJ; ++j)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4)
#pragma unroll
              for (int e = 0; e < 4; ++e)
                acc[i][j][4 * r4 + e] = c == 0 ? v[j][r4][e] : acc[i][j][4 * r4 + e] + v[j][r4][e];
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      if (threadIdx.x == 0)  // ready for the next launch
        __hip_atomic_store(g.ws_cnt + sk_tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    int m0, n0;
    coords(t, m0, n0);
    const int rows = min(GT, g.M - m0);
    // the tile's output base: row m0, and with a split output, shifted so that
    // global column n of block j lands at out + j split_stride + (n - j split_n)
    int64_t obase = (int64_t)m0 * g.ldo;
    if (g.split_n) {
      const int64_t blk = n0 / g.split_n;
      obase += blk * (g.split_stride - g.split_n);
    }
    // every store offset of the tile, (row * ldo + column) * 2 for rows < rows
    // and columns < N, stays below this bound
    const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(g.out + obase), (short)0, (int)(((int64_t)(rows - 1) * g.ldo + g.N) * 2),
        0x00020000);
    // lane-derived values are recomputed here, not held across the K loop
    int lane_e = lane;
    asm volatile("" : "+v"(lane_e));
    const int mrow = lane_e & 31;
    const int hh = lane_e >> 5;
    const uint8_t* epi = smem + G_EPI_OFF + (t % 3) * G_EPI_REG;
    uint8_t* stg = smem + G_STG_OFF + wave * 2048;
    const int wswz = (mrow >> 1) & 3;
    const int rb_row = lane_e >> 2, rb_c = lane_e & 3;  // read back 16 rows x 4 chunks per pass
    uint32_t amax = 0;
#pragma unroll
    for (int j = 0; j < G_NJ; ++j) {
      // acc[i][j]: lane l holds row m = wm 128 + 32 j + (l & 31), columns
      // 32 i + 8 q + 4 (l >> 5) + r, r < 4, of the wavefront's 64
      const int ml_w = wm * 128 + j * 32 + mrow;
      const bool mok = ml_w < rows;
      const float sa = g.sa_per_row ? *reinterpret_cast<const float*>(epi + 4 * ml_w) : sa_t;
#pragma unroll
      for (int i = 0; i < G_NI; ++i) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int nl = wn * 64 + i * 32 + 8 * q + 4 * hh;
          const bool nok = n0 + nl < g.N;
          float sb[4], bias[4];
          if (g.sb_per_col) {
            const float4 v = *reinterpret_cast<const float4*>(epi + 1024 + 4 * nl);
            sb[0] = v.x; sb[1] = v.y; sb[2] = v.z; sb[3] = v.w;
          } else {
            sb[0] = sb[1] = sb[2] = sb[3] = sb_t;
          }
          if (g.bias) {
            const uint2 bv = *reinterpret_cast<const uint2*>(epi + 2048 + 2 * nl);
            bias[0] = __uint_as_float(bv.x << 16);
            bias[1] = __uint_as_float(bv.x & 0xffff0000u);
            bias[2] = __uint_as_float(bv.y << 16);
            bias[3] = __uint_as_float(bv.y & 0xffff0000u);
          } else {
            bias[0] = bias[1] = bias[2] = bias[3] = 0.f;
          }
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = acc[i][j][4 * q + r] * sa * sb[r] + bias[r];
          typedef float f32x2v __attribute__((ext_vector_type(2)));
          typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
          bf16x2v p0 = __builtin_convertvector(f32x2v{v[0], v[1]}, bf16x2v);
          bf16x2v p1 = __builtin_convertvector(f32x2v{v[2], v[3]}, bf16x2v);
          if (EPI == 1) {
            const uint32_t b0 = __builtin_bit_cast(uint32_t, p0), b1 = __builtin_bit_cast(uint32_t, p1);
            const float r0_ = __uint_as_float(b0 << 16), r1_ = __uint_as_float(b0 & 0xffff0000u);
            const float r2_ = __uint_as_float(b1 << 16), r3_ = __uint_as_float(b1 & 0xffff0000u);
            p0 = __builtin_convertvector(f32x2v{gelu_tanh(r0_), gelu_tanh(r1_)}, bf16x2v);
            p1 = __builtin_convertvector(f32x2v{gelu_tanh(r2_), gelu_tanh(r3_)}, bf16x2v);
          }
          const uint32_t px = __builtin_bit_cast(uint32_t, p0), py = __builtin_bit_cast(uint32_t, p1);
          if (AMAX == 1 && mok && nok) {
            amax = max(amax, max((px & 0x7fffu) << 16, px & 0x7fff0000u));
            amax = max(amax, max((py & 0x7fffu) << 16, py & 0x7fff0000u));
          } else if (AMAX == 2 && mok && nok) {
            amax = max(amax, max(pos_key(px << 16), pos_key(px & 0xffff0000u)));
            amax = max(amax, max(pos_key(py << 16), pos_key(py & 0xffff0000u)));
          }
          *reinterpret_cast<uint2*>(stg + mrow * 64 + 16 * (q ^ wswz) + 8 * hh) = make_uint2(px, py);
        }
        // the 32 x 32 block back as 16 rows x 64 bytes per store
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const int rr = 16 * p + rb_row;
          const i32x4_t d =
              *reinterpret_cast<const i32x4_t*>(stg + rr * 64 + 16 * (rb_c ^ ((rr >> 1) & 3)));
          const int ml = wm * 128 + j * 32 + rr;
          const int n = n0 + wn * 64 + i * 32 + 8 * rb_c;
          const int off = (n < g.N && ml < rows) ? (int)((ml * g.ldo + n) * 2) : (int)0x80000000;
          __builtin_amdgcn_raw_buffer_store_b128(d, ro, off, 0, 0);
        }
      }
    }
    if (AMAX != 0) {
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) amax = max(amax, (uint32_t)__shfl_xor((int)amax, o));
      if (lane == 0) raise_max_word(g.amax_out, amax);
    }
#pragma unroll
    for (int i = 0; i < G_NI; ++i)
#pragma unroll
      for (int j = 0; j < G_NJ; ++j) acc[i][j] = f32x16_t{};
  }
}

template <typename Launch>
int dispatch_quant_dtype(int dtype, Launch&& launch) {
  switch (dtype) {
    case SRDIT_DTYPE_BF16: return launch((const uint16_t*)nullptr);
    case SRDIT_DTYPE_FP16: return launch((const _Float16*)nullptr);
    case SRDIT_DTYPE_FP32: return launch((const float*)nullptr);
    default:
      set_error("fp8 quantiser: dtype %d is not bf16 (0), fp16 (1) or fp32 (2)", dtype);
      return SRDIT_EUNSUPPORTED;
  }
}

int check_quant_args(const char* who, const void* x, int64_t M, int64_t K, int64_t ldx,
                     const void* xq, const float* scale) {
  SRDIT_REQUIRE(x && xq && scale, "%s: null pointer", who);
  SRDIT_REQUIRE(M > 0 && K > 0, "%s: M=%lld K=%lld must be positive", who, (long long)M,
                (long long)K);
  SRDIT_REQUIRE(K % 8 == 0 && ldx % 8 == 0 && ldx >= K,
                "%s: K=%lld and ldx=%lld must be multiples of 8 with ldx >= K", who,
                (long long)K, (long long)ldx);
  SRDIT_REQUIRE(aligned16(x) && aligned16(xq), "%s: x and xq must be 16-byte aligned", who);
  return SRDIT_OK;
}

}  // namespace
}  // namespace srdit

using namespace srdit;

extern "C" int srdit_fp8_quant_rowwise(const void* x, int64_t M, int64_t K, int64_t ldx,
                                       int dtype, void* xq, float* scale, void* stream) {
  if (int rc = check_quant_args("srdit_fp8_quant_rowwise", x, M, K, ldx, xq, scale)) return rc;
  SRDIT_REQUIRE(M < (int64_t(1) << 33), "srdit_fp8_quant_rowwise: M=%lld too large", (long long)M);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dispatch_quant_dtype(dtype, [&](auto tag) -> int {
    using T = std::remove_const_t<std::remove_pointer_t<decltype(tag)>>;
    const unsigned blocks = (unsigned)((M + 3) / 4);
    quant_rowwise_kernel<T><<<blocks, 256, 0, s>>>(static_cast<const T*>(x), M, K, ldx,
                                                   static_cast<uint8_t*>(xq), scale);
    SRDIT_LAUNCH_CHECK("quant_rowwise_kernel");
    return SRDIT_OK;
  });
}

extern "C" int srdit_fp8_quant_tensor(const void* x, int64_t M, int64_t K, int64_t ldx, int dtype,
                                      void* xq, float* scale, uint32_t* amax_ws, void* stream) {
  if (int rc = check_quant_args("srdit_fp8_quant_tensor", x, M, K, ldx, xq, scale)) return rc;
  SRDIT_REQUIRE(amax_ws, "srdit_fp8_quant_tensor: null amax workspace");
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dispatch_quant_dtype(dtype, [&](auto tag) -> int {
    using T = std::remove_const_t<std::remove_pointer_t<decltype(tag)>>;
    const int64_t rows4 = (M + 3) / 4;
    const unsigned blocks = (unsigned)(rows4 < 4096 ? rows4 : 4096);
    clear_u32_kernel<<<1, 1, 0, s>>>(amax_ws);
    SRDIT_LAUNCH_CHECK("clear_u32_kernel");
    amax_kernel<T><<<blocks, 256, 0, s>>>(static_cast<const T*>(x), M, K, ldx, amax_ws);
    SRDIT_LAUNCH_CHECK("amax_kernel");
    quant_tensor_kernel<T><<<blocks, 256, 0, s>>>(static_cast<const T*>(x), M, K, ldx,
                                                  static_cast<uint8_t*>(xq), scale, amax_ws);
    SRDIT_LAUNCH_CHECK("quant_tensor_kernel");
    return SRDIT_OK;
  });
}

namespace srdit {
namespace {
// Compute units of the current device (cached per device): the GEMM runs one
// persistent workgroup per CU.
int cu_count_of_current_device() {
  static std::mutex mu;
  static int cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (!cache[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

// Split-K of a GEMM's last, partial round of tiles.  With T tiles on G
// workgroups the persistent launch takes ceil(T / G) rounds of a whole tile's K
// stages even when the last round holds a few tiles (10800 x 3072 x 14336: 516
// tiles, two rounds and 4 tiles on 256 CUs).  Those tail = T mod G tiles can go
// to a second launch instead, each split over S workgroups along K.  Measured on
// MI355X, in K stages of a lightly loaded chip (about 1 us each): the last
// round costs nks stages unsplit, and a split tile about ceil(nks / S) + 5
// (launch, partial store, epilogue) + 4 S (the last arrival reads S partials of
// 256 KB back, latency-bound at one workgroup).  So only long K pays
// (10800 x 3072 x 14336: 475 -> 408 us; at K = 3072 the split is slower), and
// only a small tail: 208 workgroups storing and re-reading partials at once
// made a 104-tile tail slower than its unsplit round.
struct TailSplit {
  int tail = 0, split = 0;  // split == 0: one launch over every tile
};

TailSplit plan_tail_split(int64_t tiles, int64_t grid, int nks, int64_t max_units) {
  TailSplit p;
  const int64_t tail = tiles % grid;
  if (tiles < grid || tail == 0 || 8 * tail > grid) return p;
  double best = 0.75 * nks;  // split only when it saves a quarter of the round
  for (int S = 2; S <= nks && tail * S <= grid && tail * S <= max_units; ++S) {
    const double cost = (double)((nks + S - 1) / S) + 5.0 + 4.0 * S;
    if (cost < best) {
      best = cost;
      p.tail = (int)tail;
      p.split = S;
    }
  }
  return p;
}

// Split-K workspace: one arrival counter per tail tile (left 0 by every
// launch), then the partials, G_PART_BYTES per workgroup of the split launch.
constexpr int64_t WS_COUNTERS = 4096;

int fp8_gemm_launch(const void* a, const void* b, const float* sa, int64_t sa_rows, const float* sb,
                    int64_t sb_cols, const void* bias, void* out, int64_t M, int64_t N, int64_t K,
                    int64_t ldo, int epilogue, uint32_t* amax_out, void* stream, const char* who,
                    int64_t split_n = 0, int64_t split_stride = 0, bool bf16 = false,
                    void* workspace = nullptr, int64_t workspace_bytes = 0) {
  SRDIT_REQUIRE(a && b && sa && sb && out, "%s: null pointer", who);
  SRDIT_REQUIRE(M > 0 && N > 0 && K > 0, "%s: M, N, K must be positive", who);
  if (bf16) {  // bf16 operands: K elements of two bytes; the kernel counts bytes
    SRDIT_REQUIRE(K % 64 == 0 && sa_rows == 1 && sb_cols == 1 && !amax_out && !split_n,
                  "%s: bf16 operands need K %% 64 == 0 (K=%lld), no scales, amax or split", who,
                  (long long)K);
    K *= 2;
  }
  SRDIT_REQUIRE(K % 128 == 0, "%s: K=%lld must be a multiple of 128", who, (long long)K);
  SRDIT_REQUIRE(N % 16 == 0, "%s: N=%lld must be a multiple of 16", who, (long long)N);
  const int64_t width = split_n ? split_n : N;  // columns of one output block
  SRDIT_REQUIRE(ldo >= width && ldo % 8 == 0 && (255 * ldo + N) * 2 + 16 < (int64_t(1) << 31),
                "%s: ldo=%lld must be >= the output width, a multiple of 8, and keep 256 rows "
                "below 2^31 bytes", who, (long long)ldo);
  SRDIT_REQUIRE(split_n == 0 || (split_n % 256 == 0 && N % split_n == 0 && split_stride % 8 == 0 &&
                                 split_stride >= M * ldo),
                "%s: split_n=%lld must be a multiple of 256 dividing N, and split_stride=%lld a "
                "multiple of 8 of at least M*ldo", who, (long long)split_n, (long long)split_stride);
  SRDIT_REQUIRE(M * K < (int64_t(1) << 31) && N * K < (int64_t(1) << 31),
                "%s: M*K and N*K must be below 2^31 (M=%lld N=%lld K=%lld)", who, (long long)M,
                (long long)N, (long long)K);
  SRDIT_REQUIRE(sa_rows == 1 || sa_rows == M, "%s: sa_rows=%lld must be 1 or M", who,
                (long long)sa_rows);
  SRDIT_REQUIRE(sb_cols == 1 || sb_cols == N, "%s: sb_cols=%lld must be 1 or N", who,
                (long long)sb_cols);
  // per-row / per-column scales and the bias reach LDS by 16-byte DMAs
  SRDIT_REQUIRE(aligned16(a) && aligned16(b) && aligned16(out) && (!bias || aligned16(bias)) &&
                    (sa_rows == 1 || aligned16(sa)) && (sb_cols == 1 || aligned16(sb)),
                "%s: a, b, out, bias and per-row/per-column scales must be 16-byte aligned", who);
  // SRDIT_GEMM_MFMA selected the hand-written kernel when plain GEMMs went to a
  // library; every GEMM runs on it now, so the flag is accepted and ignored.
  epilogue &= ~SRDIT_GEMM_MFMA;
  const bool amax_pos = (epilogue & SRDIT_GEMM_AMAX_POS) != 0;
  epilogue &= ~SRDIT_GEMM_AMAX_POS;
  SRDIT_REQUIRE(epilogue == 0 || epilogue == 1, "%s: epilogue %d is not 0 (none) or 1 (gelu)", who,
                epilogue);
  SRDIT_REQUIRE(!amax_pos || (amax_out && epilogue == 0),
                "%s: SRDIT_GEMM_AMAX_POS needs amax_out and no GELU epilogue", who);
  GemmArgs g;
  g.a = static_cast<const uint8_t*>(a);
  g.b = static_cast<const uint8_t*>(b);
  g.sa = sa;
  g.sb = sb;
  g.bias = static_cast<const uint16_t*>(bias);
  g.out = static_cast<uint16_t*>(out);
  g.M = (int)M;
  g.N = (int)N;
  g.K = (int)K;
  g.ldo = ldo;
  g.sa_per_row = sa_rows == M && M > 1;
  g.sb_per_col = sb_cols == N && N > 1;
  g.tiles_m = (int)((M + GT - 1) / GT);
  g.tiles_n = (int)((N + GT - 1) / GT);
  g.amax_out = amax_out;
  g.split_n = split_n;
  g.split_stride = split_stride;
  const int64_t tiles = (int64_t)g.tiles_m * g.tiles_n;
  SRDIT_REQUIRE(tiles < (int64_t(1) << 31), "%s: too many tiles", who);
  SRDIT_REQUIRE(!workspace || (aligned16(workspace) && workspace_bytes >= 0),
                "%s: the workspace must be 16-byte aligned", who);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (amax_out) {
    clear_u32_kernel<<<1, 1, 0, s>>>(amax_out);
    SRDIT_LAUNCH_CHECK("clear_u32_kernel");
  }
  // one workgroup per CU, a multiple of 8 (one share per XCD), no more than the tiles need
  const int64_t cus = (cu_count_of_current_device() / 8) * 8;
  const int64_t need = (tiles + 7) / 8 * 8;
  unsigned grid = (unsigned)(cus >= 8 ? (need < cus ? need : cus) : 8);
  const int64_t max_units =
      workspace && workspace_bytes > WS_COUNTERS ? (workspace_bytes - WS_COUNTERS) / G_PART_BYTES : 0;
  const TailSplit ts = max_units >= 2 && !bf16
                           ? plan_tail_split(tiles, grid, g.K / G_FK, max_units)
                           : TailSplit{};
  auto launch = [&](const GemmArgs& ga, unsigned nwg, auto split_c) {
    constexpr bool SP = decltype(split_c)::value;
    if (bf16 && epilogue == 0) fp8_gemm_kernel<0, 0, 1><<<nwg, 512, 0, s>>>(ga);
    else if (bf16) fp8_gemm_kernel<1, 0, 1><<<nwg, 512, 0, s>>>(ga);
    else if (epilogue == 0 && !amax_out) fp8_gemm_kernel<0, 0, 0, SP><<<nwg, 512, 0, s>>>(ga);
    else if (epilogue == 0 && amax_pos) fp8_gemm_kernel<0, 2, 0, SP><<<nwg, 512, 0, s>>>(ga);
    else if (epilogue == 0) fp8_gemm_kernel<0, 1, 0, SP><<<nwg, 512, 0, s>>>(ga);
    else if (!amax_out) fp8_gemm_kernel<1, 0, 0, SP><<<nwg, 512, 0, s>>>(ga);
    else fp8_gemm_kernel<1, 1, 0, SP><<<nwg, 512, 0, s>>>(ga);
  };
  // the whole rounds (every tile when nothing is split)
  g.task_base = 0;
  g.n_tasks = (int)(tiles - ts.tail);
  g.split_k = 0;
  g.ws_part = nullptr;
  g.ws_cnt = nullptr;
  launch(g, grid, std::false_type{});
  SRDIT_LAUNCH_CHECK("fp8_gemm_kernel");
  if (ts.split) {  // the last round's tiles, split along K
    g.task_base = g.n_tasks;
    g.n_tasks = ts.tail;
    g.split_k = ts.split;
    g.ws_cnt = static_cast<uint32_t*>(workspace);
    g.ws_part = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + WS_COUNTERS);
    launch(g, (unsigned)(ts.tail * ts.split), std::true_type{});
    SRDIT_LAUNCH_CHECK("fp8_gemm_kernel (split tail)");
  }
  return SRDIT_OK;
}
}  // namespace

// The persistent GEMM on bf16 operands (contiguous rows of K elements), for
// srdit_bf16_linear's large grids: out = bf16(a w^T + bias) [then GELU].
int bf16_gemm_persistent(const void* a, const void* w, const void* bias, void* out, int64_t M,
                         int64_t N, int64_t K, int64_t ldo, int gelu, void* stream,
                         const char* who) {
  const float* unit = static_cast<const float*>(a);  // scales are not read with bf16 operands
  return fp8_gemm_launch(a, w, unit, 1, unit, 1, bias, out, M, N, K, ldo, gelu ? 1 : 0, nullptr,
                         stream, who, 0, 0, true);
}

}  // namespace srdit

extern "C" int srdit_fp8_gemm(const void* a, const void* b, const float* sa, int64_t sa_rows,
                              const float* sb, int64_t sb_cols, const void* bias, void* out,
                              int64_t M, int64_t N, int64_t K, int64_t ldo, void* stream) {
  return fp8_gemm_launch(a, b, sa, sa_rows, sb, sb_cols, bias, out, M, N, K, ldo, 0, nullptr,
                         stream, "srdit_fp8_gemm");
}

extern "C" int srdit_fp8_gemm_ex(const void* a, const void* b, const float* sa, int64_t sa_rows,
                                 const float* sb, int64_t sb_cols, const void* bias, void* out,
                                 int64_t M, int64_t N, int64_t K, int64_t ldo, int epilogue,
                                 uint32_t* amax_out, void* stream) {
  return fp8_gemm_launch(a, b, sa, sa_rows, sb, sb_cols, bias, out, M, N, K, ldo, epilogue,
                         amax_out, stream, "srdit_fp8_gemm_ex");
}

extern "C" int srdit_fp8_gemm_split(const void* a, const void* b, const float* sa, int64_t sa_rows,
                                    const float* sb, int64_t sb_cols, const void* bias, void* out,
                                    int64_t M, int64_t N, int64_t K, int64_t ldo, int64_t split_n,
                                    int64_t split_stride, void* stream) {
  SRDIT_REQUIRE(split_n > 0, "srdit_fp8_gemm_split: split_n=%lld must be positive",
                (long long)split_n);
  return fp8_gemm_launch(a, b, sa, sa_rows, sb, sb_cols, bias, out, M, N, K, ldo, 0, nullptr,
                         stream, "srdit_fp8_gemm_split", split_n, split_stride);
}

extern "C" int srdit_fp8_gemm_ws(const void* a, const void* b, const float* sa, int64_t sa_rows,
                                 const float* sb, int64_t sb_cols, const void* bias, void* out,
                                 int64_t M, int64_t N, int64_t K, int64_t ldo, int epilogue,
                                 uint32_t* amax_out, int64_t split_n, int64_t split_stride,
                                 void* workspace, int64_t workspace_bytes, void* stream) {
  SRDIT_REQUIRE(split_n >= 0, "srdit_fp8_gemm_ws: split_n=%lld must not be negative",
                (long long)split_n);
  return fp8_gemm_launch(a, b, sa, sa_rows, sb, sb_cols, bias, out, M, N, K, ldo, epilogue,
                         amax_out, stream, "srdit_fp8_gemm_ws", split_n, split_stride, false,
                         workspace, workspace_bytes);
}

extern "C" int srdit_fp8_quant_apply(const void* x, int64_t M, int64_t K, int64_t ldx, int dtype,
                                     void* xq, float* scale, const uint32_t* amax_ws, void* stream) {
  if (int rc = check_quant_args("srdit_fp8_quant_apply", x, M, K, ldx, xq, scale)) return rc;
  SRDIT_REQUIRE(amax_ws, "srdit_fp8_quant_apply: null amax word");
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dispatch_quant_dtype(dtype, [&](auto tag) -> int {
    using T = std::remove_const_t<std::remove_pointer_t<decltype(tag)>>;
    const int64_t rows4 = (M + 3) / 4;
    const unsigned blocks = (unsigned)(rows4 < 4096 ? rows4 : 4096);
    quant_tensor_kernel<T><<<blocks, 256, 0, s>>>(static_cast<const T*>(x), M, K, ldx,
                                                  static_cast<uint8_t*>(xq), scale, amax_ws);
    SRDIT_LAUNCH_CHECK("quant_tensor_kernel");
    return SRDIT_OK;
  });
}

// The GELU table: one static 128 KB array per device, addressed through
// hipGetSymbolAddress (taken once per device).  Every call rewrites it before
// its passes read it, in stream order; calls on other streams of the device
// write the same values, so overlapping calls read correct entries.
static __device__ __align__(256) uint16_t gelu_lut_table[srdit::LUT_N];

namespace srdit {
namespace {
std::mutex g_lut_mu;
void* g_lut_dev[64] = {};

int gelu_lut_of_current_device(void** out, const char* who) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  SRDIT_REQUIRE(e == hipSuccess, "%s: hipGetDevice failed: %s", who, hipGetErrorString(e));
  SRDIT_REQUIRE(dev >= 0 && dev < 64, "%s: device %d out of range", who, dev);
  std::lock_guard<std::mutex> lock(g_lut_mu);
  if (!g_lut_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(gelu_lut_table));
    if (e != hipSuccess || !p) {
      set_error("%s: hipGetSymbolAddress(gelu_lut_table) failed on device %d: %s", who, dev,
                hipGetErrorString(e));
      return SRDIT_EHIP;
    }
    g_lut_dev[dev] = p;
  }
  *out = g_lut_dev[dev];
  return SRDIT_OK;
}

int device_cu_count() { return cu_count_of_current_device(); }
}  // namespace
}  // namespace srdit

namespace srdit {
namespace {
int quant_tensor_gelu(const void* x, int64_t M, int64_t K, int64_t ldx, void* h, int64_t ldh,
                      void* xq, float* scale, uint32_t* amax_ws, const uint32_t* xmax_pos,
                      void* stream) {
  if (int rc = check_quant_args("srdit_fp8_quant_tensor_gelu", x, M, K, ldx, xq, scale)) return rc;
  SRDIT_REQUIRE(amax_ws, "srdit_fp8_quant_tensor_gelu: null amax workspace");
  SRDIT_REQUIRE(!h || (aligned16(h) && ldh >= K && ldh % 8 == 0 && h != x),
                "srdit_fp8_quant_tensor_gelu: h must be null, or 16-byte aligned with ldh >= K, "
                "ldh %% 8 == 0, and not x");
  void* lut = nullptr;
  if (int rc = gelu_lut_of_current_device(&lut, "srdit_fp8_quant_tensor_gelu")) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t rows16 = (M + LUT_WAVES - 1) / LUT_WAVES;
  const int cus = device_cu_count();
  const unsigned blocks = (unsigned)(rows16 < cus ? rows16 : cus);  // one workgroup per CU
  gelu_lut_build_kernel<<<LUT_N / 512, 256, 0, s>>>(static_cast<uint16_t*>(lut), amax_ws);
  SRDIT_LAUNCH_CHECK("gelu_lut_build_kernel");
  gelu_lut_amax_kernel<<<blocks, 64 * LUT_WAVES, 0, s>>>(
      static_cast<const uint16_t*>(x), M, K, ldx, static_cast<uint16_t*>(h), ldh,
      static_cast<const uint16_t*>(lut), amax_ws, h ? nullptr : xmax_pos);
  SRDIT_LAUNCH_CHECK("gelu_lut_amax_kernel");
  gelu_code_quant_kernel<<<blocks, 64 * LUT_WAVES, 0, s>>>(
      static_cast<const uint16_t*>(x), M, K, ldx, static_cast<const uint16_t*>(lut),
      static_cast<uint8_t*>(xq), scale, amax_ws);
  SRDIT_LAUNCH_CHECK("gelu_code_quant_kernel");
  return SRDIT_OK;
}
}  // namespace
}  // namespace srdit

extern "C" int srdit_fp8_quant_tensor_gelu(const void* x, int64_t M, int64_t K, int64_t ldx,
                                           void* h, int64_t ldh, void* xq, float* scale,
                                           uint32_t* amax_ws, void* stream) {
  return quant_tensor_gelu(x, M, K, ldx, h, ldh, xq, scale, amax_ws, nullptr, stream);
}

extern "C" int srdit_fp8_quant_tensor_gelu_ex(const void* x, int64_t M, int64_t K, int64_t ldx,
                                              void* h, int64_t ldh, void* xq, float* scale,
                                              uint32_t* amax_ws, const uint32_t* xmax_pos,
                                              void* stream) {
  return quant_tensor_gelu(x, M, K, ldx, h, ldh, xq, scale, amax_ws, xmax_pos, stream);
}

// ---------------------------------------------------------------------------
// The per-tensor fp8 Linear as one call that allocates nothing.
//
// `scratch` holds what srdit_fp8_quant_tensor + srdit_fp8_gemm_ex keep in
// caller-provided buffers: the amax word (bytes 0-3), the activation scale
// (bytes 4-7) and, from byte 256, the e4m3 codes of the activation (at most
// SRDIT_LINEAR_SCRATCH_CODES bytes, so M*K is limited to that).  Each device
// holds its own copy of the array from the library's first use on it until
// the process ends.  Host code never passes the array's name to a kernel: it
// is a host-side stand-in for the symbol.  The device address comes from
// hipGetSymbolAddress, taken once per device on the first call with that
// device current.  Every call on one device shares that device's array:
// calls that overlap on one device (two streams, or two host threads) race.
// ---------------------------------------------------------------------------
static __device__ __align__(256) uint8_t scratch[256 + SRDIT_LINEAR_SCRATCH_CODES];

namespace srdit {
namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxScratchDevices] = {};

int scratch_of_current_device(void** out, const char* who) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  SRDIT_REQUIRE(e == hipSuccess, "%s: hipGetDevice failed: %s", who, hipGetErrorString(e));
  SRDIT_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, "%s: device %d out of range", who, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error("%s: hipGetSymbolAddress(scratch) failed on device %d: %s", who, dev,
                hipGetErrorString(e));
      return SRDIT_EHIP;
    }
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return SRDIT_OK;
}
}  // namespace
}  // namespace srdit

extern "C" int srdit_fp8_linear_tensor_static(const void* x, int64_t M, int64_t K, int64_t ldx,
                                              int dtype, const void* w, const float* w_scale,
                                              int64_t w_scale_cols, const void* bias, void* out,
                                              int64_t N, int64_t ldo, void* stream) {
  const char* who = "srdit_fp8_linear_tensor_static";
  SRDIT_REQUIRE(M > 0 && K > 0 && M * K <= SRDIT_LINEAR_SCRATCH_CODES,
                "%s: M*K = %lld exceeds the static scratch (%lld e4m3 codes); use "
                "srdit_fp8_quant_tensor + srdit_fp8_gemm_ex with caller buffers", who,
                (long long)(M * K), (long long)SRDIT_LINEAR_SCRATCH_CODES);
  void* base = nullptr;
  if (int rc = scratch_of_current_device(&base, who)) return rc;
  uint8_t* sb = static_cast<uint8_t*>(base);
  uint32_t* amax = reinterpret_cast<uint32_t*>(sb);
  float* scale = reinterpret_cast<float*>(sb + 4);
  uint8_t* codes = sb + 256;
  if (int rc = check_quant_args(who, x, M, K, ldx, codes, scale)) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = dispatch_quant_dtype(dtype, [&](auto tag) -> int {
    using T = std::remove_const_t<std::remove_pointer_t<decltype(tag)>>;
    const int64_t rows4 = (M + 3) / 4;
    const unsigned blocks = (unsigned)(rows4 < 4096 ? rows4 : 4096);
    clear_u32_kernel<<<1, 1, 0, s>>>(amax);
    SRDIT_LAUNCH_CHECK("clear_u32_kernel");
    amax_kernel<T><<<blocks, 256, 0, s>>>(static_cast<const T*>(x), M, K, ldx, amax);
    SRDIT_LAUNCH_CHECK("amax_kernel");
    quant_tensor_kernel<T><<<blocks, 256, 0, s>>>(static_cast<const T*>(x), M, K, ldx, codes,
                                                  scale, amax);
    SRDIT_LAUNCH_CHECK("quant_tensor_kernel");
    return SRDIT_OK;
  });
  if (rc) return rc;
  return fp8_gemm_launch(codes, w, scale, 1, w_scale, w_scale_cols, bias, out, M, N, K, ldo,
                         SRDIT_GEMM_MFMA, nullptr, stream, who);
}
