// Fused row kernels of the refiner block for gfx950: one pass over HBM each.
//
//   ln_modulate    out = bf16( f32(bf16(LayerNorm(x) [* w + b])) * (1 + scale) + shift )
//                  and, optionally, the max |out| (float bits) into an amax word
//                  for a per-tensor fp8 quantiser of `out`
//   residual_gate  out = bf16( f32(x) + f32(y) * gate )
//   residual_ln_modulate
//                  x_out = residual_gate(x, y, gate), then ln_modulate(x_out)
//                  from the same registers: one pass for the gated residual
//                  and the LayerNorm that reads the new residual stream
//   rmsnorm_rope   out = RoPE( bf16( f32(bf16(x * rsqrt(mean(x^2) + eps))) * f32(w) ) )
//
// They restate, op for op, the elementwise chains of the reference block
// (video_refiner/wan/modules/sr_dit/models.py): WanLayerNorm (:443-503) and the
// adaLN modulation of WanAttentionBlock.forward (:1308, :1258); the gated
// residuals (:1344, :1260); WanRMSNorm (:424-440) on q and k followed by
// rope_apply (:173-214).  Each fp32 operation rounds where torch's separate
// kernels round: this file is compiled with -ffp-contract=off, so no multiply
// and add are contracted into an fma.  The reductions (mean, variance, mean of
// squares) sum in a different order than torch's.
//
// One wavefront per row at a time; a row is read from HBM once.  K % 8 == 0,
// rows 16-byte aligned.
#include "common.h"

namespace srdit {
namespace {

__device__ __forceinline__ void unpack_bf16x8(const uint4 v, float f[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));

// Round to bf16 (nearest even) and back: the value torch holds after .to(bf16).
__device__ __forceinline__ float bf16_round(float x) {
  const bf16x2v b = __builtin_convertvector(f32x2v{x, 0.f}, bf16x2v);
  return __uint_as_float(static_cast<uint32_t>(__builtin_bit_cast(uint32_t, b) & 0xffffu) << 16);
}

__device__ __forceinline__ uint4 pack_bf16x8(const float f[8]) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2v{f[2 * i], f[2 * i + 1]}, bf16x2v));
  return make_uint4(w[0], w[1], w[2], w[3]);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ __forceinline__ uint32_t wave_umax(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o));
  return v;
}

__global__ void clear_word_kernel(uint32_t* p) { *p = 0u; }

// LayerNorm over each row of x [M, K] (bf16, row stride ldx), eps, optional
// affine (w, b bf16 [K]); then, with MOD, the adaLN modulation (scale, shift
// fp32 [K]).  Output bf16 [M, K] with row stride ldo.
//
// Each wavefront walks rows grid-stride.  With CACHED (K <= 4096) a lane
// keeps its <= 8 chunks of the row in registers, so the row is read once;
// otherwise the mean, variance and output passes re-read it (L1/L2 hits).
// Per lane the chunks are summed in the order c = lane, lane + 64, ..., as the
// output pass visits them.  The amax is reduced per workgroup, then raises
// the word once per workgroup (raise_max_word).  VEC: scale and shift are
// 16-byte aligned and read as float4.
// RES (CACHED only): the row is first the gated residual x + y * gate (16-byte
// aligned fp32 gate [K]), computed as residual_gate_kernel computes it, stored
// to xo (row stride ldxo) and kept in registers for the LayerNorm.
struct ResidualIn {
  const uint16_t* y;
  int64_t ldy;
  const float* gate;
  uint16_t* xo;
  int64_t ldxo;
};

template <bool AFFINE, bool MOD, bool AMAX, bool CACHED, bool VEC, bool RES = false>
__global__ __launch_bounds__(256) void ln_modulate_kernel(
    const uint16_t* __restrict__ x, int64_t M, int K, int64_t ldx, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ b, const float* __restrict__ scale, const float* __restrict__ shift,
    float eps, uint16_t* __restrict__ out, int64_t ldo, uint32_t* __restrict__ amax_ws,
    ResidualIn res = ResidualIn{}) {
  static_assert(!RES || CACHED, "the residual prologue keeps the row in registers");
  constexpr int CPL = 8;  // cached chunks per lane
  const int lane = threadIdx.x & 63;
  const int nc = K >> 3;
  uint32_t am = 0;
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); row < M;
       row += static_cast<int64_t>(gridDim.x) * 4) {
    const uint4* xr = reinterpret_cast<const uint4*>(x + row * ldx);
    uint4 rb[CACHED ? CPL : 1];
    if constexpr (RES) {
      const uint4* yr = reinterpret_cast<const uint4*>(res.y + row * res.ldy);
      uint4 yb[CPL];
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = lane + 64 * i;
        rb[i] = c < nc ? xr[c] : make_uint4(0u, 0u, 0u, 0u);
        yb[i] = c < nc ? yr[c] : make_uint4(0u, 0u, 0u, 0u);
      }
      uint4* xor_ = reinterpret_cast<uint4*>(res.xo + row * res.ldxo);
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = lane + 64 * i;
        if (c < nc) {
          float xf[8], yf[8], o[8];
          unpack_bf16x8(rb[i], xf);
          unpack_bf16x8(yb[i], yf);
          const float4 g0 = reinterpret_cast<const float4*>(res.gate)[2 * c];
          const float4 g1 = reinterpret_cast<const float4*>(res.gate)[2 * c + 1];
          const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = __fadd_rn(xf[e], __fmul_rn(yf[e], g[e]));
          rb[i] = pack_bf16x8(o);
          xor_[c] = rb[i];
        }
      }
    } else if (CACHED) {
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = lane + 64 * i;
        rb[i] = c < nc ? xr[c] : make_uint4(0u, 0u, 0u, 0u);
      }
    }
    auto chunk = [&](int i, int c) -> uint4 { return CACHED ? rb[i] : xr[c]; };
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < (CACHED ? CPL : 1); ++i) {
      for (int c = lane + 64 * i; c < nc && (CACHED || i == 0); c += (CACHED ? nc : 64)) {
        float f[8];
        unpack_bf16x8(chunk(i, c), f);
#pragma unroll
        for (int e = 0; e < 8; ++e) s += f[e];
      }
    }
    const float mean = wave_sum(s) / static_cast<float>(K);
    float v = 0.f;
#pragma unroll
    for (int i = 0; i < (CACHED ? CPL : 1); ++i) {
      for (int c = lane + 64 * i; c < nc && (CACHED || i == 0); c += (CACHED ? nc : 64)) {
        float f[8];
        unpack_bf16x8(chunk(i, c), f);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = f[e] - mean;
          v += d * d;
        }
      }
    }
    const float rstd = rsqrtf(wave_sum(v) / static_cast<float>(K) + eps);
    uint4* orow = reinterpret_cast<uint4*>(out + row * ldo);
#pragma unroll
    for (int i = 0; i < (CACHED ? CPL : 1); ++i) {
      for (int c = lane + 64 * i; c < nc && (CACHED || i == 0); c += (CACHED ? nc : 64)) {
        float f[8];
        unpack_bf16x8(chunk(i, c), f);
        float wv[8], bv[8], sv[8], hv[8];
        if (AFFINE) {
          unpack_bf16x8(reinterpret_cast<const uint4*>(w)[c], wv);
          unpack_bf16x8(reinterpret_cast<const uint4*>(b)[c], bv);
        }
        if (MOD) {
          if (VEC) {
            const float4* s4 = reinterpret_cast<const float4*>(scale) + 2 * c;
            const float4* h4 = reinterpret_cast<const float4*>(shift) + 2 * c;
            const float4 s0 = s4[0], s1 = s4[1], h0 = h4[0], h1 = h4[1];
            sv[0] = s0.x; sv[1] = s0.y; sv[2] = s0.z; sv[3] = s0.w;
            sv[4] = s1.x; sv[5] = s1.y; sv[6] = s1.z; sv[7] = s1.w;
            hv[0] = h0.x; hv[1] = h0.y; hv[2] = h0.z; hv[3] = h0.w;
            hv[4] = h1.x; hv[5] = h1.y; hv[6] = h1.z; hv[7] = h1.w;
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              sv[e] = scale[8 * c + e];
              hv[e] = shift[8 * c + e];
            }
          }
        }
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float y = __fmul_rn(f[e] - mean, rstd);
          if (AFFINE) y = __fadd_rn(__fmul_rn(y, wv[e]), bv[e]);
          y = bf16_round(y);  // LayerNorm(...).type_as(x)
          if (MOD) y = __fadd_rn(__fmul_rn(y, __fadd_rn(1.0f, sv[e])), hv[e]);
          o[e] = y;
        }
        const uint4 pk = pack_bf16x8(o);
        orow[c] = pk;
        if (AMAX) {
          const uint32_t ww[4] = {pk.x, pk.y, pk.z, pk.w};
#pragma unroll
          for (int e = 0; e < 4; ++e)
            am = max(am, max((ww[e] & 0x7fffu) << 16, (ww[e] & 0x7fff0000u)));
        }
      }
    }
  }
  if (AMAX) {
    __shared__ uint32_t wmax[4];
    am = wave_umax(am);
    if (lane == 0) wmax[threadIdx.x >> 6] = am;
    __syncthreads();
    if (threadIdx.x == 0)
      raise_max_word(amax_ws, max(max(wmax[0], wmax[1]), max(wmax[2], wmax[3])));
  }
}

// out = bf16(f32(x) + f32(y) * gate[k]); out may alias x.
__global__ __launch_bounds__(256) void residual_gate_kernel(const uint16_t* x, int64_t M, int K,
                                                            int64_t ldx, const uint16_t* __restrict__ y,
                                                            int64_t ldy, const float* __restrict__ gate,
                                                            uint16_t* out, int64_t ldo) {
  const int nc = K >> 3;
  const int64_t total = M * nc;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t row = idx / nc;
    const int c = static_cast<int>(idx - row * nc);
    float xf[8], yf[8], o[8];
    unpack_bf16x8(reinterpret_cast<const uint4*>(x + row * ldx)[c], xf);
    unpack_bf16x8(reinterpret_cast<const uint4*>(y + row * ldy)[c], yf);
    const float4 g0 = reinterpret_cast<const float4*>(gate)[2 * c];
    const float4 g1 = reinterpret_cast<const float4*>(gate)[2 * c + 1];
    const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = __fadd_rn(xf[i], __fmul_rn(yf[i], g[i]));
    reinterpret_cast<uint4*>(out + row * ldo)[c] = pack_bf16x8(o);
  }
}

// RMSNorm over the whole row (K = heads * head_dim), weight w (bf16 [K]), then
// (ROPE) RoPE on each head: pair j of a head rotated by (cos, sin) = cs[row][j % (head_dim/2)].
// One wavefront per row.  CACHED (K <= 4096): the row stays in registers
// between the sum of squares and the output pass, its loads all issued first.
// A chunk of eight values holds pairs 4c .. 4c+3, which (head_dim a multiple
// of 8) sit at 4c mod (head_dim/2) .. +3 in the table: VEC reads them as two
// 16-byte loads.  Each lane sums its squares in chunk order either way.
template <bool ROPE, bool CACHED, bool VEC>
__global__ __launch_bounds__(256) void rmsnorm_rope_kernel(const uint16_t* __restrict__ x, int64_t M,
                                                           int K, int64_t ldx,
                                                           const uint16_t* __restrict__ w, float eps,
                                                           const float2* __restrict__ cs, int half_d,
                                                           uint16_t* __restrict__ out) {
  constexpr int CPL = 8;  // cached chunks per lane
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const uint4* xr = reinterpret_cast<const uint4*>(x + row * ldx);
  const int nc = K >> 3;
  uint4 rb[CACHED ? CPL : 1];
  if (CACHED) {
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = lane + 64 * i;
      rb[i] = c < nc ? xr[c] : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  auto chunk = [&](int i, int c) -> uint4 { return CACHED ? rb[i] : xr[c]; };
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < (CACHED ? CPL : 1); ++i) {
    for (int c = lane + 64 * i; c < nc && (CACHED || i == 0); c += (CACHED ? nc : 64)) {
      float f[8];
      unpack_bf16x8(chunk(i, c), f);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += __fmul_rn(f[e], f[e]);
    }
  }
  const float r = rsqrtf(__fadd_rn(wave_sum(ss) / static_cast<float>(K), eps));
  const float2* csr = cs + row * half_d;
  uint4* orow = reinterpret_cast<uint4*>(out + row * K);
#pragma unroll
  for (int i = 0; i < (CACHED ? CPL : 1); ++i) {
    for (int c = lane + 64 * i; c < nc && (CACHED || i == 0); c += (CACHED ? nc : 64)) {
      float f[8], wv[8], o[8];
      unpack_bf16x8(chunk(i, c), f);
      unpack_bf16x8(reinterpret_cast<const uint4*>(w)[c], wv);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = bf16_round(__fmul_rn(bf16_round(__fmul_rn(f[e], r)), wv[e]));
      if (ROPE) {
        const int jb = (4 * c) % half_d;  // first pair of the chunk within its head
        float2 t[4];
        if (VEC) {
          const float4* p4 = reinterpret_cast<const float4*>(csr + jb);
          const float4 a = p4[0], b = p4[1];
          t[0] = make_float2(a.x, a.y); t[1] = make_float2(a.z, a.w);
          t[2] = make_float2(b.x, b.y); t[3] = make_float2(b.z, b.w);
        } else {
#pragma unroll
          for (int p = 0; p < 4; ++p) t[p] = csr[jb + p];
        }
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const float a = f[2 * p], bb = f[2 * p + 1];
          o[2 * p] = __fsub_rn(__fmul_rn(a, t[p].x), __fmul_rn(bb, t[p].y));
          o[2 * p + 1] = __fadd_rn(__fmul_rn(a, t[p].y), __fmul_rn(bb, t[p].x));
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = f[e];
      }
      orow[c] = pack_bf16x8(o);
    }
  }
}

int check_rows(const char* who, const void* x, int64_t M, int K, int64_t ldx, const void* out,
               int64_t ldo) {
  SRDIT_REQUIRE(x && out, "%s: null pointer", who);
  SRDIT_REQUIRE(M > 0 && K > 0 && K % 8 == 0 && K <= (1 << 20),
                "%s: M=%lld K=%d (K must be a positive multiple of 8)", who, (long long)M, K);
  SRDIT_REQUIRE(ldx >= K && ldx % 8 == 0 && ldo >= K && ldo % 8 == 0,
                "%s: row strides ldx=%lld ldo=%lld must be >= K and multiples of 8", who,
                (long long)ldx, (long long)ldo);
  SRDIT_REQUIRE(aligned16(x) && aligned16(out), "%s: x and out must be 16-byte aligned", who);
  return SRDIT_OK;
}

}  // namespace
}  // namespace srdit

using namespace srdit;

namespace srdit {
namespace {

// The LayerNorm launch shared by srdit_ln_modulate and, with `res`, the fused
// residual of srdit_residual_ln_modulate (which only passes res for K <= 4096).
int ln_modulate_launch(const char* who, const void* x, int64_t M, int K, int64_t ldx,
                       const void* ln_w, const void* ln_b, const float* scale, const float* shift,
                       float eps, void* out, int64_t ldo, uint32_t* amax_ws, hipStream_t s,
                       const ResidualIn* res) {
  if (int rc = check_rows(who, x, M, K, ldx, out, ldo)) return rc;
  SRDIT_REQUIRE((ln_w == nullptr) == (ln_b == nullptr), "%s: give both affine tensors or neither",
                who);
  SRDIT_REQUIRE((scale == nullptr) == (shift == nullptr),
                "%s: give both modulation tensors or neither", who);
  SRDIT_REQUIRE((!ln_w || (aligned16(ln_w) && aligned16(ln_b))) &&
                    (!scale || ((reinterpret_cast<uintptr_t>(scale) & 3) == 0 &&
                                (reinterpret_cast<uintptr_t>(shift) & 3) == 0)),
                "%s: misaligned affine or modulation tensor", who);
  if (amax_ws) {
    clear_word_kernel<<<1, 1, 0, s>>>(amax_ws);
    SRDIT_LAUNCH_CHECK("clear_word_kernel");
  }
  // Grid-stride over rows: at most 2048 workgroups of 4 row-wavefronts.
  const int64_t want = (M + 3) / 4;
  const unsigned blocks = static_cast<unsigned>(want < 2048 ? want : 2048);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint16_t* wp = static_cast<const uint16_t*>(ln_w);
  const uint16_t* bp = static_cast<const uint16_t*>(ln_b);
  uint16_t* op = static_cast<uint16_t*>(out);
  const bool cached = K <= 4096;
  const bool vec = scale != nullptr && aligned16(scale) && aligned16(shift);
  const ResidualIn r = res ? *res : ResidualIn{};
#define SRDIT_LN_LAUNCH2(A, MO, AM, C, V, R)                                                   \
  ln_modulate_kernel<A, MO, AM, C, V, R><<<blocks, 256, 0, s>>>(xp, M, K, ldx, wp, bp, scale,  \
                                                                shift, eps, op, ldo, amax_ws, r)
#define SRDIT_LN_LAUNCH(A, MO, AM)                                          \
  do {                                                                       \
    if (res && vec) SRDIT_LN_LAUNCH2(A, MO, AM, true, true, true);           \
    else if (res) SRDIT_LN_LAUNCH2(A, MO, AM, true, false, true);            \
    else if (cached && vec) SRDIT_LN_LAUNCH2(A, MO, AM, true, true, false);  \
    else if (cached) SRDIT_LN_LAUNCH2(A, MO, AM, true, false, false);        \
    else SRDIT_LN_LAUNCH2(A, MO, AM, false, false, false);                   \
  } while (0)
  const bool af = ln_w != nullptr, mo = scale != nullptr, am = amax_ws != nullptr;
  if (af && mo && am) SRDIT_LN_LAUNCH(true, true, true);
  else if (af && mo) SRDIT_LN_LAUNCH(true, true, false);
  else if (af && am) SRDIT_LN_LAUNCH(true, false, true);
  else if (af) SRDIT_LN_LAUNCH(true, false, false);
  else if (mo && am) SRDIT_LN_LAUNCH(false, true, true);
  else if (mo) SRDIT_LN_LAUNCH(false, true, false);
  else if (am) SRDIT_LN_LAUNCH(false, false, true);
  else SRDIT_LN_LAUNCH(false, false, false);
#undef SRDIT_LN_LAUNCH
#undef SRDIT_LN_LAUNCH2
  SRDIT_LAUNCH_CHECK("ln_modulate_kernel");
  return SRDIT_OK;
}

}  // namespace
}  // namespace srdit

extern "C" int srdit_ln_modulate(const void* x, int64_t M, int K, int64_t ldx, const void* ln_w,
                                 const void* ln_b, const float* scale, const float* shift, float eps,
                                 void* out, int64_t ldo, uint32_t* amax_ws, void* stream) {
  return ln_modulate_launch("srdit_ln_modulate", x, M, K, ldx, ln_w, ln_b, scale, shift, eps, out,
                            ldo, amax_ws, static_cast<hipStream_t>(stream), nullptr);
}

extern "C" int srdit_residual_ln_modulate(const void* x, const void* y, const float* gate,
                                          int64_t M, int K, int64_t ldx, int64_t ldy,
                                          void* x_out, int64_t ldxo, const void* ln_w,
                                          const void* ln_b, const float* scale,
                                          const float* shift, float eps, void* out, int64_t ldo,
                                          uint32_t* amax_ws, void* stream) {
  const char* who = "srdit_residual_ln_modulate";
  if (int rc = check_rows(who, x, M, K, ldx, x_out, ldxo)) return rc;
  SRDIT_REQUIRE(y && gate && aligned16(y) && aligned16(gate) && ldy >= K && ldy % 8 == 0,
                "%s: y / gate missing or misaligned, or bad ldy", who);
  SRDIT_REQUIRE(x_out != x && x_out != out && out != x && out != y,
                "%s: x_out and out must be buffers of their own", who);
  if (K > 4096) {  // the row does not fit the registers: the two kernels one after the other
    if (int rc = srdit_residual_gate(x, y, gate, M, K, ldx, ldy, x_out, ldxo, stream)) return rc;
    return srdit_ln_modulate(x_out, M, K, ldxo, ln_w, ln_b, scale, shift, eps, out, ldo, amax_ws,
                             stream);
  }
  const ResidualIn res{static_cast<const uint16_t*>(y), ldy, gate, static_cast<uint16_t*>(x_out),
                       ldxo};
  return ln_modulate_launch(who, x, M, K, ldx, ln_w, ln_b, scale, shift, eps, out, ldo, amax_ws,
                            static_cast<hipStream_t>(stream), &res);
}

extern "C" int srdit_residual_gate(const void* x, const void* y, const float* gate, int64_t M, int K,
                                   int64_t ldx, int64_t ldy, void* out, int64_t ldo, void* stream) {
  if (int rc = check_rows("srdit_residual_gate", x, M, K, ldx, out, ldo)) return rc;
  SRDIT_REQUIRE(y && gate && aligned16(y) && aligned16(gate) && ldy >= K && ldy % 8 == 0,
                "srdit_residual_gate: y / gate missing or misaligned, or bad ldy");
  const int64_t total = M * (K / 8);
  const int64_t want = (total + 255) / 256;
  const unsigned blocks = static_cast<unsigned>(want < 65536 ? want : 65536);
  residual_gate_kernel<<<blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(x), M, K, ldx, static_cast<const uint16_t*>(y), ldy, gate,
      static_cast<uint16_t*>(out), ldo);
  SRDIT_LAUNCH_CHECK("residual_gate_kernel");
  return SRDIT_OK;
}

extern "C" int srdit_rmsnorm_rope(const void* x, int64_t M, int K, int64_t ldx, const void* w,
                                  float eps, const float* rope_cs, int head_dim, void* out,
                                  void* stream) {
  if (int rc = check_rows("srdit_rmsnorm_rope", x, M, K, ldx, out, K)) return rc;
  SRDIT_REQUIRE(w && aligned16(w) && (reinterpret_cast<uintptr_t>(rope_cs) & 7) == 0,
                "srdit_rmsnorm_rope: weight missing or weight / rope table misaligned");
  SRDIT_REQUIRE(head_dim > 0 && head_dim % 8 == 0 && K % head_dim == 0,
                "srdit_rmsnorm_rope: head_dim %d must be a multiple of 8 dividing K=%d", head_dim, K);
  const unsigned blocks = static_cast<unsigned>((M + 3) / 4);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool cached = K <= 4096, vec = rope_cs != nullptr && aligned16(rope_cs);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint16_t* wp = static_cast<const uint16_t*>(w);
  const float2* cp = reinterpret_cast<const float2*>(rope_cs);
  uint16_t* op = static_cast<uint16_t*>(out);
  const int hd = head_dim / 2;
  if (rope_cs && cached && vec)
    rmsnorm_rope_kernel<true, true, true><<<blocks, 256, 0, s>>>(xp, M, K, ldx, wp, eps, cp, hd, op);
  else if (rope_cs && cached)
    rmsnorm_rope_kernel<true, true, false><<<blocks, 256, 0, s>>>(xp, M, K, ldx, wp, eps, cp, hd, op);
  else if (rope_cs)
    rmsnorm_rope_kernel<true, false, false><<<blocks, 256, 0, s>>>(xp, M, K, ldx, wp, eps, cp, hd, op);
  else if (cached)
    rmsnorm_rope_kernel<false, true, false><<<blocks, 256, 0, s>>>(xp, M, K, ldx, wp, eps, nullptr, hd, op);
  else
    rmsnorm_rope_kernel<false, false, false><<<blocks, 256, 0, s>>>(xp, M, K, ldx, wp, eps, nullptr, hd, op);
  SRDIT_LAUNCH_CHECK("rmsnorm_rope_kernel");
  return SRDIT_OK;
}
