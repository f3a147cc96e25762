// Fused row kernels of the refiner block for gfx950: one pass over HBM each.
//
//   ln_modulate    out = bf16( f32(bf16(LayerNorm(x) [* w + b])) * (1 + scale) + shift )
//                  and, optionally, the max |out| (float bits) into an amax word
//                  for a per-tensor fp8 quantiser of `out`
//   ln_modulate_fp8  the same rows quantised to e4m3 under their per-tensor
//                  scale without storing them: an amax pass, then a pass that
//                  recomputes and quantises; optionally on x + y * gate, whose
//                  bf16 value the first pass stores as the new residual stream
//   residual_gate  out = bf16( f32(x) + f32(y) * gate )
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
#include "fp8_common.h"

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

// Arguments of the LayerNorm row kernel.
struct LnArgs {
  const uint16_t* x;  // [M, K] bf16, row stride ldx (with RES: the residual stream)
  int64_t M;
  int K;
  int64_t ldx;
  const uint16_t* w;  // affine weight / bias, bf16 [K], or null
  const uint16_t* b;
  const float* scale;  // adaLN modulation, fp32 [K], or null
  const float* shift;
  float eps;
  void* out;          // OUT 0: bf16 [M, ldo]; OUT 2: e4m3 codes [M, ldo]
  int64_t ldo;
  uint32_t* amax_ws;  // AMAX: receives max |out| bits; OUT 2: holds them (the scale's amax)
  float* qscale;      // OUT 2: the quantiser scale, written by workgroup 0
  const uint16_t* y;  // RES: x <- bf16(x + y * gate) first, stored to xres
  int64_t ldy;
  const float* gate;
  uint16_t* xres;
  int64_t ldr;
};

// LayerNorm over each row (eps, optional affine), then optionally the adaLN
// modulation, rounded to bf16 as the reference's tensors are.  OUT selects what
// is written: 0 the bf16 rows, 1 nothing (the amax pass of a two-pass
// quantiser), 2 the rows' e4m3 codes under the scale of the amax word (its
// second pass: the same arithmetic on the same inputs, so the codes are those
// of the bf16 rows a separate quantiser would read).  RES first forms the gated
// residual x + y * gate in bf16 (stored to xres) and normalises that.
//
// Each wavefront walks rows grid-stride.  With CACHED (K <= 4096) a lane
// keeps its <= 8 chunks of the row in registers, so the row is read once;
// otherwise the mean, variance and output passes re-read it (L1/L2 hits).
// Per lane the chunks are summed in the order c = lane, lane + 64, ..., as the
// output pass visits them.  The amax is reduced per workgroup, then one
// atomicMax per workgroup.  Scale and shift are read as float4 when 16-byte
// aligned.
template <int OUT, bool RES, bool AMAX, bool CACHED>
__global__ __launch_bounds__(256) void ln_modulate_kernel(LnArgs a) {
  constexpr int CPL = 8;  // cached chunks per lane
  static_assert(!RES || CACHED, "the residual is formed in the row cache");
  const int lane = threadIdx.x & 63;
  const int K = a.K;
  const int nc = K >> 3;
  const bool affine = a.w != nullptr, mod = a.scale != nullptr;
  const bool vec = mod && ((reinterpret_cast<uintptr_t>(a.scale) | reinterpret_cast<uintptr_t>(a.shift)) & 15) == 0;
  float qs = 0.f;
  if constexpr (OUT == 2) {
    qs = q8::scale_from_amax_bits(*a.amax_ws);
    if (blockIdx.x == 0 && threadIdx.x == 0) a.qscale[0] = qs;
  }
  uint32_t am = 0;
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); row < a.M;
       row += static_cast<int64_t>(gridDim.x) * 4) {
    const uint4* xr = reinterpret_cast<const uint4*>(a.x + row * a.ldx);
    uint4 rb[CACHED ? CPL : 1];
    if (CACHED) {
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = lane + 64 * i;
        if (RES) {
          if (c < nc) {
            float xf[8], yf[8], o[8];
            unpack_bf16x8(xr[c], xf);
            unpack_bf16x8(reinterpret_cast<const uint4*>(a.y + row * a.ldy)[c], yf);
            const float4 g0 = reinterpret_cast<const float4*>(a.gate)[2 * c];
            const float4 g1 = reinterpret_cast<const float4*>(a.gate)[2 * c + 1];
            const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = __fadd_rn(xf[e], __fmul_rn(yf[e], g[e]));
            rb[i] = pack_bf16x8(o);
            reinterpret_cast<uint4*>(a.xres + row * a.ldr)[c] = rb[i];
          } else {
            rb[i] = make_uint4(0u, 0u, 0u, 0u);
          }
        } else {
          rb[i] = c < nc ? xr[c] : make_uint4(0u, 0u, 0u, 0u);
        }
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
    const float rstd = rsqrtf(wave_sum(v) / static_cast<float>(K) + a.eps);
#pragma unroll
    for (int i = 0; i < (CACHED ? CPL : 1); ++i) {
      for (int c = lane + 64 * i; c < nc && (CACHED || i == 0); c += (CACHED ? nc : 64)) {
        float f[8];
        unpack_bf16x8(chunk(i, c), f);
        float wv[8], bv[8], sv[8], hv[8];
        if (affine) {
          unpack_bf16x8(reinterpret_cast<const uint4*>(a.w)[c], wv);
          unpack_bf16x8(reinterpret_cast<const uint4*>(a.b)[c], bv);
        }
        if (mod) {
          if (vec) {
            const float4* s4 = reinterpret_cast<const float4*>(a.scale) + 2 * c;
            const float4* h4 = reinterpret_cast<const float4*>(a.shift) + 2 * c;
            const float4 s0 = s4[0], s1 = s4[1], h0 = h4[0], h1 = h4[1];
            sv[0] = s0.x; sv[1] = s0.y; sv[2] = s0.z; sv[3] = s0.w;
            sv[4] = s1.x; sv[5] = s1.y; sv[6] = s1.z; sv[7] = s1.w;
            hv[0] = h0.x; hv[1] = h0.y; hv[2] = h0.z; hv[3] = h0.w;
            hv[4] = h1.x; hv[5] = h1.y; hv[6] = h1.z; hv[7] = h1.w;
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              sv[e] = a.scale[8 * c + e];
              hv[e] = a.shift[8 * c + e];
            }
          }
        }
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float y = __fmul_rn(f[e] - mean, rstd);
          if (affine) y = __fadd_rn(__fmul_rn(y, wv[e]), bv[e]);
          y = bf16_round(y);  // LayerNorm(...).type_as(x)
          if (mod) y = __fadd_rn(__fmul_rn(y, __fadd_rn(1.0f, sv[e])), hv[e]);
          o[e] = y;
        }
        const uint4 pk = pack_bf16x8(o);
        if constexpr (OUT == 0) {
          reinterpret_cast<uint4*>(static_cast<uint16_t*>(a.out) + row * a.ldo)[c] = pk;
        } else if constexpr (OUT == 2) {
          float r[8];
          unpack_bf16x8(pk, r);  // the bf16 values a separate quantiser would read
          reinterpret_cast<uint2*>(static_cast<uint8_t*>(a.out) + row * a.ldo)[c] = q8::to_e4m3x8(r, qs);
        }
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
      atomicMax(a.amax_ws, max(max(wmax[0], wmax[1]), max(wmax[2], wmax[3])));
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
template <bool ROPE>
__global__ __launch_bounds__(256) void rmsnorm_rope_kernel(const uint16_t* __restrict__ x, int64_t M,
                                                           int K, int64_t ldx,
                                                           const uint16_t* __restrict__ w, float eps,
                                                           const float2* __restrict__ cs, int half_d,
                                                           uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const uint4* xr = reinterpret_cast<const uint4*>(x + row * ldx);
  const int nc = K >> 3;
  float ss = 0.f;
  for (int c = lane; c < nc; c += 64) {
    float f[8];
    unpack_bf16x8(xr[c], f);
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += __fmul_rn(f[i], f[i]);
  }
  const float r = rsqrtf(__fadd_rn(wave_sum(ss) / static_cast<float>(K), eps));
  const float2* csr = cs + row * half_d;
  uint4* orow = reinterpret_cast<uint4*>(out + row * K);
  for (int c = lane; c < nc; c += 64) {
    float f[8], wv[8], o[8];
    unpack_bf16x8(xr[c], f);
    unpack_bf16x8(reinterpret_cast<const uint4*>(w)[c], wv);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = bf16_round(__fmul_rn(bf16_round(__fmul_rn(f[i], r)), wv[i]));
    if (ROPE) {
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const int j = ((8 * c) >> 1) + p;  // pair index within the row
        const float2 t = csr[j % half_d];
        const float a = f[2 * p], bb = f[2 * p + 1];
        o[2 * p] = __fsub_rn(__fmul_rn(a, t.x), __fmul_rn(bb, t.y));
        o[2 * p + 1] = __fadd_rn(__fmul_rn(a, t.y), __fmul_rn(bb, t.x));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = f[i];
    }
    orow[c] = pack_bf16x8(o);
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

int check_ln(const char* who, const void* ln_w, const void* ln_b, const float* scale,
             const float* shift) {
  SRDIT_REQUIRE((ln_w == nullptr) == (ln_b == nullptr), "%s: give both affine tensors or neither",
                who);
  SRDIT_REQUIRE((scale == nullptr) == (shift == nullptr),
                "%s: give both modulation tensors or neither", who);
  SRDIT_REQUIRE((!ln_w || (aligned16(ln_w) && aligned16(ln_b))) &&
                    (!scale || ((reinterpret_cast<uintptr_t>(scale) & 3) == 0 &&
                                (reinterpret_cast<uintptr_t>(shift) & 3) == 0)),
                "%s: misaligned affine or modulation tensor", who);
  return SRDIT_OK;
}

// Grid-stride over rows: at most 2048 workgroups of 4 row-wavefronts.
unsigned ln_blocks(int64_t M) {
  const int64_t want = (M + 3) / 4;
  return static_cast<unsigned>(want < 2048 ? want : 2048);
}

template <int OUT, bool RES, bool AMAX>
void ln_launch(const LnArgs& a, hipStream_t s) {
  if (a.K <= 4096)
    ln_modulate_kernel<OUT, RES, AMAX, true><<<ln_blocks(a.M), 256, 0, s>>>(a);
  else if constexpr (!RES)
    ln_modulate_kernel<OUT, false, AMAX, false><<<ln_blocks(a.M), 256, 0, s>>>(a);
}

}  // namespace
}  // namespace srdit

extern "C" int srdit_ln_modulate(const void* x, int64_t M, int K, int64_t ldx, const void* ln_w,
                                 const void* ln_b, const float* scale, const float* shift, float eps,
                                 void* out, int64_t ldo, uint32_t* amax_ws, void* stream) {
  if (int rc = check_rows("srdit_ln_modulate", x, M, K, ldx, out, ldo)) return rc;
  if (int rc = check_ln("srdit_ln_modulate", ln_w, ln_b, scale, shift)) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (amax_ws) {
    clear_word_kernel<<<1, 1, 0, s>>>(amax_ws);
    SRDIT_LAUNCH_CHECK("clear_word_kernel");
  }
  LnArgs a{};
  a.x = static_cast<const uint16_t*>(x); a.M = M; a.K = K; a.ldx = ldx;
  a.w = static_cast<const uint16_t*>(ln_w); a.b = static_cast<const uint16_t*>(ln_b);
  a.scale = scale; a.shift = shift; a.eps = eps; a.out = out; a.ldo = ldo; a.amax_ws = amax_ws;
  if (amax_ws) ln_launch<0, false, true>(a, s);
  else ln_launch<0, false, false>(a, s);
  SRDIT_LAUNCH_CHECK("ln_modulate_kernel");
  return SRDIT_OK;
}

extern "C" int srdit_ln_modulate_fp8(const void* x, int64_t M, int K, int64_t ldx,
                                     const void* ln_w, const void* ln_b, const float* scale,
                                     const float* shift, float eps, const void* res_y,
                                     int64_t ldy, const float* res_gate, void* res_out,
                                     int64_t ldr, void* xq, float* xscale, uint32_t* amax_ws,
                                     void* stream) {
  const char* who = "srdit_ln_modulate_fp8";
  if (int rc = check_rows(who, x, M, K, ldx, xq, K)) return rc;
  if (int rc = check_ln(who, ln_w, ln_b, scale, shift)) return rc;
  SRDIT_REQUIRE(xscale && amax_ws, "%s: null scale or amax word", who);
  SRDIT_REQUIRE(reinterpret_cast<uintptr_t>(xq) % 8 == 0, "%s: codes must be 8-byte aligned", who);
  const bool res = res_y != nullptr;
  if (res) {
    SRDIT_REQUIRE(res_gate && res_out && aligned16(res_y) && aligned16(res_gate) &&
                      aligned16(res_out) && ldy >= K && ldy % 8 == 0 && ldr >= K && ldr % 8 == 0,
                  "%s: residual y / gate / out missing or misaligned, or bad ldy / ldr", who);
    SRDIT_REQUIRE(K <= 4096, "%s: the residual form needs K <= 4096 (got %d)", who, K);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  clear_word_kernel<<<1, 1, 0, s>>>(amax_ws);
  SRDIT_LAUNCH_CHECK("clear_word_kernel");
  LnArgs a{};
  a.x = static_cast<const uint16_t*>(x); a.M = M; a.K = K; a.ldx = ldx;
  a.w = static_cast<const uint16_t*>(ln_w); a.b = static_cast<const uint16_t*>(ln_b);
  a.scale = scale; a.shift = shift; a.eps = eps; a.amax_ws = amax_ws;
  // pass 1: (residual,) LayerNorm, modulation, amax of the bf16 result
  if (res) {
    a.y = static_cast<const uint16_t*>(res_y); a.ldy = ldy; a.gate = res_gate;
    a.xres = static_cast<uint16_t*>(res_out); a.ldr = ldr;
    ln_launch<1, true, true>(a, s);
  } else {
    ln_launch<1, false, true>(a, s);
  }
  SRDIT_LAUNCH_CHECK("ln_modulate_kernel (amax pass)");
  // pass 2: the same rows again, quantised with the scale of that amax
  if (res) {
    a.x = static_cast<const uint16_t*>(res_out); a.ldx = ldr;
    a.y = nullptr; a.gate = nullptr; a.xres = nullptr;
  }
  a.out = xq; a.ldo = K; a.qscale = xscale;
  ln_launch<2, false, false>(a, s);
  SRDIT_LAUNCH_CHECK("ln_modulate_kernel (quantise pass)");
  return SRDIT_OK;
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
  if (rope_cs)
    rmsnorm_rope_kernel<true><<<blocks, 256, 0, s>>>(
        static_cast<const uint16_t*>(x), M, K, ldx, static_cast<const uint16_t*>(w), eps,
        reinterpret_cast<const float2*>(rope_cs), head_dim / 2, static_cast<uint16_t*>(out));
  else
    rmsnorm_rope_kernel<false><<<blocks, 256, 0, s>>>(
        static_cast<const uint16_t*>(x), M, K, ldx, static_cast<const uint16_t*>(w), eps, nullptr,
        head_dim / 2, static_cast<uint16_t*>(out));
  SRDIT_LAUNCH_CHECK("rmsnorm_rope_kernel");
  return SRDIT_OK;
}
