// Grouped block-grid window attention forward for gfx950 (MI355X): plain-mode
// windows without an anchor prefix, two 64-query members per workgroup that
// share their K/V fetches.
//
// A member is one 64-query tile of one window (a params row and an m-tile).
// The host pairs members whose KV cuboids have the same spatial extent: the
// two m-tiles of one window, or the same spatial window in neighbouring query
// frames (their frame ranges overlap).  The workgroup has four wavefronts;
// wavefronts 2m and 2m+1 own queries [0, 32) and [32, 64) of member m and run
// the single-window kernel's per-step arithmetic.
//
// Keys are streamed in blocks of 32 consecutive keys of one frame of the
// shared spatial extent.  The workgroup walks "frame slots": first the private
// slots, in which each member consumes one of its own frames (two blocks per
// step, one per member), then the shared frames, whose blocks are fetched
// once and consumed by both members.  For the +-1-frame rule this cuts the
// L2->LDS fill traffic of a pair of neighbouring query frames from 5 or 6
// frames to 3 or 4.  Fills of step i+1 go to the other half of a two-stage
// ring while step i computes; in a private slot wavefronts 2m (K) and 2m+1 (V)
// fetch member m's block, in a shared slot wavefronts 0 (K) and 1 (V) fetch it.
//
// Numerics are those of the plain kernel (blockgrid_triton.py:184-278): fp32
// scores scaled by d^-1/2, masked keys never contribute, P rounded to the
// input dtype before P.V, fp32 accumulation, O = acc / l; exp2 with the scale
// folded in, and the lazily refreshed running max of window_common.h.

#include "window_common.h"

namespace srdit {
namespace {

using namespace win;

struct GroupArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  const int32_t* params;  // [n_w, 19] plain rows
  const int32_t* groups;  // [n_groups, 4]: row0, mtile0, row1 (-1: none), mtile1
  int n_w, n_groups, hr_base, H, W;
  int64_t q_tokens, kv_tokens;
  int n_heads;
  float scale_log2;  // softmax scale * log2(e)
};

constexpr int GKN = 32;  // keys per block

// The frames a member consumes in private slots: [lo1, lo1+len1) then
// [lo2, lo2+len2) -- its frame range minus the frames shared with the partner.
struct PrivFrames {
  int lo1, len1, lo2, len2;
};

__device__ __forceinline__ PrivFrames private_frames(int a, int la, int s_lo, int nsh) {
  PrivFrames p;
  if (nsh <= 0) {
    p.lo1 = a; p.len1 = la; p.lo2 = 0; p.len2 = 0;
    return p;
  }
  const int s_hi = s_lo + nsh;
  p.lo1 = a;
  p.len1 = max(0, min(a + la, s_lo) - a);
  p.lo2 = max(a, s_hi);
  p.len2 = max(0, a + la - p.lo2);
  return p;
}

// k-th private frame of a member, -1 when it has fewer than k+1.
__device__ __forceinline__ int private_frame(const PrivFrames& p, int k) {
  if (k < p.len1) return p.lo1 + k;
  k -= p.len1;
  return k < p.len2 ? p.lo2 + k : -1;
}

template <typename T, int D>
__global__ __launch_bounds__(256) void window_group_kernel(GroupArgs a) {
  using E = Elem<T>;
  using V8 = typename E::v8;
  constexpr int KS = D / 16;      // k-steps of the S^T MFMA over the head dim
  constexpr int DT = D / 32;      // 32-row tiles of O^T over the head dim
  constexpr int NL = D / 16;      // fill loads (1 KB each) per block
  constexpr int CPK = D / 8;      // 16-byte chunks per key row
  constexpr int LPK = CPK;        // fill lanes per key row
  constexpr int KPI = 64 / CPK;   // key rows per fill load
  constexpr int BLK = GKN * D;    // elements per block
  // [stage][block] rings: 2 stages x 2 blocks x 32 keys x D, for K and for V
  __shared__ __attribute__((aligned(16))) T ksh[4 * BLK];
  __shared__ __attribute__((aligned(16))) T vsh[4 * BLK];

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int member = wave >> 1, qhalf = wave & 1, kv_role = wave & 1;  // kv_role 0: K, 1: V
  const int lane = threadIdx.x & 63;
  const int c = lane & 31, hf = lane >> 5;

  const uint32_t task = xcd_task(blockIdx.x, gridDim.x);
  const int head = static_cast<int>(task / static_cast<uint32_t>(a.n_groups));
  const int gi = static_cast<int>(task % static_cast<uint32_t>(a.n_groups));
  if (head >= a.n_heads) return;
  const int32_t* gp = a.groups + 4 * static_cast<int64_t>(gi);
  int row0 = gp[0], mt0 = gp[1], row1 = gp[2], mt1 = gp[3];
  row0 = row0 < 0 ? 0 : (row0 >= a.n_w ? a.n_w - 1 : row0);
  row1 = row1 < 0 ? -1 : (row1 >= a.n_w ? a.n_w - 1 : row1);
  const int32_t* p0 = a.params + static_cast<int64_t>(row0) * 19;
  const int32_t* p1 = row1 >= 0 ? a.params + static_cast<int64_t>(row1) * 19 : p0;

  // Shared spatial KV extent (member 0's; the host pairs equal extents) and
  // the two frame ranges.
  const int kh0 = p0[8], kh_l = p0[9], kw0 = p0[10], kw_l = p0[11];
  const int sp = kh_l > 0 && kw_l > 0 ? kh_l * kw_l : 0;
  const int a0 = p0[6], la = sp > 0 ? max(p0[7], 0) : 0;
  const int a1 = p1[6], lb = (sp > 0 && row1 >= 0) ? max(p1[7], 0) : 0;
  const int s_lo = max(a0, a1);
  const int nsh = lb > 0 ? max(0, min(a0 + la, a1 + lb) - s_lo) : 0;
  const PrivFrames pf0 = private_frames(a0, la, s_lo, nsh);
  const PrivFrames pf1 = lb > 0 ? private_frames(a1, lb, s_lo, nsh) : PrivFrames{0, 0, 0, 0};
  const int P = max(la - nsh, lb > 0 ? lb - nsh : 0);
  const int nS = (sp + GKN - 1) / GKN;
  const int nsteps = (P + nsh) * nS;
  const float r_kw = 1.0f / static_cast<float>(kw_l > 0 ? kw_l : 1);
  auto slot_frame = [&](int w, int fs_) -> int {
    return fs_ < P ? private_frame(w == 0 ? pf0 : pf1, fs_) : s_lo + (fs_ - P);
  };

  // This wavefront's 32 queries: rows m0 + 32*qhalf + [0, 32) of its member.
  const int my_row = member == 0 ? row0 : row1;
  const int my_mt = member == 0 ? mt0 : mt1;
  const int32_t* pm = member == 0 ? p0 : p1;
  const int q_t0 = pm[0], q_tl = pm[1], q_h0 = pm[2], q_w0 = pm[3], qh_l = pm[4], qw_l = pm[5];
  const int q_sp = qh_l * qw_l;
  const int lq = q_tl * q_sp;
  const int m0 = 64 * my_mt;
  const bool has_member = my_row >= 0 && qh_l > 0 && qw_l > 0 && q_tl > 0 && m0 >= 0 && m0 < lq;

  const int L = a.H * a.W;
  const int64_t tok = static_cast<int64_t>(a.n_heads) * D;
  const int tok_bytes = static_cast<int>(tok) * static_cast<int>(sizeof(T));
  const int kv_tokens = static_cast<int>(a.kv_tokens);
  // K (even wavefronts) or V (odd) of this head as a structured buffer:
  // record = token, stride = token stride in bytes.
  const T* kvb = reinterpret_cast<const T*>(kv_role == 0 ? a.k : a.v) + head * D;
  const __amdgpu_buffer_rsrc_t kvrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<T*>(kvb), static_cast<short>(tok_bytes), kv_tokens, 0x00020000);
  const LaneOff<D> lo = make_lane_offsets<D>(kv_role);

  V8 qf[KS];
  f32x16_t oacc[DT];
  float mrun = -INFINITY, lrun = 0.f;
  const int m = m0 + 32 * qhalf + c;
  const bool qvalid = has_member && m < lq;
  int64_t qflat;
  {
    const int mm = qvalid ? m : 0;
    const int qs = q_sp > 0 ? q_sp : 1, qw = qw_l > 0 ? qw_l : 1;
    const int fr = fdiv(mm, qs, 1.0f / static_cast<float>(qs));
    const int r = mm - fr * q_sp;
    const int hh = fdiv(r, qw, 1.0f / static_cast<float>(qw));
    const int ww = r - hh * qw_l;
    qflat = static_cast<int64_t>(q_t0 + fr) * L + static_cast<int64_t>(q_h0 + hh) * a.W +
            (q_w0 + ww);
    qflat = qflat < 0 ? 0 : (qflat >= a.q_tokens ? a.q_tokens - 1 : qflat);
    const V8* qp = reinterpret_cast<const V8*>(reinterpret_cast<const T*>(a.q) + head * D +
                                               qflat * tok + hf * (D / 2));
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = qvalid ? qp[ks] : V8{};
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) oacc[dt] = f32x16_t{};
  }

  // Fill of step j into stage `stage`: block b of the step is fetched by
  // wavefronts 2b (K) and 2b+1 (V).  Source lane s of a 16-lane row decodes
  // the token of the key that load (s % LPK) places in that row; DPP
  // row_newbcast hands it to the row.
  const int s16 = lane & 15;
  const int src_key = (s16 % LPK) * KPI + (lane >> 4) * (16 / LPK) + s16 / LPK;
  const int sub = s16 / LPK;
  auto fill = [&](int j, int stage) {
    const int fs_ = j / nS, s_ = j - fs_ * nS;
    const int nblk = fs_ < P ? 2 : 1;
    if (member >= nblk) return;  // uniform
    const int f = slot_frame(member, fs_);
    if (f < 0) return;           // uniform: the member has no frame in this slot
    int idx = s_ * GKN + src_key;
    idx = idx < sp ? idx : sp - 1;
    const int row = fdiv(idx, kw_l, r_kw);
    const int col = idx - row * kw_l;
    int tokv = a.hr_base + f * L + __mul24(kh0 + row, a.W) + kw0 + col;
    tokv = tokv < 0 ? 0 : (tokv >= kv_tokens ? kv_tokens - 1 : tokv);
    T* dst = (kv_role == 0 ? ksh : vsh) + (stage * 2 + member) * BLK;
    static_for<NL>([&](auto qc) {
      constexpr int q = decltype(qc)::value;
      int t = __builtin_amdgcn_mov_dpp(tokv, 0x150 + q, 0xf, 0xf, false);
      if constexpr (LPK == 8) {
        const int t1 = __builtin_amdgcn_mov_dpp(tokv, 0x150 + 8 + q, 0xf, 0xf, false);
        t = sub ? t1 : t;
      }
      buffer_load_lds_x4(kvrsrc, dst + q * 512, t, lo.fill[q]);
    });
  };

  // One step on stage `stage` (a compile-time constant, so the LDS addresses
  // are lane offsets plus immediates).
  auto step = [&](int j, int fs_, int s_, auto stage_c) {
    constexpr int stage = decltype(stage_c)::value;
    fill_barrier();  // fill j landed; step j-1's LDS reads retired in every wavefront
    if (j + 1 < nsteps) fill(j + 1, stage ^ 1);
    const int f = slot_frame(member, fs_);
    if (!has_member || f < 0) return;  // uniform
    const int blk = fs_ < P ? member : 0;
    const char* kbuf = reinterpret_cast<const char*>(ksh + (stage * 2 + blk) * BLK);
    const char* vbuf = reinterpret_cast<const char*>(vsh + (stage * 2 + blk) * BLK);

    V8 kf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kf[ks] = *reinterpret_cast<const V8*>(kbuf + lo.k[ks]);
    f32x16_t sacc = f32x16_t{};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) sacc = E::mma(kf[ks], qf[ks], sacc);
    __builtin_amdgcn_sched_group_barrier(0x100, KS, 0);  // the K reads
    __builtin_amdgcn_sched_group_barrier(0x008, KS, 0);  // then the MFMAs

    const int nvalid = sp - s_ * GKN;  // the last block of a frame can be partial
    if (nvalid < GKN) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = 8 * (r >> 2) + 4 * hf + (r & 3);
        if (key >= nvalid) sacc[r] = -INFINITY;
      }
    }
    float mx = sacc[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sacc[r]);
    mx = other_half_max(mx) * a.scale_log2;
    const bool up = mx > mrun + TAU;
    if (__any(up)) {
      const float alpha = up ? __builtin_amdgcn_exp2f(mrun - mx) : 1.0f;
      lrun *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) oacc[dt] *= alpha;
      mrun = up ? mx : mrun;
    }
    const float msub = mrun == -INFINITY ? 0.f : mrun;
    float pv[16];
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      pv[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[r], a.scale_log2, -msub));
      psum += pv[r];
    }
    lrun += psum;
    const V8 pf0 = E::pack8(&pv[0]);
    const V8 pf1 = E::pack8(&pv[8]);
    V8 vt[2][DT];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        i32x2_t half[2];
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          const char* src = vbuf + (16 * kk + 8 * h2) * CPK * 16 + lo.v[dt];
          half[h2] = __builtin_bit_cast(
              i32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(const_cast<char*>(src))));
        }
        const i32x4_t vw = {half[0][0], half[0][1], half[1][0], half[1][1]};
        vt[kk][dt] = __builtin_bit_cast(V8, vw);
      }
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) oacc[dt] = E::mma(vt[kk][dt], kk == 0 ? pf0 : pf1, oacc[dt]);
  };

  if (nsteps > 0) fill(0, 0);
  int fs = 0, s = 0;  // frame slot and spatial step of step j
  auto advance = [&]() {
    if (++s == nS) {
      s = 0;
      ++fs;
    }
  };
  int j = 0;
  for (; j + 1 < nsteps; j += 2) {
    step(j, fs, s, std::integral_constant<int, 0>{});
    advance();
    step(j + 1, fs, s, std::integral_constant<int, 1>{});
    advance();
  }
  if (j < nsteps) step(j, fs, s, std::integral_constant<int, 0>{});

  // O = acc / l ; lane (c, hf) writes dims dt*32 + 8*g4 + 4*hf + [0, 4) of its query
  const float lt = half_sum(lrun);
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  if (!qvalid) return;
  T* op = reinterpret_cast<T*>(a.o) + head * D + qflat * tok;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const f32x2_t lo2 = {oacc[dt][g4 * 4 + 0] * inv, oacc[dt][g4 * 4 + 1] * inv};
      const f32x2_t hi2 = {oacc[dt][g4 * 4 + 2] * inv, oacc[dt][g4 * 4 + 3] * inv};
      const i32x2_t w = {__builtin_bit_cast(int, __builtin_convertvector(lo2, typename E::h2)),
                         __builtin_bit_cast(int, __builtin_convertvector(hi2, typename E::h2))};
      *reinterpret_cast<i32x2_t*>(op + dt * 32 + g4 * 8 + hf * 4) = w;
    }
}

template <typename T, int D>
int launch_group(const GroupArgs& a, uint32_t grid, hipStream_t stream) {
  hipLaunchKernelGGL((window_group_kernel<T, D>), dim3(grid), dim3(256), 0, stream, a);
  SRDIT_LAUNCH_CHECK("window_group_kernel");
  return SRDIT_OK;
}

}  // namespace
}  // namespace srdit

extern "C" int srdit_window_attn_grouped_fwd(const void* q, const void* k, const void* v, void* o,
                                             const int32_t* params, const int32_t* groups,
                                             int n_w, int n_groups, int hr_base, int H, int W,
                                             int64_t q_tokens, int64_t kv_tokens, int n_heads,
                                             int head_dim, float scale, int dtype, void* stream) {
  using namespace srdit;
  SRDIT_REQUIRE(q && k && v && o && params && groups, "srdit_window_attn_grouped_fwd: null pointer");
  SRDIT_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o),
                "srdit_window_attn_grouped_fwd: q/k/v/o must be 16-byte aligned");
  SRDIT_REQUIRE(n_w >= 1 && n_groups >= 1 && n_heads >= 1 && H >= 1 && W >= 1 && hr_base >= 0,
                "srdit_window_attn_grouped_fwd: bad sizes (n_w=%d n_groups=%d n_heads=%d H=%d W=%d "
                "hr_base=%d)", n_w, n_groups, n_heads, H, W, hr_base);
  SRDIT_REQUIRE(q_tokens >= 1 && kv_tokens >= 1 && q_tokens < (1LL << 24),
                "srdit_window_attn_grouped_fwd: token counts out of range");
  SRDIT_REQUIRE(static_cast<int64_t>(H) * W < (1LL << 22), "srdit_window_attn_grouped_fwd: grid too large");
  SRDIT_REQUIRE(kv_tokens * n_heads * head_dim * 2 < (1LL << 31),
                "srdit_window_attn_grouped_fwd: K/V must span fewer than 2^31 bytes");
  SRDIT_REQUIRE(static_cast<int64_t>(n_heads) * head_dim * 2 < (1LL << 14),
                "srdit_window_attn_grouped_fwd: token stride n_heads*head_dim*2 must be below 16384 "
                "bytes (structured-buffer stride)");
  if (head_dim != 64 && head_dim != 128) {
    set_error("srdit_window_attn_grouped_fwd: head_dim %d unsupported (64 or 128)", head_dim);
    return SRDIT_EUNSUPPORTED;
  }
  if (dtype != SRDIT_DTYPE_BF16 && dtype != SRDIT_DTYPE_FP16) {
    set_error("srdit_window_attn_grouped_fwd: dtype code %d unsupported", dtype);
    return SRDIT_EUNSUPPORTED;
  }
  const int64_t grid64 = static_cast<int64_t>(n_groups) * n_heads;
  SRDIT_REQUIRE(grid64 < (1LL << 31), "srdit_window_attn_grouped_fwd: too many tasks");
  GroupArgs a;
  a.q = q; a.k = k; a.v = v; a.o = o; a.params = params; a.groups = groups;
  a.n_w = n_w; a.n_groups = n_groups; a.hr_base = hr_base; a.H = H; a.W = W;
  a.q_tokens = q_tokens; a.kv_tokens = kv_tokens; a.n_heads = n_heads;
  a.scale_log2 = scale * 1.4426950408889634f;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const uint32_t grid = static_cast<uint32_t>(grid64);
  if (dtype == SRDIT_DTYPE_BF16)
    return head_dim == 128 ? launch_group<__bf16, 128>(a, grid, s) : launch_group<__bf16, 64>(a, grid, s);
  return head_dim == 128 ? launch_group<_Float16, 128>(a, grid, s) : launch_group<_Float16, 64>(a, grid, s);
}
