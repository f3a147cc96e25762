// Grouped block-grid window attention forward for gfx950 (MI355X): plain-mode
// windows without an anchor prefix, two 64-query members per workgroup.
//
// A member is one 64-query tile of one window (a params row and an m-tile).
// The host pairs members whose KV cuboids have the same spatial extent: the
// two m-tiles of one window, or the same spatial window in neighbouring query
// frames (their frame ranges overlap).  Wavefront w of the workgroup owns
// member w, all 64 of its queries, as two 32-query halves.
//
// Keys are streamed in blocks of 32 consecutive keys of one frame of the
// shared spatial extent.  The workgroup walks "frame slots": first the
// private slots, in which each member consumes one of its own frames (two
// blocks per step, one per member), then the shared frames, whose blocks are
// fetched once and consumed by both members.  Sharing cuts the L2->LDS fill
// traffic of a +-1-frame pair from 5 to 3 (edge pairs) or 6 to 4 frames.
//
// Per step and member (32 keys x 64 queries):
//   S^T[32 x 32] (x2 halves) = K[32 x D] . Q^T[D x 32]    v_mfma_f32_32x32x16
//   O^T[D x 32]  (x2 halves) += V^T[D x 32] . P^T[32 x 32]
// Each K fragment (ds_read_b128) and each V^T fragment (ds_read_b64_tr_b16)
// feeds both halves, so LDS reads per MFMA are half those of a 32-query
// wavefront.  Wavefront 0 fetches the step's K blocks and wavefront 1 its V
// blocks straight into LDS (buffer_load ... lds) one step ahead, into a
// two-stage ring.
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
__global__ __launch_bounds__(128) void window_group_kernel(GroupArgs a) {
  using E = Elem<T>;
  using V8 = typename E::v8;
  constexpr int KS = D / 16;      // k-steps of the S^T MFMA over the head dim
  constexpr int DT = D / 32;      // 32-row tiles of O^T over the head dim
  constexpr int NL = D / 16;      // fill loads (1 KB each) per block
  constexpr int CPK = D / 8;      // 16-byte chunks per key row
  constexpr int LPK = CPK;        // fill lanes per key row
  constexpr int KPI = 64 / CPK;   // key rows per fill load
  constexpr int BLK = GKN * D;    // elements per block
  auto swz_k = [](int key) { return (key * CPK / 16) % CPK; };
  auto swz_v = [](int key) {
    return D == 128 ? ((4 * (key & 3)) ^ (8 * ((key >> 2) & 1))) : (key % CPK);
  };
  // [stage][block] rings: 2 x 2 x 32 keys x D, for K and for V
  __shared__ __attribute__((aligned(16))) T ksh[4 * BLK];
  __shared__ __attribute__((aligned(16))) T vsh[4 * BLK];

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int c = lane & 31, hf = lane >> 5;
  const int g = lane >> 4, i16 = lane & 15;

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

  // This wavefront's member.
  const int my_row = wave == 0 ? row0 : row1;
  const int my_mt = wave == 0 ? mt0 : mt1;
  const int32_t* pm = wave == 0 ? p0 : p1;
  const int q_t0 = pm[0], q_tl = pm[1], q_h0 = pm[2], q_w0 = pm[3], qh_l = pm[4], qw_l = pm[5];
  const int q_sp = qh_l * qw_l;
  const int lq = q_tl * q_sp;
  const int m0 = 64 * my_mt;
  const bool has_member = my_row >= 0 && qh_l > 0 && qw_l > 0 && q_tl > 0 && m0 >= 0 && m0 < lq;

  const int L = a.H * a.W;
  const int64_t tok = static_cast<int64_t>(a.n_heads) * D;
  const int tok_bytes = static_cast<int>(tok) * static_cast<int>(sizeof(T));
  const int kv_tokens = static_cast<int>(a.kv_tokens);
  // K (wavefront 0) or V (wavefront 1) of this head as a buffer resource.
  const T* kvb = reinterpret_cast<const T*>(wave == 0 ? a.k : a.v) + head * D;
  const __amdgpu_buffer_rsrc_t kvrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<T*>(kvb), 0,
      kv_tokens * tok_bytes - head * D * static_cast<int>(sizeof(T)), 0x00020000);

  // Queries: half h, lane (c, hf) -> row m = m0 + 32h + c of the member.
  V8 qf[2][KS];
  f32x16_t oacc[2][DT];
  float mrun[2], lrun[2];
  int64_t qflat[2];
  bool qvalid[2];
  {
    const T* qb = reinterpret_cast<const T*>(a.q) + head * D;
    const float r_qsp = 1.0f / static_cast<float>(q_sp > 0 ? q_sp : 1);
    const float r_qw = 1.0f / static_cast<float>(qw_l > 0 ? qw_l : 1);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int m = m0 + 32 * h + c;
      qvalid[h] = has_member && m < lq;
      const int mm = qvalid[h] ? m : 0;
      const int fr = fdiv(mm, q_sp > 0 ? q_sp : 1, r_qsp);
      const int r = mm - fr * q_sp;
      const int hh = fdiv(r, qw_l > 0 ? qw_l : 1, r_qw);
      const int ww = r - hh * qw_l;
      int64_t qt = static_cast<int64_t>(q_t0 + fr) * L + static_cast<int64_t>(q_h0 + hh) * a.W +
                   (q_w0 + ww);
      qt = qt < 0 ? 0 : (qt >= a.q_tokens ? a.q_tokens - 1 : qt);
      qflat[h] = qt;
      const V8* qp = reinterpret_cast<const V8*>(qb + qt * tok + hf * (D / 2));
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) qf[h][ks] = qvalid[h] ? qp[ks] : V8{};
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) oacc[h][dt] = f32x16_t{};
      mrun[h] = -INFINITY;
      lrun[h] = 0.f;
    }
  }

  // Step j -> (frame slot fs, spatial step s), and the frame member w consumes
  // there (-1: none).  A private slot's step holds one block per member (block
  // w); a shared slot's step holds one block (block 0).
  auto slot_frame = [&](int w, int fs_) -> int {
    return fs_ < P ? private_frame(w == 0 ? pf0 : pf1, fs_) : s_lo + (fs_ - P);
  };
  auto my_frame = [&](int j) -> int {
    if (!has_member || j < 0 || j >= nsteps) return -1;
    return slot_frame(wave, j / nS);
  };
  // LDS block ring: 4 block slots for K and 4 for V.  Step j takes nb(j)
  // consecutive slots (mod 4) starting at slot_start(j); steps are placed in
  // order, so a shared-phase step can be fetched up to three steps ahead and a
  // private-phase step one step ahead.
  const int PnS = P * nS;
  auto nb = [&](int j) -> int { return j < PnS ? 2 : 1; };
  auto slot_start = [&](int j) -> int { return (j < PnS ? 2 * j : 2 * PnS + (j - PnS)) & 3; };
  // loads this wavefront issues for step j: one group of NL per fetched block
  auto step_loads = [&](int j) -> int {
    const int fs_ = j / nS;
    if (fs_ >= P) return NL;
    return NL * ((slot_frame(0, fs_) >= 0) + (slot_frame(1, fs_) >= 0));
  };

  // Fill of step j: wavefront 0 loads its K blocks, wavefront 1 its V blocks.
  // As in the plain kernel, source lane s of a 16-lane row decodes the token of
  // the key that load (s % LPK) places in that row, and DPP row_newbcast hands
  // it to the row.
  auto fill = [&](int j) {
    const int fs_ = j / nS, s_ = j - fs_ * nS;
    const int nblk = fs_ < P ? 2 : 1;
    const int s16 = lane & 15;
    const int src_key = (s16 % LPK) * KPI + (lane >> 4) * (16 / LPK) + s16 / LPK;
    int idx = s_ * GKN + src_key;
    idx = idx < sp ? idx : sp - 1;
    const int row = fdiv(idx, kw_l, r_kw);
    const int col = idx - row * kw_l;
    const int sp_tok = (kh0 + row) * a.W + kw0 + col;
    const int sub = s16 / LPK, pos = lane % CPK;
    const int st0 = slot_start(j);
    for (int b = 0; b < nblk; ++b) {
      const int f = slot_frame(b, fs_);
      if (f < 0) continue;  // uniform: that member has no frame in this slot
      int tokv = a.hr_base + f * L + sp_tok;
      tokv = tokv < 0 ? 0 : (tokv >= kv_tokens ? kv_tokens - 1 : tokv);
      T* dst = (wave == 0 ? ksh : vsh) + ((st0 + b) & 3) * BLK;
      static_for<NL>([&](auto qc) {
        constexpr int q = decltype(qc)::value;
        int t = __builtin_amdgcn_mov_dpp(tokv, 0x150 + q, 0xf, 0xf, false);
        if constexpr (LPK == 8) {
          const int t1 = __builtin_amdgcn_mov_dpp(tokv, 0x150 + 8 + q, 0xf, 0xf, false);
          t = sub ? t1 : t;
        }
        const int key = q * KPI + (lane >> 4) * (16 / LPK) + sub;
        const int chunk_off = (pos ^ (wave == 0 ? swz_k(key) : swz_v(key))) * 16;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            kvrsrc, (lds_void_t*)(dst + q * 512), 16,
            static_cast<int>(__umul24(t, tok_bytes)) + chunk_off, 0, 0, 0);
      });
    }
  };

  // S^T = K Q^T for both halves; each K fragment feeds two MFMAs.
  auto scores = [&](const T* kbuf, f32x16_t (&sacc)[2]) {
    V8 kf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      kf[ks] = *reinterpret_cast<const V8*>(kbuf + (c * CPK + ((hf * KS + ks) ^ swz_k(c))) * 8);
    sacc[0] = f32x16_t{};
    sacc[1] = f32x16_t{};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      sacc[0] = E::mma(kf[ks], qf[0][ks], sacc[0]);
      sacc[1] = E::mma(kf[ks], qf[1][ks], sacc[1]);
    }
  };
  // keys past the spatial extent in the last block of a frame
  auto mask_tail = [&](int j, f32x16_t (&sacc)[2]) {
    const int nvalid = sp - (j % nS) * GKN;
    if (nvalid < GKN) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = 8 * (r >> 2) + 4 * hf + (r & 3);
        if (key >= nvalid) {
          sacc[0][r] = -INFINITY;
          sacc[1][r] = -INFINITY;
        }
      }
    }
  };
  // row max of both halves, log2 units
  auto rowmax = [&](const f32x16_t (&sacc)[2], float (&mx)[2]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float m_ = sacc[h][0];
#pragma unroll
      for (int r = 1; r < 16; ++r) m_ = fmaxf(m_, sacc[h][r]);
      mx[h] = other_half_max(m_) * a.scale_log2;
    }
  };
  // lazy refresh of the running max before the step's exponentials
  auto rescale = [&](const float (&mx)[2]) {
    const bool up0 = mx[0] > mrun[0] + TAU, up1 = mx[1] > mrun[1] + TAU;
    if (__any(up0 || up1)) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const bool up = h == 0 ? up0 : up1;
        const float alpha = up ? __builtin_amdgcn_exp2f(mrun[h] - mx[h]) : 1.0f;
        lrun[h] *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) oacc[h][dt] *= alpha;
        mrun[h] = up ? mx[h] : mrun[h];
      }
    }
  };
  // P = exp2(s * scale_log2 - m) for half h, its row sum, packed MFMA operands
  auto probs = [&](const f32x16_t& sh, int h, V8 (&pf)[2]) {
    const float msub = mrun[h] == -INFINITY ? 0.f : mrun[h];
    float pv[16];
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      pv[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sh[r], a.scale_log2, -msub));
      psum += pv[r];
    }
    lrun[h] += psum;
    pf[0] = E::pack8(&pv[0]);
    pf[1] = E::pack8(&pv[8]);
  };
  // V^T fragments of a block: lane reads 8 bytes of chunk L = 4dt + 2(g&1) +
  // (i16&3)/2, half (i16&1), of key 16kk + 8h2 + 4hf + i16/4
  auto vfrag = [&](const T* vbuf, int kk, int dt) -> V8 {
    const int Lc = 4 * dt + 2 * (g & 1) + ((i16 & 3) >> 1);
    i32x2_t half[2];
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const int key = 16 * kk + 8 * h2 + 4 * hf + (i16 >> 2);
      const T* src = vbuf + (key * CPK + (Lc ^ swz_v(key))) * 8 + 4 * (i16 & 1);
      half[h2] = __builtin_bit_cast(
          i32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(const_cast<T*>(src))));
    }
    const i32x4_t vw = {half[0][0], half[0][1], half[1][0], half[1][1]};
    return __builtin_bit_cast(V8, vw);
  };

  // Main loop.  At the top of iteration i the barrier retires step i-1 in
  // both wavefronts (its slots become free) after this wavefront's loads for
  // step i have landed; loads of later steps stay in flight.
  int issued = 0, used = 0, inflight = 0;  // steps fetched, slots held, loads of steps > i
  while (issued < nsteps && used + nb(issued) <= 4) {
    fill(issued);
    used += nb(issued);
    inflight += step_loads(issued);
    ++issued;
  }
  for (int i = 0; i < nsteps; ++i) {
    inflight -= step_loads(i);
    fill_barrier_keep(inflight);
    if (i > 0) used -= nb(i - 1);
    while (issued < nsteps && used + nb(issued) <= 4) {
      fill(issued);
      used += nb(issued);
      inflight += step_loads(issued);
      ++issued;
    }
    if (my_frame(i) >= 0) {
      const int blk = (i / nS) < P ? wave : 0;
      const int slot = (slot_start(i) + blk) & 3;
      f32x16_t sacc[2];
      scores(ksh + slot * BLK, sacc);
      mask_tail(i, sacc);
      float mx[2];
      rowmax(sacc, mx);
      rescale(mx);
      const T* vbuf = vsh + slot * BLK;
      V8 pf[2][2];
      probs(sacc[0], 0, pf[0]);
      probs(sacc[1], 1, pf[1]);
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const V8 vt = vfrag(vbuf, kk, dt);
          oacc[0][dt] = E::mma(vt, pf[0][kk], oacc[0][dt]);
          oacc[1][dt] = E::mma(vt, pf[1][kk], oacc[1][dt]);
        }
    }
  }

  // O = acc / l ; lane (c, hf) writes dims dt*32 + 8*g4 + 4*hf + [0, 4) of its query
  T* ob = reinterpret_cast<T*>(a.o) + head * D;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float lt = half_sum(lrun[h]);
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
    if (!qvalid[h]) continue;
    T* op = ob + qflat[h] * tok;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const f32x2_t lo = {oacc[h][dt][g4 * 4 + 0] * inv, oacc[h][dt][g4 * 4 + 1] * inv};
        const f32x2_t hi = {oacc[h][dt][g4 * 4 + 2] * inv, oacc[h][dt][g4 * 4 + 3] * inv};
        const i32x2_t w = {__builtin_bit_cast(int, __builtin_convertvector(lo, typename E::h2)),
                           __builtin_bit_cast(int, __builtin_convertvector(hi, typename E::h2))};
        *reinterpret_cast<i32x2_t*>(op + dt * 32 + g4 * 8 + hf * 4) = w;
      }
  }
}

template <typename T, int D>
int launch_group(const GroupArgs& a, uint32_t grid, hipStream_t stream) {
  hipLaunchKernelGGL((window_group_kernel<T, D>), dim3(grid), dim3(128), 0, stream, a);
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
  SRDIT_REQUIRE(static_cast<int64_t>(n_heads) * head_dim * 2 < (1LL << 24),
                "srdit_window_attn_grouped_fwd: token stride too large");
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
