// Block-grid window attention forward for gfx950 (MI355X).
//
// One workgroup of two wavefronts owns one task = (window, 64-query tile,
// head); wavefront w owns queries [32w, 32w + 32) of the tile.  The workgroup
// walks the window's KV cuboid 32 keys per step with an online softmax:
//
//   S^T[32 keys x 32 queries] = K[32 x D] . Q^T[D x 32]      (v_mfma 32x32x16)
//   O^T[D x 32 queries]      += V^T[D x 32 keys] . P^T[32 x 32]
//
// Computing S transposed puts one query per lane (column = lane % 32), so the
// softmax statistics are lane-local: a lane and its partner lane+32 hold the
// same query's 16+16 keys, and one permlane32 swap combines them.  The S^T
// accumulator registers feed the P^T operand of the second MFMA directly (the
// contraction over keys uses the accumulator's own key order).
//
// K and V tiles of a step are fetched once per workgroup straight into LDS
// with global_load_lds_dwordx4 (wavefront 0 fetches K, wavefront 1 fetches V)
// into two-stage rings, so the fetch of step i+1 overlaps step i.  K is read
// back as the MFMA A operand with ds_read_b128, V^T with ds_read_b64_tr_b16.
// Two wavefronts per SIMD keep the matrix pipe busy while the other one runs
// its softmax.
//
// Semantics follow the reference kernels
// (video_refiner/wan/modules/sr_dit/blockgrid_triton.py:184-278 plain,
//  :281-389 per-frame anchor): scale applied to q.k in fp32, masked keys never
// contribute, a fully masked tile leaves the running statistics unchanged,
// P is rounded to the input dtype before P.V, fp32 accumulation, O = acc / l.
// The exponential is evaluated as exp2 of log2(e)-scaled logits, and the
// running max is refreshed lazily (see TAU).

#include "window_common.h"

namespace srdit {
namespace {

using namespace win;

struct WinArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  const int32_t* params;
  const int32_t* order;
  int n_w, m_tiles, p_stride, hr_base, H, W;
  int64_t q_tokens, kv_tokens;
  int n_heads;
  float scale_log2;  // softmax scale * log2(e)
  int ring_R, ring_nc;       // in-place KV cache layout (ring_R == 0: plain)
  const int32_t* ring_head;  // device int32: ring slot of the oldest cached frame
  uint32_t* amax_out;        // max |O| bits, or null
};

constexpr int WAVES = 2;  // wavefronts per workgroup, 32 queries each
constexpr int KN = 32;    // keys per step
constexpr int STAGES = 2; // LDS ring: the unrolled step pair alternates the two stages


template <typename T, int D>
struct Tile {
  using E = Elem<T>;
  using V8 = typename E::v8;
  static constexpr int KS = D / 16;  // k-steps of the S^T MFMA over the head dim
  static constexpr int DT = D / 32;  // 32-row tiles of O^T over the head dim
  static constexpr int NL = D / 16;  // 16-byte fill loads per lane per tile

  V8 qf[KS];           // Q^T operand: lane (c, hf), k-step ks -> dims [hf*D/2 + 8ks, +8)
  f32x16_t oacc[DT];   // O^T accumulator, rows = head dims, column = query c
  float mrun, lrun;    // running max (log2 units, lazily refreshed) and sum
};

// Token of key j of a run, walked forward KN keys per step: the lane keeps its
// key's index within the current frame, the frame's logical index and that
// frame's first token (the ring maps logical frames to physical ones).
struct KeyCursor {
  int rr;         // index of the key within its frame of the run
  int f;          // logical frame: t0 + t
  int frame_tok;  // token of that frame's first cuboid cell: base + phys(f) * frame_len
};

__device__ __forceinline__ KeyCursor cursor_at(const KeyRun& k, int j) {
  const int sp = k.rows * k.cols;
  const int t = fdiv(j, sp, k.r_sp);
  KeyCursor c;
  c.rr = j - t * sp;
  c.f = k.t0 + t;
  c.frame_tok = k.base + ring_frame(k.ring, c.f) * k.frame_len;
  return c;
}

__device__ __forceinline__ int cursor_token(const KeyRun& k, const KeyCursor& c) {
  const int row = fdiv(c.rr, k.cols, k.r_cols);
  const int col = c.rr - row * k.cols;
  return c.frame_tok + __mul24(k.r0 + row, k.Wg) + (k.c0 + col);
}

__device__ __forceinline__ void cursor_advance(const KeyRun& k, KeyCursor& c, int by) {
  const int sp = k.rows * k.cols;
  c.rr += by;
  bool moved = false;
  while (c.rr >= sp) {  // at most ceil(by / sp) frames
    c.rr -= sp;
    ++c.f;
    moved = true;
  }
  if (moved) c.frame_tok = k.base + ring_frame(k.ring, c.f) * k.frame_len;
}

// Walk one key run with the online softmax.  `seg` >= 0 restricts the run to
// queries of frame `seg` (per-frame anchor), -1 admits all.  Must be called
// by both wavefronts of the workgroup with the same run (barriers inside).
// `kvrsrc` is a structured buffer over this head's K (wavefront 0) or V
// (wavefront 1): record = token, stride = token stride in bytes.
template <typename T, int D>
__device__ __forceinline__ void attend_run(Tile<T, D>& st, const KeyRun& run, int seg, int wave,
                                           int qframe, bool qvalid, __amdgpu_buffer_rsrc_t kvrsrc,
                                           int kv_tokens, float scale_log2, T* ksh, T* vsh,
                                           const LaneOff<D>& lo) {
  using TT = Tile<T, D>;
  using E = typename TT::E;
  using V8 = typename TT::V8;
  constexpr int KS = TT::KS, DT = TT::DT, NL = TT::NL;
  constexpr int TILE = KN * D;  // elements per LDS stage
  constexpr int CPK = D / 8;    // 16-byte chunks per key row
  constexpr int LPK = CPK;      // fill lanes per key row
  constexpr int KPI = 64 / CPK; // key rows per fill load
  if (run.n <= 0) return;
  const int lane = threadIdx.x & 63;
  const int hf = lane >> 5;
  const int nsteps = (run.n + KN - 1) / KN;
  const bool admit = (seg < 0) || (qvalid && qframe == seg);

  // Fill of step i into stage i & 1: wavefront 0 loads K, wavefront 1 loads V.
  // Source lane s of a 16-lane row r holds the token of the key that load
  // (s % LPK) places in that row's sub-row s / LPK; DPP row_newbcast hands it
  // to the row's lanes.  The lane's key advances KN keys per step.
  const int s16 = lane & 15;
  const int src_key = (s16 % LPK) * KPI + (lane >> 4) * (16 / LPK) + s16 / LPK;
  KeyCursor cur = cursor_at(run, src_key < run.n ? src_key : run.n - 1);
  int fill_key = src_key;
  const int sub = s16 / LPK;
  T* const fill_base = wave == 0 ? ksh : vsh;
  auto fill = [&](int stage) {  // stage is a constant after inlining
    int tokv = cursor_token(run, cur);
    tokv = tokv < 0 ? 0 : (tokv >= kv_tokens ? kv_tokens - 1 : tokv);
    // keys past the run are clamped tokens; their scores are masked
    fill_key += KN;
    if (fill_key < run.n) cursor_advance(run, cur, KN);
    static_for<NL>([&](auto qc) {
      constexpr int q = decltype(qc)::value;
      int t = __builtin_amdgcn_mov_dpp(tokv, 0x150 + q, 0xf, 0xf, false);
      if constexpr (LPK == 8) {
        const int t1 = __builtin_amdgcn_mov_dpp(tokv, 0x150 + 8 + q, 0xf, 0xf, false);
        t = sub ? t1 : t;
      }
      buffer_load_lds_x4(kvrsrc, fill_base + stage * TILE + q * 512, t, lo.fill[q]);
    });
  };

  // One step on stage `stage` (a compile-time constant, so every LDS address
  // below is a lane offset plus an immediate).
  auto step = [&](int i, auto stage_c) {
    constexpr int stage = decltype(stage_c)::value;
    // Fill i has landed in both halves and step i-1's LDS reads are done, so
    // the other stage (step i-1's) may be refilled with step i+1.
    fill_barrier();
    if (i + 1 < nsteps) fill(stage ^ 1);
    const char* kbuf = reinterpret_cast<const char*>(ksh + stage * TILE);
    const char* vbuf = reinterpret_cast<const char*>(vsh + stage * TILE);

    // S^T = K Q^T: all K fragments of the step first, then the MFMA chain
    V8 kf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kf[ks] = *reinterpret_cast<const V8*>(kbuf + lo.k[ks]);
    f32x16_t sacc = f32x16_t{};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) sacc = E::mma(kf[ks], st.qf[ks], sacc);
    __builtin_amdgcn_sched_group_barrier(0x100, KS, 0);  // the K reads
    __builtin_amdgcn_sched_group_barrier(0x008, KS, 0);  // then the MFMAs

    // masking on a partial last step or inside an anchor segment
    const int nvalid = run.n - i * KN;
    if (nvalid < KN || seg >= 0) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = 8 * (r >> 2) + 4 * hf + (r & 3);
        if (!(key < nvalid && admit)) sacc[r] = -INFINITY;
      }
    }

    // online softmax, one query per lane, lazily rescaled
    float mx = sacc[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sacc[r]);
    mx = other_half_max(mx) * scale_log2;
    // A lane rescales when its max grew by more than TAU (mx is then finite);
    // a lane with a fully masked tile (mx = -inf) never does.
    const bool up = mx > st.mrun + TAU;
    if (__any(up)) {
      const float alpha = up ? __builtin_amdgcn_exp2f(st.mrun - mx) : 1.0f;  // 0 on a first tile
      st.lrun *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) st.oacc[dt] *= alpha;
      st.mrun = up ? mx : st.mrun;
    }
    // until the first unmasked score the running max is -inf and every P is 0
    const float msub = st.mrun == -INFINITY ? 0.f : st.mrun;
    float pv[16];
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      pv[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[r], scale_log2, -msub));
      psum += pv[r];
    }
    st.lrun += psum;
    const V8 pf0 = E::pack8(&pv[0]);
    const V8 pf1 = E::pack8(&pv[8]);

    // O^T += V^T P^T, V^T via transposing LDS reads: the lane receives four
    // consecutive keys (16kk + 8h2 + 4hf + i16/4 ...) of head dim dt*32 + c.
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
      for (int dt = 0; dt < DT; ++dt) st.oacc[dt] = E::mma(vt[kk][dt], kk == 0 ? pf0 : pf1, st.oacc[dt]);
  };

  fill(0);
  int i = 0;
  for (; i + 1 < nsteps; i += 2) {
    step(i, std::integral_constant<int, 0>{});
    step(i + 1, std::integral_constant<int, 1>{});
  }
  if (i < nsteps) step(i, std::integral_constant<int, 0>{});
  fill_barrier();  // stages free for the next run
}

template <typename T, int D, int MODE>
__global__ __launch_bounds__(64 * WAVES) void window_attn_kernel(WinArgs a) {
  using TT = Tile<T, D>;
  using E = typename TT::E;
  using V8 = typename TT::V8;
  constexpr int KS = TT::KS, DT = TT::DT;
  __shared__ __attribute__((aligned(16))) T ksh[STAGES * KN * D];
  __shared__ __attribute__((aligned(16))) T vsh[STAGES * KN * D];

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int lane = threadIdx.x & 63;
  const int c = lane & 31, hf = lane >> 5;
  const uint32_t task = xcd_task(blockIdx.x, gridDim.x);
  // Head-major: each XCD walks whole heads, so the workgroups sharing its L2
  // read overlapping KV cuboids of one head.
  const uint32_t per_head = static_cast<uint32_t>(a.n_w) * static_cast<uint32_t>(a.m_tiles);
  const int head = static_cast<int>(task / per_head);
  const uint32_t rest = task % per_head;
  const int mt = static_cast<int>(rest % static_cast<uint32_t>(a.m_tiles));
  const uint32_t wslot = rest / static_cast<uint32_t>(a.m_tiles);
  if (wslot >= static_cast<uint32_t>(a.n_w) || head >= a.n_heads) return;
  int wid = a.order[wslot];
  wid = wid < 0 ? 0 : (wid >= a.n_w ? a.n_w - 1 : wid);
  const int32_t* p = a.params + static_cast<int64_t>(wid) * a.p_stride;

  int q_t0, q_tl, q_h0, q_w0, qh_l, qw_l, kv_t0, kv_tl, kh0, kh_l, kw0, kw_l, a_frames;
  int kh0_a, kh_l_a, kw0_a, kw_l_a, h_a, w_a;
  if (MODE == 0) {
    q_t0 = p[0]; q_tl = p[1]; q_h0 = p[2]; q_w0 = p[3]; qh_l = p[4]; qw_l = p[5];
    kv_t0 = p[6]; kv_tl = p[7]; kh0 = p[8]; kh_l = p[9]; kw0 = p[10]; kw_l = p[11];
    a_frames = p[12]; kh0_a = p[13]; kh_l_a = p[14]; kw0_a = p[15]; kw_l_a = p[16];
    h_a = p[17]; w_a = p[18];
  } else {
    q_t0 = 0; q_h0 = p[0]; q_w0 = p[1]; qh_l = p[2]; qw_l = p[3];
    kv_t0 = p[4]; kv_tl = p[5]; kh0 = p[6]; kh_l = p[7]; kw0 = p[8]; kw_l = p[9];
    q_tl = p[10]; a_frames = 0; kh0_a = p[11]; kh_l_a = p[12]; kw0_a = p[13]; kw_l_a = p[14];
    h_a = p[15]; w_a = p[16];
  }
  const int q_sp = qh_l * qw_l;
  const int lq = q_tl * q_sp;
  const int m0 = mt * 64;
  if (q_sp <= 0 || q_tl <= 0 || m0 >= lq) return;  // uniform over the workgroup

  const int L = a.H * a.W;
  const int64_t tok = static_cast<int64_t>(a.n_heads) * D;
  const T* qb = reinterpret_cast<const T*>(a.q) + head * D;
  // K (wavefront 0) or V (wavefront 1) of this head as a structured buffer:
  // record = token, stride = token stride in bytes; the hardware checks the
  // record index against kv_tokens.
  const int tok_bytes = static_cast<int>(tok) * static_cast<int>(sizeof(T));
  const T* kvb = reinterpret_cast<const T*>(wave == 0 ? a.k : a.v) + head * D;
  const __amdgpu_buffer_rsrc_t kvrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<T*>(kvb), static_cast<short>(tok_bytes), static_cast<int>(a.kv_tokens), 0x00020000);
  const LaneOff<D> lo = make_lane_offsets<D>(wave);
  const int kv_tokens = static_cast<int>(a.kv_tokens);
  T* ob = reinterpret_cast<T*>(a.o) + head * D;

  // this lane's query: row m of the window, frame qframe of the window's frames
  TT st;
  const int m = m0 + 32 * wave + c;
  const bool qvalid = m < lq;
  const int mm = qvalid ? m : 0;
  const int qframe = fdiv(mm, q_sp, 1.0f / static_cast<float>(q_sp));
  int64_t qflat;
  {
    const int r = mm - qframe * q_sp;
    const int hh = fdiv(r, qw_l, 1.0f / static_cast<float>(qw_l));
    const int ww = r - hh * qw_l;
    qflat = static_cast<int64_t>(q_t0 + qframe) * L + static_cast<int64_t>(q_h0 + hh) * a.W +
            (q_w0 + ww);
    qflat = qflat < 0 ? 0 : (qflat >= a.q_tokens ? a.q_tokens - 1 : qflat);
    const V8* qp = reinterpret_cast<const V8*>(qb + qflat * tok + hf * (D / 2));
    // Every lane loads (qflat is clamped in bounds): no exec branch between
    // the loads; lanes past the window's queries are zeroed after the load.
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) st.qf[ks] = qp[ks];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) st.qf[ks] = qvalid ? st.qf[ks] : V8{};
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) st.oacc[dt] = f32x16_t{};
    st.mrun = -INFINITY;
    st.lrun = 0.f;
  }

  const int sp_hr = kh_l * kw_l;
  const int sp_a = kh_l_a * kw_l_a;
  const KvRing ring = load_ring(a.ring_R, a.ring_nc, a.ring_head);
  const bool anchor_ok = kh_l_a > 0 && kw_l_a > 0 && h_a > 0 && w_a > 0;
  if (MODE == 0) {
    // anchor prefix (a_frames whole-chunk anchor frames), then the HR cuboid
    if (a_frames > 0 && anchor_ok) {
      KeyRun ar = make_run(a_frames * sp_a, 0, h_a * w_a, 0, kh0_a, kw0_a, kh_l_a, kw_l_a, w_a);
      attend_run<T, D>(st, ar, -1, wave, qframe, qvalid, kvrsrc, kv_tokens, a.scale_log2,
                       ksh, vsh, lo);
    }
    if (sp_hr > 0 && kv_tl > 0) {
      KeyRun hr = make_run(kv_tl * sp_hr, a.hr_base, L, kv_t0, kh0, kw0, kh_l, kw_l, a.W, ring);
      attend_run<T, D>(st, hr, -1, wave, qframe, qvalid, kvrsrc, kv_tokens, a.scale_log2,
                       ksh, vsh, lo);
    }
  } else {
    // per-frame anchor: query frame s sees anchor frame s only, over the
    // frames this tile holds; then the shared HR cuboid
    if (anchor_ok) {
      const int f_lo = m0 / q_sp;
      const int f_hi = (min(lq, m0 + 64) - 1) / q_sp;
      for (int s = f_lo; s <= f_hi; ++s) {
        KeyRun ar = make_run(sp_a, s * h_a * w_a, h_a * w_a, 0, kh0_a, kw0_a,
                             kh_l_a, kw_l_a, w_a);
        attend_run<T, D>(st, ar, s, wave, qframe, qvalid, kvrsrc, kv_tokens, a.scale_log2,
                         ksh, vsh, lo);
      }
    }
    if (sp_hr > 0 && kv_tl > 0) {
      KeyRun hr = make_run(kv_tl * sp_hr, a.hr_base, L, kv_t0, kh0, kw0, kh_l, kw_l, a.W, ring);
      attend_run<T, D>(st, hr, -1, wave, qframe, qvalid, kvrsrc, kv_tokens, a.scale_log2,
                       ksh, vsh, lo);
    }
  }

  // O = acc / l ; lane (c, hf) writes dims dt*32 + 8*g4 + 4*hf + [0, 4)
  const float lt = half_sum(st.lrun);
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  uint32_t am = 0;
  if (qvalid) {
    T* op = ob + qflat * tok;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const f32x2_t lo = {st.oacc[dt][g4 * 4 + 0] * inv, st.oacc[dt][g4 * 4 + 1] * inv};
        const f32x2_t hi = {st.oacc[dt][g4 * 4 + 2] * inv, st.oacc[dt][g4 * 4 + 3] * inv};
        const auto l = __builtin_convertvector(lo, typename E::h2);
        const auto u = __builtin_convertvector(hi, typename E::h2);
        const i32x2_t w = {__builtin_bit_cast(int, l), __builtin_bit_cast(int, u)};
        *reinterpret_cast<i32x2_t*>(op + dt * 32 + g4 * 8 + hf * 4) = w;
        if (a.amax_out) am = max(am, max(abs_bits2(l), abs_bits2(u)));
      }
  }
  if (a.amax_out) wave_amax_out(a.amax_out, am);
}

__global__ void clear_amax_kernel(uint32_t* p) { *p = 0u; }

template <typename T, int D>
int launch_window(const WinArgs& a, int mode, uint32_t grid, hipStream_t stream) {
  if (a.amax_out) {
    hipLaunchKernelGGL(clear_amax_kernel, dim3(1), dim3(1), 0, stream, a.amax_out);
    SRDIT_LAUNCH_CHECK("clear_amax_kernel");
  }
  if (mode == 0)
    hipLaunchKernelGGL((window_attn_kernel<T, D, 0>), dim3(grid), dim3(64 * WAVES), 0, stream, a);
  else
    hipLaunchKernelGGL((window_attn_kernel<T, D, 1>), dim3(grid), dim3(64 * WAVES), 0, stream, a);
  SRDIT_LAUNCH_CHECK("window_attn_kernel");
  return SRDIT_OK;
}

}  // namespace
}  // namespace srdit

namespace srdit {
namespace {

int window_entry(const char* fn, const void* q, const void* k, const void* v, void* o,
                 const int32_t* params, const int32_t* order, int n_w, int m_tiles, int p_stride,
                 int hr_base, int H, int W, int64_t q_tokens, int64_t kv_tokens, int n_heads,
                 int head_dim, float scale, int mode, int ring_R, int ring_nc,
                 const int32_t* ring_head, uint32_t* amax_out, int dtype, void* stream) {
  SRDIT_REQUIRE(q && k && v && o && params && order, "%s: null pointer", fn);
  SRDIT_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o),
                "%s: q/k/v/o must be 16-byte aligned", fn);
  SRDIT_REQUIRE(mode == 0 || mode == 1, "%s: mode must be 0 or 1, got %d", fn, mode);
  SRDIT_REQUIRE(p_stride == (mode == 0 ? 19 : 17),
                "%s: p_stride %d does not match mode %d", fn, p_stride, mode);
  SRDIT_REQUIRE(n_w >= 1 && m_tiles >= 1 && n_heads >= 1 && H >= 1 && W >= 1 && hr_base >= 0,
                "%s: bad sizes (n_w=%d m_tiles=%d n_heads=%d H=%d W=%d hr_base=%d)", fn,
                n_w, m_tiles, n_heads, H, W, hr_base);
  SRDIT_REQUIRE(q_tokens >= 1 && kv_tokens >= 1 && q_tokens < (1LL << 31) && kv_tokens < (1LL << 31),
                "%s: token counts out of range", fn);
  SRDIT_REQUIRE(static_cast<int64_t>(H) * W < (1LL << 22), "%s: grid too large", fn);
  SRDIT_REQUIRE(kv_tokens * n_heads * head_dim * 2 < (1LL << 31) && q_tokens < (1LL << 24),
                "%s: K/V must span fewer than 2^31 bytes and 2^24 tokens", fn);
  SRDIT_REQUIRE(static_cast<int64_t>(n_heads) * head_dim * 2 < (1LL << 14),
                "%s: token stride n_heads*head_dim*2 must be below 16384 bytes "
                "(structured-buffer stride)", fn);
  if (head_dim != 64 && head_dim != 128) {
    set_error("%s: head_dim %d unsupported (64 or 128)", fn, head_dim);
    return SRDIT_EUNSUPPORTED;
  }
  if (dtype != SRDIT_DTYPE_BF16 && dtype != SRDIT_DTYPE_FP16) {
    set_error("%s: dtype code %d unsupported", fn, dtype);
    return SRDIT_EUNSUPPORTED;
  }
  const int64_t grid64 = static_cast<int64_t>(n_w) * m_tiles * n_heads;
  SRDIT_REQUIRE(grid64 < (1LL << 31), "%s: too many tasks", fn);
  WinArgs a;
  a.q = q; a.k = k; a.v = v; a.o = o; a.params = params; a.order = order;
  a.n_w = n_w; a.m_tiles = m_tiles; a.p_stride = p_stride; a.hr_base = hr_base; a.H = H; a.W = W;
  a.q_tokens = q_tokens; a.kv_tokens = kv_tokens; a.n_heads = n_heads;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.ring_R = ring_R; a.ring_nc = ring_nc; a.ring_head = ring_head; a.amax_out = amax_out;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const uint32_t grid = static_cast<uint32_t>(grid64);
  if (dtype == SRDIT_DTYPE_BF16)
    return head_dim == 128 ? launch_window<__bf16, 128>(a, mode, grid, s)
                           : launch_window<__bf16, 64>(a, mode, grid, s);
  return head_dim == 128 ? launch_window<_Float16, 128>(a, mode, grid, s)
                         : launch_window<_Float16, 64>(a, mode, grid, s);
}

}  // namespace
}  // namespace srdit

extern "C" int srdit_window_attn_fwd(const void* q, const void* k, const void* v, void* o,
                                     const int32_t* params, const int32_t* order, int n_w,
                                     int m_tiles, int p_stride, int hr_base, int H, int W,
                                     int64_t q_tokens, int64_t kv_tokens, int n_heads,
                                     int head_dim, float scale, int mode, int dtype,
                                     void* stream) {
  return srdit::window_entry("srdit_window_attn_fwd", q, k, v, o, params, order, n_w, m_tiles,
                             p_stride, hr_base, H, W, q_tokens, kv_tokens, n_heads, head_dim,
                             scale, mode, 0, 0, nullptr, nullptr, dtype, stream);
}

extern "C" int srdit_window_attn_fwd_ex(const void* q, const void* k, const void* v, void* o,
                                        const int32_t* params, const int32_t* order, int n_w,
                                        int m_tiles, int p_stride, int hr_base, int H, int W,
                                        int64_t q_tokens, int64_t kv_tokens, int n_heads,
                                        int head_dim, float scale, int mode, int ring_frames,
                                        int ring_cached, const int32_t* ring_head,
                                        uint32_t* amax_out, int dtype, void* stream) {
  using namespace srdit;
  const char* fn = "srdit_window_attn_fwd_ex";
  if (ring_frames != 0) {
    SRDIT_REQUIRE(ring_head != nullptr, "%s: null ring_head", fn);
    SRDIT_REQUIRE(ring_frames >= 1 && ring_cached >= 0 && ring_cached <= ring_frames,
                  "%s: need 0 <= ring_cached <= ring_frames (got %d, %d)", fn, ring_cached,
                  ring_frames);
    SRDIT_REQUIRE(hr_base >= 0 && static_cast<int64_t>(hr_base) +
                      static_cast<int64_t>(ring_frames) * H * W <= kv_tokens,
                  "%s: kv_tokens %lld do not cover the anchor prefix and %d ring frames", fn,
                  static_cast<long long>(kv_tokens), ring_frames);
  }
  return window_entry(fn, q, k, v, o, params, order, n_w, m_tiles, p_stride, hr_base, H, W,
                      q_tokens, kv_tokens, n_heads, head_dim, scale, mode, ring_frames,
                      ring_cached, ring_head, amax_out, dtype, stream);
}
