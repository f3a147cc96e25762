// Grouped block-grid window attention forward for gfx950 (MI355X): plain-mode
// windows without an anchor prefix, two 64-query members per workgroup that
// share their K/V fetches, or one member per workgroup (MEMBERS = 1).
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
// frames to 3 or 4.  Fills run two steps ahead into rings (K two stages, V
// three) while the current step computes; in a private slot
// wavefronts 2m (K) and 2m+1 (V) fetch member m's block, in a shared slot
// wavefronts 0 (K) and 1 (V) fetch it.
//
// The one-member form (two wavefronts, 40 KB of LDS, four workgroups per CU)
// runs faster than pairs that share only part of their frames; pairs of the
// two m-tiles of one window (identical KV) run faster in the two-member form.
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
  int ring_R, ring_nc;       // in-place KV cache layout (ring_R == 0: plain)
  const int32_t* ring_head;  // device int32: ring slot of the oldest cached frame
  uint32_t* amax_out;        // max |O| bits, or null
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

// Per-wavefront fill cursor: the step it fetches next and, per lane, the
// row/column (within the spatial extent) of the key whose token the lane
// decodes for the row broadcast.  Advancing one step adds 32 keys:
// dq = 32 / kw_l rows and dr = 32 % kw_l columns, with one carry.
struct FillCursor {
  int fs, s;     // frame slot and spatial step of the next fill
  int row, col;  // per lane
  int fbase;     // token of (frame, kh0, kw0) for the current frame slot, -1: no frame
  bool part;     // this wavefront fetches in the current frame slot
  int blk;       // LDS byte offset of the slot's block within a stage
};

// AMODE: 0 plain rows without an anchor prefix; with one member per workgroup
// also 2, plain rows whose anchor prefix (a_frames whole-chunk anchor frames)
// every query sees, or 1, per-frame anchor rows (17 fields) where query frame
// s sees anchor frame s only.  The anchor frames are walked after the HR
// frames, as extra frame slots with the anchor grid's extent.
// PACK (one member, AMODE 0): a 64-row tile may hold the queries of two
// windows whose KV cuboids differ only in their columns (tile table rows of
// five: window A, A's first query, A's rows in the tile, window B or -1, B's
// first query).  The tile walks the union of the two column ranges, which the
// host makes exactly 32 tokens wide, so each 32-key step is one token row of
// the union and a key's column is its index in the step: every lane sets the
// scores of the columns outside its own window to -inf, from a 32-bit column
// set fixed for the whole walk.  A tile of one window (B = -1) walks that
// window.  A table whose union is not 32 wide gives wrong numbers, never an
// access outside the tensors (every token index is clamped).
// Two wavefronts per SIMD: the register budget is 256 per lane (the compiler
// would otherwise reach for accumulation registers and drop to one).
template <typename T, int D, int MEMBERS, int AMODE, bool PACK = false>
__global__ __launch_bounds__(128 * MEMBERS) __attribute__((amdgpu_waves_per_eu(2, 2)))
void window_group_kernel(GroupArgs a) {
  static_assert(AMODE == 0 || MEMBERS == 1, "anchors run one member per workgroup");
  static_assert(!PACK || (MEMBERS == 1 && AMODE == 0), "packed tiles run one plain member");
  constexpr int PST = AMODE == 1 ? 17 : 19;  // params row stride
  using E = Elem<T>;
  using V8 = typename E::v8;
  constexpr int KS = D / 16;      // k-steps of the S^T MFMA over the head dim
  constexpr int DT = D / 32;      // 32-row tiles of O^T over the head dim
  constexpr int NL = D / 16;      // fill loads (1 KB each) per block
  constexpr int CPK = D / 8;      // 16-byte chunks per key row
  constexpr int LPK = CPK;        // fill lanes per key row
  constexpr int KPI = 64 / CPK;   // key rows per fill load
  constexpr int BLK = GKN * D;    // elements per block
  constexpr int BLKB = BLK * static_cast<int>(sizeof(T));
  // [stage][block] rings: 2 stages x MEMBERS blocks x 32 keys x D, for K and for V
  __shared__ __attribute__((aligned(16))) T ksh[2 * MEMBERS * BLK];
  // The V ring has three stages and V is fetched two steps ahead, as K is:
  // 40 KB per member, so the one-member form still fits four workgroups and
  // the two-member form two workgroups in a CU's 160 KB.
  constexpr int VST = 3;
  __shared__ __attribute__((aligned(16))) T vsh[VST * MEMBERS * BLK];

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // kv_role 0: K, 1: V
  const int member = MEMBERS == 2 ? wave >> 1 : 0, qhalf = wave & 1, kv_role = wave & 1;
  const int lane = threadIdx.x & 63;
  const int c = lane & 31, hf = lane >> 5;

  const uint32_t task = xcd_task(blockIdx.x, gridDim.x);
  const int head = static_cast<int>(task / static_cast<uint32_t>(a.n_groups));
  const int gi = static_cast<int>(task % static_cast<uint32_t>(a.n_groups));
  if (head >= a.n_heads) return;
  const int32_t* gp = a.groups + (PACK ? 5 : 4) * static_cast<int64_t>(gi);
  int row0 = gp[0], mt0 = gp[1], row1 = PACK ? gp[3] : gp[2], mt1 = PACK ? 0 : gp[3];
  // PACK: A's rows in the tile (the rest are B's, from B's query pk_qb0 on)
  const int pk_na = PACK ? min(max(gp[2], 0), 64) : 64, pk_qb0 = PACK ? max(gp[4], 0) : 0;
  row0 = row0 < 0 ? 0 : (row0 >= a.n_w ? a.n_w - 1 : row0);
  row1 = ((MEMBERS == 1 && !PACK) || row1 < 0) ? -1 : (row1 >= a.n_w ? a.n_w - 1 : row1);
  const int32_t* p0 = a.params + static_cast<int64_t>(row0) * PST;
  const int32_t* p1 = row1 >= 0 ? a.params + static_cast<int64_t>(row1) * PST : p0;

  // Shared spatial KV extent (member 0's; the host pairs equal extents; a
  // packed tile of two windows walks the union of their columns) and the two
  // frame ranges.
  constexpr int F = AMODE == 1 ? -2 : 0;  // field offset of the HR cuboid in a 17-field row
  const int kh0 = p0[F + 8], kh_l = p0[F + 9];
  int kw0 = p0[F + 10], kw_l = p0[F + 11];
  if (PACK && row1 >= 0) {
    const int e0 = kw0 + kw_l, b0 = p1[F + 10], e1 = b0 + p1[F + 11];
    kw0 = min(kw0, b0);
    kw_l = max(e0, e1) - kw0;
  }
  const int sp = kh_l > 0 && kw_l > 0 ? kh_l * kw_l : 0;
  const int a0 = p0[F + 6], la = sp > 0 ? max(p0[F + 7], 0) : 0;
  const int a1 = p1[F + 6], lb = (!PACK && sp > 0 && row1 >= 0) ? max(p1[F + 7], 0) : 0;
  const int s_lo = max(a0, a1);
  const int nsh = lb > 0 ? max(0, min(a0 + la, a1 + lb) - s_lo) : 0;
  const PrivFrames pf0 = private_frames(a0, la, s_lo, nsh);
  const PrivFrames pf1 = lb > 0 ? private_frames(a1, lb, s_lo, nsh) : PrivFrames{0, 0, 0, 0};
  const PrivFrames pfm = member == 0 ? pf0 : pf1;
  const int P = max(la - nsh, lb > 0 ? lb - nsh : 0);
  const int nS = (sp + GKN - 1) / GKN;
  const int first_shared = P * nS;  // steps before it are private (one block per member)
  // This member's frame in slot fs_ (-1: none), without branches.
  auto frame_of = [&](int fs_) __attribute__((always_inline)) -> int {
    const int k2 = fs_ - pfm.len1;
    const int fpriv = fs_ < pfm.len1 ? pfm.lo1 + fs_ : (k2 < pfm.len2 ? pfm.lo2 + k2 : -1);
    return fs_ < P ? fpriv : (fs_ < P + nsh ? s_lo + (fs_ - P) : -1);
  };

  // This wavefront's 32 queries: rows m0 + 32*qhalf + [0, 32) of its member.
  const int my_row = member == 0 ? row0 : row1;
  const int my_mt = member == 0 ? mt0 : mt1;
  const int32_t* pm = member == 0 ? p0 : p1;
  int q_t0, q_tl, q_h0, q_w0, qh_l, qw_l;
  if constexpr (AMODE == 1) {
    q_t0 = 0; q_h0 = pm[0]; q_w0 = pm[1]; qh_l = pm[2]; qw_l = pm[3]; q_tl = pm[10];
  } else {
    q_t0 = pm[0]; q_tl = pm[1]; q_h0 = pm[2]; q_w0 = pm[3]; qh_l = pm[4]; qw_l = pm[5];
  }
  const int q_sp = qh_l * qw_l;
  const int lq = q_tl * q_sp;
  // PACK: A's rows start at its query mt0 (not an m-tile); B's query geometry
  const int m0 = PACK ? mt0 : 64 * my_mt;
  const bool has_member = my_row >= 0 && qh_l > 0 && qw_l > 0 && q_tl > 0 && m0 >= 0 && m0 < lq;
  // B's query geometry is read where it is used (the prologue's Q fills and
  // the epilogue's O stores) through an opaque copy of its row pointer, so it
  // is not held in registers across the walk: the kernel sits at its register
  // limit.
  struct QGeo {
    int t0, h0, w0, hl, wl, lq;
  };
  // One read per call site group (the prologue, the epilogue), none for a
  // tile of one window.
  auto b_geo = [&]() __attribute__((always_inline)) -> QGeo {
    QGeo g{0, 0, 0, 1, 1, 0};
    if (PACK && row1 >= 0) {  // uniform
      const int32_t* pb = p1;
      asm volatile("" : "+s"(pb));
      g.t0 = pb[0]; g.h0 = pb[2]; g.w0 = pb[3];
      g.hl = max(pb[4], 1); g.wl = max(pb[5], 1);
      g.lq = max(pb[1], 0) * pb[4] * pb[5];
    }
    return g;
  };

  // Anchor slots (AMODE 1, 2): n_anc frames of the anchor grid h_a x w_a over
  // the extent (kh0_a, kh_l_a, kw0_a, kw_l_a), after the HR slots.  AMODE 1
  // walks the anchor frames f_lo .. f_lo + n_anc - 1 of this tile's query
  // frames, each admitted to that frame's queries only.
  int n_anc = 0, kh0_a = 0, kh_l_a = 0, kw0_a = 0, kw_l_a = 0, h_a = 0, w_a = 0, f_lo = 0;
  if constexpr (AMODE != 0) {
    const int* pa = pm + (AMODE == 1 ? 11 : 13);
    kh0_a = pa[0]; kh_l_a = pa[1]; kw0_a = pa[2]; kw_l_a = pa[3]; h_a = pa[4]; w_a = pa[5];
    const bool anchor_ok = kh_l_a > 0 && kw_l_a > 0 && h_a > 0 && w_a > 0 && has_member;
    if (AMODE == 1) {
      f_lo = q_sp > 0 ? m0 / q_sp : 0;
      const int f_hi = q_sp > 0 ? (min(lq, m0 + 64) - 1) / q_sp : -1;
      n_anc = anchor_ok ? f_hi - f_lo + 1 : 0;
    } else {
      n_anc = anchor_ok ? max(pm[12], 0) : 0;
    }
  }
  const int sp_a = kh_l_a * kw_l_a;
  const int nS_a = (sp_a + GKN - 1) / GKN;
  const int nslots = P + nsh + n_anc;
  const int nsteps = (P + nsh) * nS + n_anc * nS_a;
  // Slots this member consumes a block in, bit fs (the host limits a window
  // to 16 KV frames, so a pair has at most 32 slots).
  uint32_t act = 0;
  if (has_member) {
    for (int fs_ = 0; fs_ < nslots && fs_ < 32; ++fs_)
      if (fs_ >= P + nsh || frame_of(fs_) >= 0) act |= 1u << fs_;
  }
  auto active = [&](int fs_) __attribute__((always_inline)) -> bool {
    return ((act >> (fs_ & 31)) & 1u) != 0 && fs_ < 32;
  };

  const int L = a.H * a.W;
  const int64_t tok = static_cast<int64_t>(a.n_heads) * D;
  const int tok_bytes = static_cast<int>(tok) * static_cast<int>(sizeof(T));
  const int kv_tokens = static_cast<int>(a.kv_tokens);
  // K (even wavefronts) or V (odd) of this head as a structured buffer
  // (record = token, stride = token stride in bytes): base, base_hi |
  // stride << 16, num_records, flags.
  const uint64_t kva = reinterpret_cast<uint64_t>(reinterpret_cast<const T*>(kv_role == 0 ? a.k : a.v) +
                                                  head * D);
  const i32x4_t kvrsrc = {static_cast<int>(static_cast<uint32_t>(kva)),
                          static_cast<int>(static_cast<uint32_t>(kva >> 32) |
                                           (static_cast<uint32_t>(tok_bytes) << 16)),
                          kv_tokens, 0x00020000};
  const uint32_t lds_fill_base =
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>(kv_role == 0 ? ksh : vsh));
  const LaneOff<D> lo = make_lane_offsets<D>(kv_role);

  V8 qf[KS];
  f32x16_t oacc[DT];
  // Row r (0..31) of this wavefront's 32 queries: tile row 32*qhalf + r, which
  // is query m0 + tile row of the window (PACK: of window A below pk_na rows,
  // else query pk_qb0 + (tile row - pk_na) of window B).
  auto in_b = [&](int r) __attribute__((always_inline)) -> bool {
    return PACK && 32 * qhalf + r >= pk_na;
  };
  auto row_ok_g = [&](int r, const QGeo& gb) __attribute__((always_inline)) -> bool {
    if (in_b(r)) return row1 >= 0 && pk_qb0 + 32 * qhalf + r - pk_na < gb.lq;
    return has_member && m0 + 32 * qhalf + r < lq && (!PACK || 32 * qhalf + r < pk_na);
  };
  auto row_ok = [&](int r) __attribute__((always_inline)) -> bool {
    if constexpr (PACK) return row_ok_g(r, b_geo());
    return row_ok_g(r, QGeo{0, 0, 0, 1, 1, 0});
  };
  const bool qvalid = row_ok(c);
  const int m = m0 + 32 * qhalf + c;  // this lane's query (the anchored forms)
  // Token of row r, clamped into Q (gb: window B's geometry, PACK only).
  auto row_token_g = [&](int r, const QGeo& gb) __attribute__((always_inline)) -> int {
    const bool b = in_b(r);
    const int mr = b ? pk_qb0 + 32 * qhalf + r - pk_na : m0 + 32 * qhalf + r;
    const int mm = row_ok_g(r, gb) ? mr : 0;
    const int hl = b ? gb.hl : qh_l, wl = b ? gb.wl : qw_l;
    const int qs = hl * wl > 0 ? hl * wl : 1, qw = wl > 0 ? wl : 1;
    const int fr = fdiv(mm, qs, 1.0f / static_cast<float>(qs));
    const int rr = mm - fr * qs;
    const int hh = fdiv(rr, qw, 1.0f / static_cast<float>(qw));
    const int ww = rr - hh * qw;
    const int t = ((b ? gb.t0 : q_t0) + fr) * L + ((b ? gb.h0 : q_h0) + hh) * a.W +
                  ((b ? gb.w0 : q_w0) + ww);
    return t < 0 ? 0 : (t >= a.q_tokens ? static_cast<int>(a.q_tokens) - 1 : t);
  };
  auto row_token = [&](int r) __attribute__((always_inline)) -> int {
    if constexpr (PACK) return row_token_g(r, b_geo());
    return row_token_g(r, QGeo{0, 0, 0, 1, 1, 0});
  };
  int qframe;  // this lane's query frame within the window
  // The anchored forms (AMODE 1, 2) sit at the register limit: they load Q
  // straight into registers and store O from them, each lane its own query's
  // row.  The plain form stages both through LDS (the prologue and epilogue).
  int64_t qflat = 0;
  {
    const int mm = qvalid ? m : 0;
    const int qs = q_sp > 0 ? q_sp : 1, qw = qw_l > 0 ? qw_l : 1;
    const int fr = fdiv(mm, qs, 1.0f / static_cast<float>(qs));
    qframe = fr;
    if constexpr (AMODE != 0) {
      const int r = mm - fr * q_sp;
      const int hh = fdiv(r, qw, 1.0f / static_cast<float>(qw));
      const int ww = r - hh * qw_l;
      qflat = static_cast<int64_t>(q_t0 + fr) * L + static_cast<int64_t>(q_h0 + hh) * a.W +
              (q_w0 + ww);
      qflat = qflat < 0 ? 0 : (qflat >= a.q_tokens ? a.q_tokens - 1 : qflat);
      const V8* qp = reinterpret_cast<const V8*>(reinterpret_cast<const T*>(a.q) + head * D +
                                                 qflat * tok + hf * (D / 2));
      // Q enters the S^T MFMA pre-scaled by scale*log2(e) (rounded once to T), so
      // the scores come out in log2 units; lanes past the window's queries hold 0.
      V8 raw[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) raw[ks] = qp[ks];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        float x[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = qvalid ? static_cast<float>(raw[ks][i]) * a.scale_log2 : 0.f;
        qf[ks] = E::pack8(x);
      }
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) oacc[dt] = f32x16_t{};
  }

  // ---- fills ----------------------------------------------------------------
  // Step t goes to K stage t % 2 and V stage t % VST.  In a private step block
  // b holds member b's keys and is fetched by wavefronts 2b (K) and 2b+1 (V);
  // in a shared step block 0 is fetched by wavefronts 0 and 1.  K and V are
  // fetched two steps ahead of their use.
  // Source lane s of a 16-lane row decodes the
  // token of the key that load (s % LPK) places in that row; DPP row_newbcast
  // hands it to the row.
  const int s16 = lane & 15;
  const int src_key = (s16 % LPK) * KPI + (lane >> 4) * (16 / LPK) + s16 / LPK;
  const int sub = s16 / LPK;
  // Walk of a rows x cols extent (row stride rs tokens) 32 keys per step: the
  // lane's first (row, col), the per-step advance dq rows + dr columns, the
  // last key of the extent (frame-relative) and the steps per frame.
  struct Walk {
    int rows, rs, kwl, dq, dr, row_start, col_start, last_tok, nS;
  };
  auto make_walk = [&](int rows, int cols, int rs) __attribute__((always_inline)) -> Walk {
    Walk g;
    g.rows = rows; g.rs = rs;
    g.kwl = cols > 0 ? cols : 1;
    g.dq = GKN / g.kwl; g.dr = GKN - g.dq * g.kwl;
    g.row_start = fdiv(src_key, g.kwl, 1.0f / static_cast<float>(g.kwl));
    g.col_start = src_key - g.row_start * g.kwl;
    g.last_tok = (rows - 1) * rs + (cols - 1);
    g.nS = (rows * cols + GKN - 1) / GKN;
    return g;
  };
  const Walk hr_walk = make_walk(kh_l, kw_l, a.W);
  const int frame0_tok = a.hr_base + kh0 * a.W + kw0;
  const KvRing ring = load_ring(a.ring_R, a.ring_nc, a.ring_head);
  auto fbase_of = [&](int fs_) __attribute__((always_inline)) -> int {
    if (AMODE != 0 && fs_ >= P + nsh) {  // anchor frame: no HR base, no ring
      const int af = (AMODE == 1 ? f_lo : 0) + (fs_ - P - nsh);
      return af * h_a * w_a + kh0_a * w_a + kw0_a;
    }
    const int f = frame_of(fs_);
    return f >= 0 ? frame0_tok + ring_frame(ring, f) * L : -1;
  };
  FillCursor cur;
  Walk cw = hr_walk;  // the cursor's current extent
  // Per-slot state of the cursor, refreshed when it enters a frame slot.
  auto cursor_slot = [&]() __attribute__((always_inline)) {
    const bool priv = cur.fs < P;
    if (AMODE != 0 && cur.fs == P + nsh) cw = make_walk(kh_l_a, kw_l_a, w_a);
    cur.fbase = fbase_of(cur.fs);
    cur.part = (priv || member == 0) && cur.fbase >= 0;
    cur.blk = priv ? member * BLKB : 0;
  };
  cur.fs = 0; cur.s = 0; cur.row = cw.row_start; cur.col = cw.col_start;
  cursor_slot();
  constexpr int look = 2;  // steps ahead the fills run
  // Fetch the cursor's step into stage `stage` and advance.
  auto fill_next = [&](int stage) __attribute__((always_inline)) {
    if (__builtin_expect(cur.part, 1)) {  // uniform
      int t = cur.row < cw.rows ? __mul24(cur.row, cw.rs) + cur.col : cw.last_tok;
      t += cur.fbase;
      t = static_cast<int>(min(static_cast<uint32_t>(t), static_cast<uint32_t>(kv_tokens - 1)));
      const uint32_t dst = lds_fill_base + static_cast<uint32_t>(stage * MEMBERS * BLKB + cur.blk);
      static_for<NL>([&](auto qc) __attribute__((always_inline)) {
        constexpr int q = decltype(qc)::value;
        int tq = __builtin_amdgcn_mov_dpp(t, 0x150 + q, 0xf, 0xf, false);
        if constexpr (LPK == 8) {
          const int t1 = __builtin_amdgcn_mov_dpp(t, 0x150 + 8 + q, 0xf, 0xf, false);
          tq = sub ? t1 : tq;
        }
        dma_x4(kvrsrc, dst + q * 1024, tq, lo.fill[q]);
      });
    }
    if (__builtin_expect(++cur.s == cw.nS, 0)) {  // uniform: next frame slot
      cur.s = 0;
      ++cur.fs;
      cursor_slot();
      cur.row = cw.row_start;
      cur.col = cw.col_start;
    } else {
      cur.row += cw.dq;
      cur.col += cw.dr;
      const bool carry = cur.col >= cw.kwl;
      cur.col -= carry ? cw.kwl : 0;
      cur.row += carry ? 1 : 0;
    }
  };

  // ---- compute --------------------------------------------------------------
  // Iteration j issues the S^T MFMAs of step j+1 and then the softmax and P.V
  // of step j, so the matrix core works on step j+1 while the vector ALU
  // exponentiates step j.  ka/va are this wavefront's LDS lane offsets of the
  // K block of step j+1 and the V block of step j (the member's own block in
  // private steps, block 0 in shared ones); stages are immediates.
  auto blk_off = [&](int t) __attribute__((always_inline)) -> int {
    return (t < first_shared && member == 1) ? BLKB : 0;
  };
  int ka[KS], va[DT];
  int koff = blk_off(0), voff = blk_off(0);
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) ka[ks] = lo.k[ks] + koff;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) va[dt] = lo.v[dt] + voff;

  struct KOps { V8 f[KS]; };
  struct VOps { V8 t[2][DT]; };
  auto read_k = [&](auto stage_c) __attribute__((always_inline)) -> KOps {
    constexpr int stage = decltype(stage_c)::value;
    const char* kb = reinterpret_cast<const char*>(ksh) + stage * MEMBERS * BLKB;
    KOps r;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) r.f[ks] = *reinterpret_cast<const V8*>(kb + ka[ks]);
    return r;
  };
  auto read_v = [&](auto stage_c) __attribute__((always_inline)) -> VOps {
    constexpr int stage = decltype(stage_c)::value;
    const char* vb = reinterpret_cast<const char*>(vsh) + stage * MEMBERS * BLKB;
    VOps r;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        i32x2_t half[2];
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          const char* src = vb + (16 * kk + 8 * h2) * CPK * 16 + va[dt];
          half[h2] = __builtin_bit_cast(
              i32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(const_cast<char*>(src))));
        }
        const i32x4_t vw = {half[0][0], half[0][1], half[1][0], half[1][1]};
        r.t[kk][dt] = __builtin_bit_cast(V8, vw);
      }
    }
    return r;
  };

  // Softmax state.  The running max m (log2 units) is subtracted inside the
  // S^T MFMA: its C input holds -m in every slot, so the MFMA yields s - m.
  // m is set from the first active block and raised only when a block's P
  // would pass PMAX (its row sum exceeds PMAX, or is not finite); between
  // raises P = exp2(s - m) <= PMAX, which the final O = acc / l cancels.
  constexpr float PMAX = 4294967296.0f;  // 2^32
  float lrun = 0.f;        // this lane's half of the row sum
  float mrun = 0.f;        // running max, valid once minit
  bool minit = false;      // wave-uniform: m has been set
  // PACK, two windows: this lane's window's columns [mlo, mhi) of the 32-wide
  // union, as a 32-bit set of the columns outside it.  S^T entry r holds key
  // 8*(r/4) + 4*hf + r%4 of the step, i.e. that column; mask_cols sets the
  // entries of outside columns to -inf after the S^T MFMAs of every step.
  uint32_t colmask = 0;
  if (PACK && row1 >= 0) {
    const bool b = in_b(c);
    const int mlo = (b ? p1[F + 10] : p0[F + 10]) - kw0;
    const int mhi = mlo + (b ? p1[F + 11] : p0[F + 11]);
    const uint32_t lo_bits = mlo <= 0 ? 0u : (mlo >= 32 ? ~0u : ((1u << mlo) - 1u));
    const uint32_t hi_bits = mhi >= 32 ? 0u : (mhi <= 0 ? ~0u : ~((1u << mhi) - 1u));
    colmask = lo_bits | hi_bits;
  }
  auto mask_cols = [&](f32x16_t& sc) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = 8 * (r >> 2) + 4 * hf + (r & 3);
      if ((colmask >> key) & 1u) sc[r] = -INFINITY;
    }
  };
  f32x16_t cneg = f32x16_t{};
  const typename E::h2 ones2 = {static_cast<T>(1.0f), static_cast<T>(1.0f)};

  auto s_mfma = [&](const KOps& kf) __attribute__((always_inline)) -> f32x16_t {
    f32x16_t acc = E::mma(kf.f[0], qf[0], cneg);
#pragma unroll
    for (int ks = 1; ks < KS; ++ks) acc = E::mma(kf.f[ks], qf[ks], acc);
    return acc;
  };
  // Partial last block of a frame: keys >= nvalid never contribute.
  auto mask_tail = [&](f32x16_t& sc, int nvalid) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = 8 * (r >> 2) + 4 * hf + (r & 3);
      if (key >= nvalid) sc[r] = -INFINITY;
    }
  };
  auto row_max = [&](const f32x16_t& sc) __attribute__((always_inline)) -> float {
    float mx = __builtin_fmaxf(sc[0], sc[1]);
#pragma unroll
    for (int r = 2; r < 16; ++r) mx = __builtin_fmaxf(mx, sc[r]);
    return other_half_max(mx);  // both key halves of the query
  };
  // P = exp2(sc) rounded to T, and the sum of the rounded values (the ones
  // P.V uses), two per dot2.  Each packed word is copied to a scalar before
  // its bit cast: clang casts element 0 for a bit cast of a vector element
  // with a loop index.
  auto exp_pack = [&](const f32x16_t& sc, V8& pa, V8& pb) __attribute__((always_inline)) -> float {
    float pv[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) pv[r] = __builtin_amdgcn_exp2f(sc[r]);
    pa = E::pack8(&pv[0]);
    pb = E::pack8(&pv[8]);
    const i32x4_t wa = __builtin_bit_cast(i32x4_t, pa), wb = __builtin_bit_cast(i32x4_t, pb);
    float ps = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int w = wa[i];
      ps = E::dot2(__builtin_bit_cast(typename E::h2, w), ones2, ps);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int w = wb[i];
      ps = E::dot2(__builtin_bit_cast(typename E::h2, w), ones2, ps);
    }
    return ps;
  };
  auto shift = [&](f32x16_t& sc, float d) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 16; ++r) sc[r] -= d;
  };
  auto set_cneg = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 16; ++r) cneg[r] = -mrun;
  };
  auto pv_mfma = [&](const VOps& vt, const V8& pa, const V8& pb) __attribute__((always_inline)) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) oacc[dt] = E::mma(vt.t[0][dt], pa, oacc[dt]);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) oacc[dt] = E::mma(vt.t[1][dt], pb, oacc[dt]);
  };

  // Slots this wavefront computes: the member's, less (AMODE 1) the anchor
  // frames none of its valid queries is admitted to.  Such a slot would add
  // exp2(-inf) = 0 to every row, so its softmax, P.V and S^T MFMAs are
  // skipped; the fills go on (both wavefronts share them).
  uint32_t wact = act;
  if constexpr (AMODE == 1) {
    for (int k = 0; k < n_anc; ++k) {
      const int fs_ = P + nsh + k;
      if (fs_ < 32 && !__any(qvalid && qframe == f_lo + k)) wact &= ~(1u << fs_);
    }
  }
  auto wactive = [&](int fs_) __attribute__((always_inline)) -> bool {
    return ((wact >> (fs_ & 31)) & 1u) != 0 && fs_ < 32;
  };

  // Prologue.  Each wavefront stages its 32 query rows into its own 8 KB of the
  // V ring's stages 1 and 2 with the fill DMA: whole 256-byte rows per 16 lanes
  // in the K tile layout (row r, chunk L at slot L ^ swz_k(r)), so the loads are
  // full cache lines and the reads below are the K operand's conflict-free
  // pattern.  K of steps 0 and 1 and V of step 0 land with it; V of step 1
  // follows once every wavefront has read its Q.  Then the S^T of step 0.
  constexpr int CPKQ = D / 8, LPKQ = CPKQ, KPIQ = 64 / CPKQ;
  const uint32_t qreg = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(vsh)) +
                        static_cast<uint32_t>((MEMBERS + wave) * BLKB);
  if constexpr (AMODE == 0) {
    const uint64_t qa = reinterpret_cast<uint64_t>(reinterpret_cast<const T*>(a.q) + head * D);
    const i32x4_t qrsrc = {static_cast<int>(static_cast<uint32_t>(qa)),
                           static_cast<int>(static_cast<uint32_t>(qa >> 32) |
                                            (static_cast<uint32_t>(tok_bytes) << 16)),
                           static_cast<int>(a.q_tokens), 0x00020000};
    const int pos = lane % CPKQ, sub_q = (lane & 15) / LPKQ;
    const QGeo gb = b_geo();
    static_for<NL>([&](auto qc) __attribute__((always_inline)) {
      constexpr int qi = decltype(qc)::value;
      const int r = qi * KPIQ + (lane >> 4) * (16 / LPKQ) + sub_q;
      dma_x4(qrsrc, qreg + qi * 1024, row_token_g(r, gb), (pos ^ swz_k<D>(r)) * 16);
    });
  }
  if (nsteps > 0) fill_next(0);
  if (nsteps > 1 && (AMODE != 0 || kv_role == 0)) fill_next(1);
  fill_barrier();
  if constexpr (AMODE == 0) {
    // Q enters the S^T MFMA pre-scaled by scale*log2(e) (rounded once to T), so
    // the scores come out in log2 units; lanes past the window's queries hold 0.
    const char* qb = reinterpret_cast<const char*>(vsh) + (MEMBERS + wave) * BLKB;
    V8 raw[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) raw[ks] = *reinterpret_cast<const V8*>(qb + lo.k[ks]);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      float x[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = qvalid ? static_cast<float>(raw[ks][i]) * a.scale_log2 : 0.f;
      qf[ks] = E::pack8(x);
    }
  }
  if constexpr (AMODE == 0) {
    fill_barrier();  // every wavefront has its Q: V stage 1 is free
    if (nsteps > 1 && kv_role == 1) fill_next(1);
  }
  f32x16_t s_cur = f32x16_t{};
  if (nsteps > 0 && wactive(0)) s_cur = s_mfma(read_k(std::integral_constant<int, 0>{}));

  int fs = 0, s = 0;  // frame slot and spatial step of step j
  bool do_pv = nsteps > 0 && wactive(0);  // this wavefront consumes step j
  int nS_c = nS;                               // steps per frame of step j's slot
  int tail_valid = sp - (nS - 1) * GKN;        // keys of that frame's last block
  bool admit = true;  // AMODE 1 anchor slots: this lane's query frame is the slot's
  auto iteration = [&](int j, auto stage_c, auto vstage_c) __attribute__((always_inline)) {
    constexpr int stage = decltype(stage_c)::value;    // K stage of step j: j % 2
    constexpr int vstage = decltype(vstage_c)::value;  // V stage of step j: j % VST
    fill_barrier();  // K of j+1 and V of j landed; iteration j-1's LDS reads retired everywhere
    // Step j+2: K into stage j % 2, V into stage (j+2) % 3.  Both were last
    // read in iteration j-1, which every wavefront has finished.
    // The fill is issued at wave priority 1, so the DMA of step j+2 leaves ahead
    // of the other wavefront's MFMA and softmax issue on the SIMD (A/B: equal to
    // 4% faster on c3, the shipped geometry and dense cross-attention).
    __builtin_amdgcn_s_setprio(1);
    if (j + look < nsteps) fill_next(kv_role == 0 ? stage : (vstage + 2) % VST);
    __builtin_amdgcn_s_setprio(0);
    // private -> shared: the K block of step j+1 and the V block of step j
    // move to block 0 (once each; member 1 only)
    if (__builtin_expect(j + 1 == first_shared && member == 1, 0)) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) ka[ks] -= BLKB;
    }
    if (__builtin_expect(j == first_shared && member == 1 && j > 0, 0)) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) va[dt] -= BLKB;
    }
    // The S^T MFMAs of step j+1 run with the softmax of an active step j (on a
    // stale block when the wavefront skips step j+1: that result is never
    // consumed), and otherwise only when step j+1 starts a computed slot.
    const KOps kf = read_k(std::integral_constant<int, stage ^ 1>{});
    f32x16_t s_next;
    if (__builtin_expect(do_pv, 1)) {  // uniform
      if (__builtin_expect(s == nS_c - 1 && tail_valid < GKN, 0)) mask_tail(s_cur, tail_valid);
      if (PACK && row1 >= 0) mask_cols(s_cur);  // uniform
      if (AMODE == 1 && __builtin_expect(fs >= P + nsh, 0)) {
#pragma unroll
        for (int r = 0; r < 16; ++r) s_cur[r] = admit ? s_cur[r] : -INFINITY;
      }
      const VOps vt = read_v(std::integral_constant<int, vstage>{});
      if (__builtin_expect(!minit, 0)) {  // first active block: m = its row max
        mrun = row_max(s_cur);
        mrun = mrun == -INFINITY ? 0.f : mrun;  // a lane the block does not admit
        shift(s_cur, mrun);
        set_cneg();
        minit = true;
      }
      // S^T MFMAs of step j+1 interleaved with the exponentials of step j,
      // then P.V of step j interleaved with the conversions and row sums.
      s_next = s_mfma(kf);
      V8 pa, pb;
      float ps = exp_pack(s_cur, pa, pb);
      if (__builtin_expect(__any(!(ps <= PMAX)), 0)) {  // raise m (rare)
        const float d = fmaxf(row_max(s_cur), 0.f);
        const float alpha = __builtin_amdgcn_exp2f(-d);
        lrun *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) oacc[dt] *= alpha;
        mrun += d;
        set_cneg();
        shift(s_cur, d);
        shift(s_next, d);  // issued with the old m
        ps = exp_pack(s_cur, pa, pb);
      }
      lrun += ps;
      pv_mfma(vt, pa, pb);
      static_for<KS>([&](auto) __attribute__((always_inline)) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // three VALU
      });
      static_for<2 * DT>([&](auto) __attribute__((always_inline)) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);
      });
    } else if ((s + 1 == nS_c) && wactive(fs + 1)) {  // uniform: step j+1 starts a computed slot
      s_next = s_mfma(kf);
    } else {
      s_next = s_cur;  // step j+1 is skipped too: its scores are never read
    }
    s_cur = s_next;
    if (__builtin_expect(++s == nS_c, 0)) {  // uniform: next frame slot
      s = 0;
      ++fs;
      do_pv = wactive(fs);
      if (AMODE != 0 && fs >= P + nsh && n_anc > 0) {  // anchor slots: the anchor extent
        nS_c = nS_a;
        tail_valid = sp_a - (nS_a - 1) * GKN;
        admit = AMODE != 1 || qframe == f_lo + (fs - P - nsh);
      }
    }
  };
  // Unrolled by 6 so that both ring stages (j % 2, j % 3) are immediates.
  static_assert(VST == 3, "the unrolling below assumes a three-stage V ring");
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  int j = 0;
  for (; j + 5 < nsteps; j += 6) {
    iteration(j, I0{}, I0{});
    iteration(j + 1, I1{}, I1{});
    iteration(j + 2, I0{}, I2{});
    iteration(j + 3, I1{}, I0{});
    iteration(j + 4, I0{}, I1{});
    iteration(j + 5, I1{}, I2{});
  }
  if (j < nsteps) iteration(j, I0{}, I0{});  // j % 6 == 0 here
  if (j + 1 < nsteps) iteration(j + 1, I1{}, I1{});
  if (j + 2 < nsteps) iteration(j + 2, I0{}, I2{});
  if (j + 3 < nsteps) iteration(j + 3, I1{}, I0{});
  if (j + 4 < nsteps) iteration(j + 4, I0{}, I1{});

  // O = acc / l, staged through this wavefront's 8 KB of the V ring in the Q
  // layout (lane (c, hf) holds dims dt*32 + 8*g4 + 4*hf + [0, 4) of query c),
  // then written out as whole 256-byte rows, 16 lanes per row.
  const float lt = half_sum(lrun);
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  uint32_t am = 0;
  if constexpr (AMODE != 0) {
    if (qvalid) {
      T* op = reinterpret_cast<T*>(a.o) + head * D + qflat * tok;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const f32x2_t lo2 = {oacc[dt][g4 * 4 + 0] * inv, oacc[dt][g4 * 4 + 1] * inv};
          const f32x2_t hi2 = {oacc[dt][g4 * 4 + 2] * inv, oacc[dt][g4 * 4 + 3] * inv};
          const auto l = __builtin_convertvector(lo2, typename E::h2);
          const auto u = __builtin_convertvector(hi2, typename E::h2);
          const i32x2_t w = {__builtin_bit_cast(int, l), __builtin_bit_cast(int, u)};
          *reinterpret_cast<i32x2_t*>(op + dt * 32 + g4 * 8 + hf * 4) = w;
          if (a.amax_out) am = max(am, max(abs_bits2(l), abs_bits2(u)));
        }
    }
    if (a.amax_out) wave_amax_out(a.amax_out, am);
    return;
  }
  fill_barrier();  // every wavefront is done with the ring
  char* ob = reinterpret_cast<char*>(vsh) + (MEMBERS + wave) * BLKB;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const f32x2_t lo2 = {oacc[dt][g4 * 4 + 0] * inv, oacc[dt][g4 * 4 + 1] * inv};
      const f32x2_t hi2 = {oacc[dt][g4 * 4 + 2] * inv, oacc[dt][g4 * 4 + 3] * inv};
      const auto l = __builtin_convertvector(lo2, typename E::h2);
      const auto u = __builtin_convertvector(hi2, typename E::h2);
      const i32x2_t w = {__builtin_bit_cast(int, l), __builtin_bit_cast(int, u)};
      const int chunk = dt * 4 + g4;
      *reinterpret_cast<i32x2_t*>(ob + (c * CPKQ + (chunk ^ swz_k<D>(c))) * 16 + hf * 8) = w;
      if (a.amax_out && qvalid) am = max(am, max(abs_bits2(l), abs_bits2(u)));
    }
  compiler_fence();
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wavefront's LDS writes done
  compiler_fence();
  {
    const int pos = lane % CPKQ, sub_q = (lane & 15) / LPKQ;
    const QGeo gb = b_geo();
#pragma unroll
    for (int qi = 0; qi < NL; ++qi) {
      const int r = qi * KPIQ + (lane >> 4) * (16 / LPKQ) + sub_q;
      const i32x4_t v = *reinterpret_cast<const i32x4_t*>(ob + (r * CPKQ + (pos ^ swz_k<D>(r))) * 16);
      if (row_ok_g(r, gb)) {
        T* op = reinterpret_cast<T*>(a.o) + head * D + static_cast<int64_t>(row_token_g(r, gb)) * tok +
                pos * 8;
        *reinterpret_cast<i32x4_t*>(op) = v;
      }
    }
  }
  if (a.amax_out) wave_amax_out(a.amax_out, am);
}

__global__ void clear_amax_kernel(uint32_t* p) { *p = 0u; }

template <typename T, int D>
int launch_group(const GroupArgs& a, int members, int amode, uint32_t grid, hipStream_t stream,
                 bool pack = false) {
  if (a.amax_out) {
    hipLaunchKernelGGL(clear_amax_kernel, dim3(1), dim3(1), 0, stream, a.amax_out);
    SRDIT_LAUNCH_CHECK("clear_amax_kernel");
  }
  if (pack)
    hipLaunchKernelGGL((window_group_kernel<T, D, 1, 0, true>), dim3(grid), dim3(128), 0, stream, a);
  else if (amode == 1)
    hipLaunchKernelGGL((window_group_kernel<T, D, 1, 1>), dim3(grid), dim3(128), 0, stream, a);
  else if (amode == 2)
    hipLaunchKernelGGL((window_group_kernel<T, D, 1, 2>), dim3(grid), dim3(128), 0, stream, a);
  else if (members == 1)
    hipLaunchKernelGGL((window_group_kernel<T, D, 1, 0>), dim3(grid), dim3(128), 0, stream, a);
  else
    hipLaunchKernelGGL((window_group_kernel<T, D, 2, 0>), dim3(grid), dim3(256), 0, stream, a);
  SRDIT_LAUNCH_CHECK("window_group_kernel");
  return SRDIT_OK;
}

}  // namespace
}  // namespace srdit

namespace srdit {
namespace {

int group_entry(const char* fn, const void* q, const void* k, const void* v, void* o,
                const int32_t* params, const int32_t* groups, int n_w, int n_groups, int hr_base,
                int H, int W, int64_t q_tokens, int64_t kv_tokens, int n_heads, int head_dim,
                float scale, int ring_R, int ring_nc, const int32_t* ring_head,
                uint32_t* amax_out, int members, int amode, int dtype, void* stream,
                bool pack = false) {
  SRDIT_REQUIRE(q && k && v && o && params && groups, "%s: null pointer", fn);
  SRDIT_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o),
                "%s: q/k/v/o must be 16-byte aligned", fn);
  SRDIT_REQUIRE(n_w >= 1 && n_groups >= 1 && n_heads >= 1 && H >= 1 && W >= 1 && hr_base >= 0,
                "%s: bad sizes (n_w=%d n_groups=%d n_heads=%d H=%d W=%d "
                "hr_base=%d)", fn, n_w, n_groups, n_heads, H, W, hr_base);
  SRDIT_REQUIRE(q_tokens >= 1 && kv_tokens >= 1 && q_tokens < (1LL << 24),
                "%s: token counts out of range", fn);
  SRDIT_REQUIRE(static_cast<int64_t>(H) * W < (1LL << 22), "%s: grid too large", fn);
  SRDIT_REQUIRE(kv_tokens * n_heads * head_dim * 2 < (1LL << 31),
                "%s: K/V must span fewer than 2^31 bytes", fn);
  // Q and O are read and written through structured buffers too
  SRDIT_REQUIRE(q_tokens * n_heads * head_dim * 2 < (1LL << 31),
                "%s: Q/O must span fewer than 2^31 bytes", fn);
  SRDIT_REQUIRE(static_cast<int64_t>(n_heads) * head_dim * 2 < (1LL << 14),
                "%s: token stride n_heads*head_dim*2 must be below 16384 "
                "bytes (structured-buffer stride)", fn);
  SRDIT_REQUIRE(scale > 0.f && scale < 1e30f,
                "%s: softmax scale must be positive and finite", fn);
  if (head_dim != 64 && head_dim != 128) {
    set_error("%s: head_dim %d unsupported (64 or 128)", fn, head_dim);
    return SRDIT_EUNSUPPORTED;
  }
  if (dtype != SRDIT_DTYPE_BF16 && dtype != SRDIT_DTYPE_FP16) {
    set_error("%s: dtype code %d unsupported", fn, dtype);
    return SRDIT_EUNSUPPORTED;
  }
  const int64_t grid64 = static_cast<int64_t>(n_groups) * n_heads;
  SRDIT_REQUIRE(grid64 < (1LL << 31), "%s: too many tasks", fn);
  GroupArgs a;
  a.q = q; a.k = k; a.v = v; a.o = o; a.params = params; a.groups = groups;
  a.n_w = n_w; a.n_groups = n_groups; a.hr_base = hr_base; a.H = H; a.W = W;
  a.q_tokens = q_tokens; a.kv_tokens = kv_tokens; a.n_heads = n_heads;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.ring_R = ring_R; a.ring_nc = ring_nc; a.ring_head = ring_head; a.amax_out = amax_out;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const uint32_t grid = static_cast<uint32_t>(grid64);
  SRDIT_REQUIRE(members == 1 || members == 2, "%s: members must be 1 or 2, got %d", fn, members);
  SRDIT_REQUIRE(amode >= 0 && amode <= 2 && (amode == 0 || members == 1),
                "%s: anchor mode %d (0 none, 1 per frame, 2 whole chunk) needs one member per "
                "workgroup", fn, amode);
  SRDIT_REQUIRE(!pack || (members == 1 && amode == 0),
                "%s: packed tiles run one plain member per workgroup", fn);
  if (dtype == SRDIT_DTYPE_BF16)
    return head_dim == 128 ? launch_group<__bf16, 128>(a, members, amode, grid, s, pack)
                           : launch_group<__bf16, 64>(a, members, amode, grid, s, pack);
  return head_dim == 128 ? launch_group<_Float16, 128>(a, members, amode, grid, s, pack)
                         : launch_group<_Float16, 64>(a, members, amode, grid, s, pack);
}

}  // namespace
}  // namespace srdit

extern "C" int srdit_window_attn_grouped_fwd(const void* q, const void* k, const void* v, void* o,
                                             const int32_t* params, const int32_t* groups,
                                             int n_w, int n_groups, int hr_base, int H, int W,
                                             int64_t q_tokens, int64_t kv_tokens, int n_heads,
                                             int head_dim, float scale, int dtype, void* stream) {
  return srdit::group_entry("srdit_window_attn_grouped_fwd", q, k, v, o, params, groups, n_w,
                            n_groups, hr_base, H, W, q_tokens, kv_tokens, n_heads, head_dim,
                            scale, 0, 0, nullptr, nullptr, 2, 0, dtype, stream);
}

extern "C" int srdit_window_attn_grouped_fwd_ex(const void* q, const void* k, const void* v,
                                                void* o, const int32_t* params,
                                                const int32_t* groups, int n_w, int n_groups,
                                                int hr_base, int H, int W, int64_t q_tokens,
                                                int64_t kv_tokens, int n_heads, int head_dim,
                                                float scale, int ring_frames, int ring_cached,
                                                const int32_t* ring_head, uint32_t* amax_out,
                                                int members, int anchor_mode, int dtype,
                                                void* stream) {
  using namespace srdit;
  const char* fn = "srdit_window_attn_grouped_fwd_ex";
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
  return group_entry(fn, q, k, v, o, params, groups, n_w, n_groups, hr_base, H, W, q_tokens,
                     kv_tokens, n_heads, head_dim, scale, ring_frames, ring_cached, ring_head,
                     amax_out, members, anchor_mode, dtype, stream);
}

extern "C" int srdit_window_attn_packed_fwd(const void* q, const void* k, const void* v, void* o,
                                            const int32_t* params, const int32_t* tiles,
                                            int n_w, int n_tiles, int hr_base, int H, int W,
                                            int64_t q_tokens, int64_t kv_tokens, int n_heads,
                                            int head_dim, float scale, int ring_frames,
                                            int ring_cached, const int32_t* ring_head,
                                            uint32_t* amax_out, int dtype, void* stream) {
  using namespace srdit;
  const char* fn = "srdit_window_attn_packed_fwd";
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
  return group_entry(fn, q, k, v, o, params, tiles, n_w, n_tiles, hr_base, H, W, q_tokens,
                     kv_tokens, n_heads, head_dim, scale, ring_frames, ring_cached, ring_head,
                     amax_out, 1, 0, dtype, stream, true);
}
