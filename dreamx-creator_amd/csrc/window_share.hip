// Shared-fetch block-grid window attention forward for gfx950 (MI355X).
//
// Up to MEMBERS (2 or 4) 64-query members (a params row and an m-tile each)
// per workgroup of 2*MEMBERS wavefronts; wavefronts 2m and 2m+1 own queries
// [0, 32) and [32, 64) of member m.  The workgroup walks a host-built step schedule: in every step
// each active member consumes one 32-key unit (4 token rows x 8 token columns
// of one KV frame), and a unit that several members consume in the same step
// is fetched once for all of them.  Neighbouring windows of the block grid
// overlap in most of their units, so each K/V byte moved from L2 into LDS
// serves about twice as many queries as in a one-window workgroup.
//
// Record r (16 int32, host-built; a workgroup of n steps has n + 1): words 0-7
// up to four fill units issued at iteration r-2 (frame << 24 | token offset
// of the unit's first key in its frame, k_slot | v_slot << 8), words 8-11 one
// word per member for step r (k_slot | v_slot << 5 | valid rows << 10 | valid
// columns << 13; zero: idle), word 12 the number of fill units, word 13
// flags (zero).  A member's active steps form a prefix of the workgroup's steps
// (once idle it stays idle).  The eight 1 KB pieces (4 keys each) of a unit's
// K and of its V are split evenly over the wavefronts (wavefront w fetches
// pieces [w*P, w*P + P), P = 4 / MEMBERS), so the fill work of a step is
// spread over all of them.  LDS holds 5*MEMBERS slots of 8 KB that K and V
// tiles share: four members take all 160 KB of a CU, two members 80 KB (two
// workgroups per CU).
//
// Pipeline: the S^T MFMAs of step s run at iteration s-1 (beside the softmax
// of step s-1), the softmax and P.V of step s at iteration s.  Record r's fill
// list (the units of step r) is issued at iteration r-2; every iteration
// starts with a full wait and a barrier.  The host places units in LDS slots
// so that a fill never targets a slot read in the same or a later iteration.
// (Fills three steps ahead with counted waits measured slower: the extra
// control outweighed the latency it hid.)
//
// Numerics are those of the plain kernel (blockgrid_triton.py:184-278): masked
// keys never contribute, P rounded to the input dtype before P.V, fp32
// accumulation, O = acc / l.  As in the grouped kernel, Q is pre-scaled by
// scale*log2(e) and rounded once, the running max is subtracted inside the S
// MFMA and raised only on overflow of the row sum.  The order in which a
// member walks its keys differs from the reference's t-major order; the
// online softmax makes the result independent of it up to rounding.

#include "window_common.h"

namespace srdit {
namespace {

using namespace win;

struct ShareArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  const int32_t* params;    // [n_w, 19] plain rows
  const int32_t* groups;    // [n_groups, 8]: (row, m-tile) x 4; row -1: no member
  const int32_t* step_off;  // [n_groups + 1]
  const int32_t* steps;     // [total steps, 16]
  int n_w, n_groups, hr_base, H, W;
  int64_t q_tokens, kv_tokens;
  int n_heads;
  float scale_log2;
  int ring_R, ring_nc;
  const int32_t* ring_head;
  uint32_t* amax_out;
};

constexpr int SH_KEYS = 32;       // keys per unit
constexpr int SH_STEP_WORDS = 16;
// LDS slots of 8 KB, shared by K and V tiles: five per member.
constexpr int sh_slots(int members) { return 5 * members; }

__device__ __forceinline__ void sh_dma_x4(i32x4_t rsrc, uint32_t lds, int index, int offset) {
  const i32x2_t va = {index, offset};
  asm volatile("buffer_load_dwordx4 %0, %1, 0 idxen offen lds" ::"v"(va), "s"(rsrc), "{m0}"(lds)
               : "memory");
}

template <typename T, int MEMBERS>
__global__ __launch_bounds__(128 * MEMBERS) __attribute__((amdgpu_waves_per_eu(2, 2)))
void window_share_kernel(ShareArgs a) {
  constexpr int D = 128;
  constexpr int SH_SLOTS = sh_slots(MEMBERS);
  // 1 KB fill pieces (4 keys) of a unit's K (and of its V) per wavefront
  constexpr int PIECES = 4 / MEMBERS;
  using E = Elem<T>;
  using V8 = typename E::v8;
  constexpr int KS = D / 16;   // k-steps of the S^T MFMA over the head dim
  constexpr int DT = D / 32;   // 32-row tiles of O^T over the head dim
  constexpr int CPK = D / 8;   // 16-byte chunks per key row
  constexpr int BLK = SH_KEYS * D;
  constexpr int BLKB = BLK * static_cast<int>(sizeof(T));  // 8 KB
  __shared__ __attribute__((aligned(16))) T sh[SH_SLOTS * BLK];

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int member = wave >> 1, qhalf = wave & 1;
  const int lane = threadIdx.x & 63;
  const int c = lane & 31, hf = lane >> 5;

  const uint32_t task = xcd_task(blockIdx.x, gridDim.x);
  const int head = static_cast<int>(task / static_cast<uint32_t>(a.n_groups));
  const int gi = static_cast<int>(task % static_cast<uint32_t>(a.n_groups));
  if (head >= a.n_heads) return;
  static_assert(MEMBERS == 2 || MEMBERS == 4, "two or four members per workgroup");
  const int s_begin = a.step_off[gi];
  // n steps have n + 1 records (the last carries fills only)
  const int nsteps = a.step_off[gi + 1] - s_begin - 1;
  // The step table is read-only for the whole launch: read through the
  // constant address space, so the loads are scalar and not ordered against
  // the fills' memory clobbers.
  typedef __attribute__((address_space(4))) const int32_t cint32_t;
  cint32_t* rec0 = (cint32_t*)(a.steps + static_cast<int64_t>(s_begin) * SH_STEP_WORDS);

  // This wavefront's member and 32 queries.
  int my_row = a.groups[8 * static_cast<int64_t>(gi) + 2 * member];
  const int my_mt = a.groups[8 * static_cast<int64_t>(gi) + 2 * member + 1];
  my_row = my_row >= a.n_w ? -1 : my_row;
  const int32_t* pm = a.params + static_cast<int64_t>(my_row < 0 ? 0 : my_row) * 19;
  const int q_t0 = pm[0], q_tl = pm[1], q_h0 = pm[2], q_w0 = pm[3], qh_l = pm[4], qw_l = pm[5];
  const int q_sp = qh_l * qw_l;
  const int lq = q_tl * q_sp;
  const int m0 = 64 * my_mt;
  const bool has_member = my_row >= 0 && qh_l > 0 && qw_l > 0 && q_tl > 0 && m0 >= 0 && m0 < lq;

  const int L = a.H * a.W;
  const int64_t tok = static_cast<int64_t>(a.n_heads) * D;
  const int tok_bytes = static_cast<int>(tok) * static_cast<int>(sizeof(T));
  const int kv_tokens = static_cast<int>(a.kv_tokens);
  // K and V of this head as structured buffers (record = token).
  auto make_rsrc = [&](const void* base) __attribute__((always_inline)) -> i32x4_t {
    const uint64_t p = reinterpret_cast<uint64_t>(reinterpret_cast<const T*>(base) + head * D);
    return i32x4_t{static_cast<int>(static_cast<uint32_t>(p)),
                   static_cast<int>(static_cast<uint32_t>(p >> 32) |
                                    (static_cast<uint32_t>(tok_bytes) << 16)),
                   kv_tokens, 0x00020000};
  };
  const i32x4_t krsrc = make_rsrc(a.k), vrsrc = make_rsrc(a.v);
  const uint32_t sh_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sh));
  // Fill pieces of this wavefront: pieces PIECES*wave + p (keys 4*piece +
  // lane/16 of a unit), 16-byte chunk (lane % 16) of the key's LDS row,
  // fetched from the head-row chunk the row's swizzle puts there.
  int fill_k_off[PIECES], fill_v_off[PIECES], fill_tok[PIECES];
#pragma unroll
  for (int pc = 0; pc < PIECES; ++pc) {
    const int fkey = 4 * (PIECES * wave + pc) + (lane >> 4), fpos = lane & 15;
    fill_k_off[pc] = (fpos ^ swz_k<D>(fkey)) * 16;
    fill_v_off[pc] = (fpos ^ swz_v<D>(fkey)) * 16;
    fill_tok[pc] = (fkey >> 3) * a.W + (fkey & 7);  // key's token offset in the unit
  }
  const KvRing ring = load_ring(a.ring_R, a.ring_nc, a.ring_head);
  const LaneOff<D> lo = make_lane_offsets<D>(0);

  V8 qf[KS];
  f32x16_t oacc[DT];
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
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) oacc[dt] = f32x16_t{};
  }

  // ---- fills ----------------------------------------------------------------
  // A step record as this wavefront uses it: the fill words, their count and
  // its member's word, read by scalar loads issued together an iteration
  // before they are needed.
  struct StepRec {
    i32x8_t fill;
    int nf, flags;
  };
  typedef __attribute__((address_space(4))) const i32x8_t ci32x8_t;
  auto load_fills = [&](int r) __attribute__((always_inline)) -> StepRec {
    StepRec x;
    if (r <= nsteps) {  // uniform
      cint32_t* p = rec0 + static_cast<int64_t>(r) * SH_STEP_WORDS;
      x.fill = *reinterpret_cast<ci32x8_t*>(p);
      x.nf = p[12];
      x.flags = p[13];
    } else {
      x.fill = i32x8_t{};
      x.nf = 0;
      x.flags = 0;
    }
    return x;
  };
  auto load_word = [&](int st) __attribute__((always_inline)) -> int {
    return (st < nsteps && has_member) ? rec0[static_cast<int64_t>(st) * SH_STEP_WORDS + 8 + member]
                                       : 0;
  };
  // This wavefront's piece of every unit of a step, K and V.
  auto fill_step = [&](const StepRec& r) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (u < r.nf) {  // uniform
        const int wa = r.fill[2 * u];
        const int wb = r.fill[2 * u + 1];
        const int f = static_cast<int>(static_cast<uint32_t>(wa) >> 24);
        // logical KV frame -> ring slot, in scalar selects
        int pf = ring.head + f;
        pf = pf >= ring.R ? pf - ring.R : pf;
        pf = ring.R <= 0 ? f : (f < ring.nc ? pf : ring.R + (f - ring.nc));
        const int base = a.hr_base + pf * L + (wa & 0xFFFFFF);
        // slots clamped into the rings: a malformed table stays inside LDS
        const int ksl = min(wb & 0xFF, SH_SLOTS - 1), vsl = min((wb >> 8) & 0xFF, SH_SLOTS - 1);
#pragma unroll
        for (int pc = 0; pc < PIECES; ++pc) {
          // an index past kv_tokens reads zeros (buffer range check)
          const int t = base + fill_tok[pc];
          const int piece = (PIECES * wave + pc) * 1024;
          const uint32_t kd = sh_lds + static_cast<uint32_t>(ksl * BLKB + piece);
          const uint32_t vd = sh_lds + static_cast<uint32_t>(vsl * BLKB + piece);
          sh_dma_x4(krsrc, kd, t, fill_k_off[pc]);
          sh_dma_x4(vrsrc, vd, t, fill_v_off[pc]);
        }
      }
    }
  };
  auto w_active = [](int w) __attribute__((always_inline)) -> bool { return ((w >> 10) & 7) != 0; };

  // ---- compute --------------------------------------------------------------
  struct KOps { V8 f[KS]; };
  struct VOps { V8 t[2][DT]; };
  auto read_k = [&](int slot) __attribute__((always_inline)) -> KOps {
    slot = min(slot, SH_SLOTS - 1);
    const char* kb = reinterpret_cast<const char*>(sh) + slot * BLKB;
    KOps r;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) r.f[ks] = *reinterpret_cast<const V8*>(kb + lo.k[ks]);
    return r;
  };
  auto read_v = [&](int slot) __attribute__((always_inline)) -> VOps {
    slot = min(slot, SH_SLOTS - 1);
    const char* vb = reinterpret_cast<const char*>(sh) + slot * BLKB;
    VOps r;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        i32x2_t half[2];
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          const char* src = vb + (16 * kk + 8 * h2) * CPK * 16 + lo.v[dt];
          half[h2] = __builtin_bit_cast(
              i32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(const_cast<char*>(src))));
        }
        const i32x4_t vw = {half[0][0], half[0][1], half[1][0], half[1][1]};
        r.t[kk][dt] = __builtin_bit_cast(V8, vw);
      }
    }
    return r;
  };

  constexpr float PMAX = 4294967296.0f;  // 2^32
  float lrun = 0.f;
  float mrun = 0.f;
  bool minit = false;
  f32x16_t cneg = f32x16_t{};
  const typename E::h2 ones2 = {static_cast<T>(1.0f), static_cast<T>(1.0f)};

  auto s_mfma = [&](const KOps& kf) __attribute__((always_inline)) -> f32x16_t {
    f32x16_t acc = E::mma(kf.f[0], qf[0], cneg);
#pragma unroll
    for (int ks = 1; ks < KS; ++ks) acc = E::mma(kf.f[ks], qf[ks], acc);
    return acc;
  };
  // Keys of a unit cut by the grid edge: key k sits at row k/8, column k%8.
  auto mask_unit = [&](f32x16_t& sc, int nrows, int ncols) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = 8 * (r >> 2) + 4 * hf + (r & 3);
      if ((key >> 3) >= nrows || (key & 7) >= ncols) sc[r] = -INFINITY;
    }
  };
  auto row_max = [&](const f32x16_t& sc) __attribute__((always_inline)) -> float {
    float mx = __builtin_fmaxf(sc[0], sc[1]);
#pragma unroll
    for (int r = 2; r < 16; ++r) mx = __builtin_fmaxf(mx, sc[r]);
    return other_half_max(mx);
  };
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

  // Prologue: records 0 and 1 ("iterations -2, -1"), a full wait; S^T of step 0.
  int w_cur = load_word(0), w_1 = load_word(1);
  StepRec r_2;
  {
    const StepRec r0 = load_fills(0), r1 = load_fills(1);
    r_2 = load_fills(2);
    fill_step(r0);
    fill_step(r1);
  }
  fill_barrier();
  f32x16_t s_cur = f32x16_t{};
  if (w_active(w_cur)) s_cur = s_mfma(read_k(w_cur & 31));

  auto iteration = [&](int j) __attribute__((always_inline)) {
    fill_barrier();  // fills of steps <= j+1 landed; iteration j-1's LDS reads retired everywhere
    __builtin_amdgcn_s_setprio(1);
    fill_step(r_2);  // record j+2
    __builtin_amdgcn_s_setprio(0);
    const int w_next = w_1;
    // K of step j+1 (step j's own slot when the member idles in step j+1: the
    // scores are then never read).
    const KOps kf = read_k((w_active(w_next) ? w_next : w_cur) & 31);
    f32x16_t s_next;
    if (__builtin_expect(w_active(w_cur), 1)) {  // uniform
      const int nrows = (w_cur >> 10) & 7, ncols = (w_cur >> 13) & 15;
      if (__builtin_expect(nrows < 4 || ncols < 8, 0)) mask_unit(s_cur, nrows, ncols);
      const VOps vt = read_v((w_cur >> 5) & 31);
      if (__builtin_expect(!minit, 0)) {  // first active unit: m = its row max
        mrun = row_max(s_cur);
        mrun = mrun == -INFINITY ? 0.f : mrun;
        shift(s_cur, mrun);
        set_cneg();
        minit = true;
      }
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
    } else {
      s_next = s_cur;  // idle from here on: a member's active steps are a prefix
    }
    s_cur = s_next;
    w_cur = w_next;
    w_1 = load_word(j + 2);
    r_2 = load_fills(j + 3);  // waited for by the next iteration's barrier
  };
  // Unrolled by two, so the scores of consecutive steps alternate registers.
  int j = 0;
  for (; j + 1 < nsteps; j += 2) {
    iteration(j);
    iteration(j + 1);
  }
  if (j < nsteps) iteration(j);

  // O = acc / l ; lane (c, hf) writes dims dt*32 + 8*g4 + 4*hf + [0, 4) of its query
  const float lt = half_sum(lrun);
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  uint32_t am = 0;
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
}

__global__ void share_clear_amax_kernel(uint32_t* p) { *p = 0u; }

}  // namespace
}  // namespace srdit

extern "C" int srdit_window_attn_shared_fwd(
    const void* q, const void* k, const void* v, void* o, const int32_t* params,
    const int32_t* groups, const int32_t* step_off, const int32_t* steps, int n_w, int n_groups,
    int hr_base, int H, int W, int64_t q_tokens, int64_t kv_tokens, int n_heads, int head_dim,
    float scale, int ring_frames, int ring_cached, const int32_t* ring_head, uint32_t* amax_out,
    int members, int dtype, void* stream) {
  using namespace srdit;
  const char* fn = "srdit_window_attn_shared_fwd";
  SRDIT_REQUIRE(members == 2 || members == 4, "%s: members must be 2 or 4, got %d", fn, members);
  SRDIT_REQUIRE(q && k && v && o && params && groups && step_off && steps, "%s: null pointer", fn);
  SRDIT_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o),
                "%s: q/k/v/o must be 16-byte aligned", fn);
  SRDIT_REQUIRE(n_w >= 1 && n_groups >= 1 && n_heads >= 1 && H >= 1 && W >= 1 && hr_base >= 0,
                "%s: bad sizes (n_w=%d n_groups=%d n_heads=%d H=%d W=%d hr_base=%d)", fn, n_w,
                n_groups, n_heads, H, W, hr_base);
  SRDIT_REQUIRE(q_tokens >= 1 && kv_tokens >= 1 && q_tokens < (1LL << 24) &&
                    kv_tokens < (1LL << 31),
                "%s: token counts out of range", fn);
  SRDIT_REQUIRE(static_cast<int64_t>(H) * W < (1LL << 22), "%s: grid too large", fn);
  SRDIT_REQUIRE(kv_tokens * n_heads * head_dim * 2 < (1LL << 31),
                "%s: K/V must span fewer than 2^31 bytes", fn);
  SRDIT_REQUIRE(static_cast<int64_t>(n_heads) * head_dim * 2 < (1LL << 14),
                "%s: token stride n_heads*head_dim*2 must be below 16384 bytes", fn);
  SRDIT_REQUIRE(scale > 0.f && scale < 1e30f, "%s: softmax scale must be positive and finite", fn);
  if (ring_frames != 0) {
    SRDIT_REQUIRE(ring_head != nullptr, "%s: null ring_head", fn);
    SRDIT_REQUIRE(ring_frames >= 1 && ring_cached >= 0 && ring_cached <= ring_frames,
                  "%s: need 0 <= ring_cached <= ring_frames (got %d, %d)", fn, ring_cached,
                  ring_frames);
  }
  if (head_dim != 128) {
    set_error("%s: head_dim %d unsupported (128)", fn, head_dim);
    return SRDIT_EUNSUPPORTED;
  }
  if (dtype != SRDIT_DTYPE_BF16 && dtype != SRDIT_DTYPE_FP16) {
    set_error("%s: dtype code %d unsupported", fn, dtype);
    return SRDIT_EUNSUPPORTED;
  }
  const int64_t grid64 = static_cast<int64_t>(n_groups) * n_heads;
  SRDIT_REQUIRE(grid64 < (1LL << 31), "%s: too many tasks", fn);
  ShareArgs a;
  a.q = q; a.k = k; a.v = v; a.o = o; a.params = params; a.groups = groups;
  a.step_off = step_off; a.steps = steps;
  a.n_w = n_w; a.n_groups = n_groups; a.hr_base = hr_base; a.H = H; a.W = W;
  a.q_tokens = q_tokens; a.kv_tokens = kv_tokens; a.n_heads = n_heads;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.ring_R = ring_frames; a.ring_nc = ring_cached; a.ring_head = ring_head;
  a.amax_out = amax_out;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (amax_out) {
    hipLaunchKernelGGL(share_clear_amax_kernel, dim3(1), dim3(1), 0, s, amax_out);
    SRDIT_LAUNCH_CHECK("share_clear_amax_kernel");
  }
  const uint32_t grid = static_cast<uint32_t>(grid64);
  const dim3 block(128 * members);
  if (dtype == SRDIT_DTYPE_BF16) {
    if (members == 4)
      hipLaunchKernelGGL((window_share_kernel<__bf16, 4>), dim3(grid), block, 0, s, a);
    else
      hipLaunchKernelGGL((window_share_kernel<__bf16, 2>), dim3(grid), block, 0, s, a);
  } else {
    if (members == 4)
      hipLaunchKernelGGL((window_share_kernel<_Float16, 4>), dim3(grid), block, 0, s, a);
    else
      hipLaunchKernelGGL((window_share_kernel<_Float16, 2>), dim3(grid), block, 0, s, a);
  }
  SRDIT_LAUNCH_CHECK("window_share_kernel");
  return SRDIT_OK;
}
