// Dense attention over a short context for gfx950 (MI355X): every query of a
// head attends every key of that head.  This is the refiner's cross-attention
// over the text tokens (WanT2VCrossAttention.forward, models.py:1042-1062:
// q from the video tokens, k and v from the context, softmax(q k^T d^-1/2) v).
//
// Persistent workgroups of four wavefronts, two per CU.  A task is 128
// consecutive queries of one head (32 per wavefront); each workgroup walks a
// range of tasks, and the keys of a task stream through LDS 32 at a time, as in
// the window kernels: K two steps ahead and V one step ahead, each into a
// two-stage ring.  A task's step count is rounded up to even (a step past the
// keys is fully masked), so ring stages are fixed per step parity and the
// loop unrolls by two with immediate stages.  The fill stream runs on across
// task boundaries, so the next task's first keys are in flight while a task
// ends.
//
// What makes it persistent is the query side.  A workgroup that starts, loads
// its queries and stores its outputs once leaves the CU idle while its queries
// arrive; with every workgroup in step that was a third of a 512-key launch.
// Here wavefronts 0 and 1 issue the K and V fills, and wavefronts 2 and 3
// prefetch the queries of the next task into LDS while the current task runs.
// Their only wait on that prefetch is at the next task's start, because they
// issue no fills and so never wait on the vector-memory counter at the
// per-step barrier.  Outputs go through LDS and leave as whole 128-byte row
// pieces, stored by wavefronts 2 and 3 only (a fixed count per task: rows past
// the queries fall outside the store descriptor), so wavefronts 0 and 1 have
// nothing but fills to wait for.
//
// Numerics are those of the window kernels: q pre-scaled by scale * log2(e)
// and rounded to the input type, base-2 softmax with the running max
// subtracted inside the S^T MFMA and raised only when a block's P would pass
// 2^32, P rounded to the input type before P.V, fp32 accumulation, O = acc / l.

#include "window_common.h"

namespace srdit {
namespace {

using namespace win;

struct DenseArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  int q_tokens, kv_tokens, n_heads;
  int tiles;    // query tiles of DQT per head
  int n_tasks;  // n_heads * tiles
  float scale_log2;
  uint32_t* amax_out;  // max |O| bits, or null
};

constexpr int DKN = 32;   // keys per step
constexpr int DQT = 128;  // queries per task: four wavefronts of 32

template <int N>
__device__ __forceinline__ void vm_wait_lgkm() {
  waitcnt_vm_keep<N>();  // vmcnt(N) lgkmcnt(0)
}

template <typename T, int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void dense_attn_kernel(DenseArgs a) {
  using E = Elem<T>;
  using V8 = typename E::v8;
  constexpr int KS = D / 16;   // k-steps of the S^T MFMA over the head dim
  constexpr int DT = D / 32;   // 32-row tiles of O^T over the head dim
  constexpr int NL = D / 16;   // 1 KB fill loads per block of 32 rows
  constexpr int CPK = D / 8;   // 16-byte chunks per row
  constexpr int LPK = CPK;     // fill lanes per row
  constexpr int KPI = 64 / CPK;  // rows per fill load
  constexpr int BLK = DKN * D;
  constexpr int BLKB = BLK * static_cast<int>(sizeof(T));
  constexpr int OH = D / 64;   // 64-dim halves of the output staged through LDS
  constexpr int NST = 8 * OH;  // output stores of wavefronts 2 and 3 per task
  __shared__ __attribute__((aligned(16))) T ksh[2 * BLK];
  __shared__ __attribute__((aligned(16))) T vsh[2 * BLK];
  __shared__ __attribute__((aligned(16))) T qsh[4 * BLK];  // 32 query rows per wavefront
  __shared__ __attribute__((aligned(16))) T ostg[DQT * 64];  // 128 output rows x 64 dims

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int c = lane & 31, hf = lane >> 5;
  const bool filler = wave < 2;  // wavefront 0 fetches K, wavefront 1 V
  const int role = wave & 1;

  // This workgroup's tasks: XCD x owns one contiguous range of the task list
  // (head-major, so a head's tasks share that XCD's L2), walked by its
  // workgroups with a stride of their count.
  const uint32_t n_tasks = static_cast<uint32_t>(a.n_tasks);
  const uint32_t xcd = blockIdx.x & 7u, wslot = blockIdx.x >> 3, per = gridDim.x >> 3;
  const uint32_t r0 = xcd * (n_tasks >> 3) + min(xcd, n_tasks & 7u);
  const uint32_t r1 = r0 + (n_tasks >> 3) + (xcd < (n_tasks & 7u) ? 1u : 0u);
  const int my_tasks = (r0 + wslot < r1) ? static_cast<int>((r1 - r0 - wslot + per - 1) / per) : 0;
  if (my_tasks == 0) return;
  auto task_of = [&](int t) __attribute__((always_inline)) -> int {
    return static_cast<int>(r0 + wslot + per * static_cast<uint32_t>(t));
  };
  int nsteps = (a.kv_tokens + DKN - 1) / DKN;
  nsteps += nsteps & 1;                 // even: the last step may hold no key
  const int total = my_tasks * nsteps;  // steps of the whole walk
  const int tok_bytes = a.n_heads * D * static_cast<int>(sizeof(T));

  // Structured buffer over one head's slice: record = token (stride = the
  // token stride in bytes), nrec records.
  auto srd = [&](const void* base, int head, int nrec) __attribute__((always_inline)) -> i32x4_t {
    const uint64_t p = reinterpret_cast<uint64_t>(static_cast<const T*>(base) +
                                                  static_cast<int64_t>(head) * D);
    return i32x4_t{static_cast<int>(static_cast<uint32_t>(p)),
                   static_cast<int>(static_cast<uint32_t>(p >> 32) |
                                    (static_cast<uint32_t>(tok_bytes) << 16)),
                   nrec, 0x00020000};
  };
  const LaneOff<D> lo = make_lane_offsets<D>(role);
  // Row of the 32-row block that load q of this lane fills: q * KPI + key_lane.
  const int key_lane = (lane >> 4) * (16 / LPK) + (lane & 15) / LPK;

  // ---- fills (wavefronts 0 and 1) -------------------------------------------
  // Global step G of the walk is key block G % nsteps of task G / nsteps; its
  // K and V go to stage G % 2 of their rings.  Wavefront 0 fetches K two steps
  // ahead, wavefront 1 V one step ahead; each wavefront's cursor walks the
  // steps of its own ring.
  int f_t = 0, f_j = 0;
  i32x4_t f_rsrc = srd(role == 0 ? a.k : a.v, task_of(0) / a.tiles, a.kv_tokens);
  const uint32_t k_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(ksh));
  const uint32_t v_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(vsh));
  auto fill_next = [&](uint32_t dst) __attribute__((always_inline)) {
    const int base = f_j * DKN + key_lane;
    static_for<NL>([&](auto qc) __attribute__((always_inline)) {
      constexpr int q = decltype(qc)::value;
      const int tok = min(base + q * KPI, a.kv_tokens - 1);
      dma_x4(f_rsrc, dst + q * 1024, tok, lo.fill[q]);
    });
    if (++f_j == nsteps) {
      f_j = 0;
      if (++f_t < my_tasks) f_rsrc = srd(role == 0 ? a.k : a.v, task_of(f_t) / a.tiles, a.kv_tokens);
    }
  };
  auto fill_stage = [&](int stage) __attribute__((always_inline)) {
    fill_next((role == 0 ? k_lds : v_lds) + static_cast<uint32_t>(stage * BLKB));
  };

  // ---- query prefetch (wavefronts 2 and 3) ----------------------------------
  // Rows of wavefront w's 32 queries of task t into its 8 KB of qsh, in the K
  // tile layout (row r, chunk L at slot L ^ swz_k(r)); wavefront 2 loads the
  // rows of wavefronts 0 and 1, wavefront 3 those of 2 and 3.
  const uint32_t q_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(qsh));
  auto q_prefetch = [&](int t) __attribute__((always_inline)) {
    const int task = task_of(t);
    const int q0 = (task % a.tiles) * DQT;
    const i32x4_t qr = srd(a.q, task / a.tiles, a.q_tokens);
    const int pos = lane % CPK;
#pragma unroll
    for (int w2 = 0; w2 < 2; ++w2) {
      const int wr = 2 * (wave - 2) + w2;
      static_for<NL>([&](auto qc) __attribute__((always_inline)) {
        constexpr int qi = decltype(qc)::value;
        const int r = qi * KPI + key_lane;
        const int tok = min(q0 + 32 * wr + r, a.q_tokens - 1);
        dma_x4(qr, q_lds + static_cast<uint32_t>(wr * BLKB + qi * 1024), tok,
               (pos ^ swz_k<D>(r)) * 16);
      });
    }
  };

  // ---- compute ---------------------------------------------------------------
  struct KOps { V8 f[KS]; };
  struct VOps { V8 t[2][DT]; };
  auto read_k = [&](auto stage_c) __attribute__((always_inline)) -> KOps {
    constexpr int stage = decltype(stage_c)::value;
    const char* kb = reinterpret_cast<const char*>(ksh) + stage * BLKB;
    KOps r;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) r.f[ks] = *reinterpret_cast<const V8*>(kb + lo.k[ks]);
    return r;
  };
  auto read_v = [&](auto stage_c) __attribute__((always_inline)) -> VOps {
    constexpr int stage = decltype(stage_c)::value;
    const char* vb = reinterpret_cast<const char*>(vsh) + stage * BLKB;
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

  V8 qf[KS];
  f32x16_t oacc[DT];
  constexpr float PMAX = 4294967296.0f;  // 2^32
  float lrun = 0.f, mrun = 0.f;
  bool minit = false;
  f32x16_t cneg = f32x16_t{};
  const typename E::h2 ones2 = {static_cast<T>(1.0f), static_cast<T>(1.0f)};

  auto s_mfma = [&](const KOps& kf) __attribute__((always_inline)) -> f32x16_t {
    f32x16_t acc = E::mma(kf.f[0], qf[0], cneg);
#pragma unroll
    for (int ks = 1; ks < KS; ++ks) acc = E::mma(kf.f[ks], qf[ks], acc);
    return acc;
  };
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

  // The barrier of every step G.  Wavefronts 0 and 1 first wait for the fill
  // they issued one step ago (K of step G + 1, V of step G; they issue
  // nothing else), wavefronts 2 and 3 only for their LDS reads.
  auto step_barrier = [&]() __attribute__((always_inline)) {
    compiler_fence();
    if (filler) {
      vm_wait_lgkm<0>();
    } else {
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    }
    __builtin_amdgcn_s_barrier();
    compiler_fence();
  };

  // Prologue: K of steps 0 and 1, V of step 0, the queries of the first task.
  if (filler) {
    fill_stage(0);
    if (role == 0) fill_stage(1);  // total >= 2: nsteps is even
  } else {
    q_prefetch(0);
  }

  uint32_t am = 0;
  f32x16_t s_cur = f32x16_t{};
  int G = 0;
  for (int t = 0; t < my_tasks; ++t) {
    const int task = task_of(t);
    const int head = task / a.tiles;
    const int q0 = (task % a.tiles) * DQT;
    // ---- task start: this task's queries, the K and the V of its first step
    // (G) landed.  Newer than K of step G: K of step G + 1 (always issued:
    // the task has at least two steps); than V of step G: nothing; than the
    // query prefetch of wavefronts 2 and 3: the previous task's output stores.
    compiler_fence();
    if (filler) {
      if (role == 0) vm_wait_lgkm<NL>(); else vm_wait_lgkm<0>();
    } else {
      if (t == 0) vm_wait_lgkm<0>(); else vm_wait_lgkm<NST>();
    }
    __builtin_amdgcn_s_barrier();
    compiler_fence();
    const int my_q = q0 + 32 * wave + c;  // this lane's query
    const bool qvalid = my_q < a.q_tokens;
    {
      const char* qb = reinterpret_cast<const char*>(qsh) + wave * BLKB;
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
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) oacc[dt] = f32x16_t{};
    lrun = 0.f;
    mrun = 0.f;
    minit = false;
    cneg = f32x16_t{};
    s_cur = s_mfma(read_k(std::integral_constant<int, 0>{}));  // G is even
    // Once every wavefront has read its queries, the next task's go into the
    // same LDS (issued here, outside the step loop, so that its addresses do
    // not hold registers across the loop).
    compiler_fence();
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    compiler_fence();
    if (!filler && t + 1 < my_tasks) q_prefetch(t + 1);

    // Step j of the task (global step G, G % 2 == j % 2): scores of step
    // j + 1 with the softmax and P.V of step j.
    auto iteration = [&](int j, auto stage_c) __attribute__((always_inline)) {
      constexpr int stage = decltype(stage_c)::value;  // G % 2
      step_barrier();
      if (filler) {
        // K of step G + 2 into K stage G % 2 (read in step G - 1), V of step
        // G + 1 into V stage (G + 1) % 2 (read in step G - 1)
        __builtin_amdgcn_s_setprio(1);
        if (G + 2 - role < total) fill_stage(role == 0 ? stage : stage ^ 1);
        __builtin_amdgcn_s_setprio(0);
      }
      const bool more = j + 1 < nsteps;  // uniform
      if (__builtin_expect(DKN * (j + 1) > a.kv_tokens, 0)) mask_tail(s_cur, a.kv_tokens - DKN * j);
      const VOps vt = read_v(std::integral_constant<int, stage>{});
      if (__builtin_expect(!minit, 0)) {  // first block: m = its row max
        mrun = row_max(s_cur);
        mrun = mrun == -INFINITY ? 0.f : mrun;
        shift(s_cur, mrun);
        set_cneg();
        minit = true;
      }
      f32x16_t s_next = s_cur;
      if (__builtin_expect(more, 1)) s_next = s_mfma(read_k(std::integral_constant<int, stage ^ 1>{}));
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
      s_cur = s_next;
    };
    for (int j = 0; j < nsteps; j += 2) {
      iteration(j, std::integral_constant<int, 0>{});
      ++G;
      iteration(j + 1, std::integral_constant<int, 1>{});
      ++G;
    }

    // ---- epilogue: O = acc / l through LDS, 64 head dims at a time.  Every
    // wavefront writes its 32 rows (lane (c, hf) holds dims dt*32 + 8*g4 +
    // 4*hf + [0, 4) of query c) into ostg, row r of the 128 at 128 r bytes with
    // 16-byte chunk L at slot L ^ (r & 7); then wavefronts 2 and 3 store rows
    // [0, 64) and [64, 128) as whole 128-byte pieces, 8 rows per instruction.
    // Rows past the queries get an offset outside the store descriptor.
    const float lt = half_sum(lrun);
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
    const __amdgpu_buffer_rsrc_t orsrc = __builtin_amdgcn_make_buffer_rsrc(
        static_cast<void*>(static_cast<T*>(a.o) + static_cast<int64_t>(head) * D),
        static_cast<short>(0), (a.q_tokens - 1) * tok_bytes + D * static_cast<int>(sizeof(T)),
        0x00020000);
    char* const stg = reinterpret_cast<char*>(ostg);
    // lane-derived values are recomputed here, not held across the step loop
    int lane_e = lane;
    asm volatile("" : "+v"(lane_e));
    const int c_e = lane_e & 31, hf_e = lane_e >> 5;
#pragma unroll
    for (int h = 0; h < OH; ++h) {
      const int r = 32 * wave + c_e;
#pragma unroll
      for (int d2 = 0; d2 < 2; ++d2)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int dt = 2 * h + d2;
          const f32x2_t lo2 = {oacc[dt][g4 * 4 + 0] * inv, oacc[dt][g4 * 4 + 1] * inv};
          const f32x2_t hi2 = {oacc[dt][g4 * 4 + 2] * inv, oacc[dt][g4 * 4 + 3] * inv};
          const auto l = __builtin_convertvector(lo2, typename E::h2);
          const auto u = __builtin_convertvector(hi2, typename E::h2);
          const i32x2_t w = {__builtin_bit_cast(int, l), __builtin_bit_cast(int, u)};
          *reinterpret_cast<i32x2_t*>(stg + r * 128 + (((4 * d2 + g4) ^ (r & 7)) * 16) + 8 * hf_e) = w;
          const uint32_t m = max(abs_bits2(l), abs_bits2(u));
          am = qvalid ? max(am, m) : am;
        }
      compiler_fence();
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wavefront's rows are in LDS
      __builtin_amdgcn_s_barrier();
      compiler_fence();
      if (!filler) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int rr = 64 * (wave - 2) + 8 * i + (lane_e >> 3), L = lane_e & 7;
          const i32x4_t dv = *reinterpret_cast<const i32x4_t*>(stg + rr * 128 + ((L ^ (rr & 7)) * 16));
          const int qi = q0 + rr;
          const int off = qi < a.q_tokens
                              ? qi * tok_bytes + (64 * h + 8 * L) * static_cast<int>(sizeof(T))
                              : static_cast<int>(0x80000000);
          __builtin_amdgcn_raw_buffer_store_b128(dv, orsrc, off, 0, 0);
        }
      }
      compiler_fence();
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the staged rows are read
      __builtin_amdgcn_s_barrier();
      compiler_fence();
    }
  }
  if (a.amax_out) wave_amax_out(a.amax_out, am);
}

__global__ void clear_dense_amax_kernel(uint32_t* p) { *p = 0u; }

template <typename T, int D>
int launch_dense(const DenseArgs& a, uint32_t grid, hipStream_t stream) {
  if (a.amax_out) {
    hipLaunchKernelGGL(clear_dense_amax_kernel, dim3(1), dim3(1), 0, stream, a.amax_out);
    SRDIT_LAUNCH_CHECK("clear_dense_amax_kernel");
  }
  hipLaunchKernelGGL((dense_attn_kernel<T, D>), dim3(grid), dim3(256), 0, stream, a);
  SRDIT_LAUNCH_CHECK("dense_attn_kernel");
  return SRDIT_OK;
}

int cu_count() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;
  return n;
}

}  // namespace
}  // namespace srdit

extern "C" int srdit_dense_attn_fwd(const void* q, const void* k, const void* v, void* o,
                                    int64_t q_tokens, int64_t kv_tokens, int n_heads,
                                    int head_dim, float scale, uint32_t* amax_out, int dtype,
                                    void* stream) {
  using namespace srdit;
  const char* fn = "srdit_dense_attn_fwd";
  SRDIT_REQUIRE(q && k && v && o, "%s: null pointer", fn);
  SRDIT_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o),
                "%s: q/k/v/o must be 16-byte aligned", fn);
  SRDIT_REQUIRE(q_tokens >= 1 && kv_tokens >= 1 && n_heads >= 1,
                "%s: need q_tokens, kv_tokens and n_heads >= 1", fn);
  SRDIT_REQUIRE(static_cast<int64_t>(n_heads) * head_dim * 2 < (1LL << 14),
                "%s: token stride n_heads*head_dim*2 must be below 16384 bytes "
                "(structured-buffer stride)", fn);
  SRDIT_REQUIRE(q_tokens * n_heads * head_dim * 2 < (1LL << 31) &&
                    kv_tokens * n_heads * head_dim * 2 < (1LL << 31),
                "%s: Q/O and K/V must each span fewer than 2^31 bytes", fn);
  SRDIT_REQUIRE(scale > 0.f && scale < 1e30f, "%s: softmax scale must be positive and finite", fn);
  if (head_dim != 64 && head_dim != 128) {
    set_error("%s: head_dim %d unsupported (64 or 128)", fn, head_dim);
    return SRDIT_EUNSUPPORTED;
  }
  if (dtype != SRDIT_DTYPE_BF16 && dtype != SRDIT_DTYPE_FP16) {
    set_error("%s: dtype code %d unsupported", fn, dtype);
    return SRDIT_EUNSUPPORTED;
  }
  DenseArgs a;
  a.q = q; a.k = k; a.v = v; a.o = o;
  a.q_tokens = static_cast<int>(q_tokens);
  a.kv_tokens = static_cast<int>(kv_tokens);
  a.n_heads = n_heads;
  a.tiles = static_cast<int>((q_tokens + DQT - 1) / DQT);
  const int64_t tasks = static_cast<int64_t>(a.tiles) * n_heads;
  SRDIT_REQUIRE(tasks < (1LL << 31), "%s: too many tasks", fn);
  a.n_tasks = static_cast<int>(tasks);
  a.scale_log2 = scale * 1.4426950408889634f;
  a.amax_out = amax_out;
  // two workgroups per CU, a multiple of 8 (one share per XCD), no more than
  // the tasks need
  const int64_t slots = static_cast<int64_t>(cu_count() / 8 * 8) * 2;
  const int64_t need = (tasks + 7) / 8 * 8;
  const uint32_t grid = static_cast<uint32_t>(slots >= 8 ? (need < slots ? need : slots) : 8);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (dtype == SRDIT_DTYPE_BF16)
    return head_dim == 128 ? launch_dense<__bf16, 128>(a, grid, s) : launch_dense<__bf16, 64>(a, grid, s);
  return head_dim == 128 ? launch_dense<_Float16, 128>(a, grid, s)
                         : launch_dense<_Float16, 64>(a, grid, s);
}
