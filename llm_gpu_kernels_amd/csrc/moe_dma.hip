// bf16 weight-streaming grouped GEMMs with global -> LDS direct loads, for
// few rows per expert (the streaming regime of moe_stream.hip): gate/up +
// SwiGLU (reference: _dynamic_grouped_gate_up_swiglu, moe_fused.py:18-73;
// cuda_gate_up_bf16, cuda_gate_up.cu:53-131) and the down projection
// (_dynamic_grouped, moe.py:69-95).
//
// Units like the register-streaming kernel's -- (task, 16 act columns) with
// 16 gate + 16 up weight rows, or (task, 64 hidden columns) of down -- and
// the same split-K over eight MFMA waves with a fixed-order reduction, but the
// weights reach the matrix cores through LDS:
//  * eight loader waves move each unit's 32 (64) weight rows in K-stages of KC
//    elements with gfx950's 16-byte global -> LDS loads; every load
//    instruction reads one contiguous 1 KiB piece (one row's KC = 512
//    elements, or two rows' 256), the pattern HBM streams fastest (6.5 TB/s
//    measured, against 5.3-5.6 TB/s for the 16 rows x 64 bytes of a direct
//    MFMA-operand load).  The loaders own every wait on those loads;
//  * the stages form a ring of NS buffers in LDS, NS - 1 stages ahead; one
//    workgroup barrier per stage publishes a stage and frees the oldest;
//  * the MFMA waves read their K-slice of a stage as MFMA A fragments
//    (16-byte chunks XOR-swizzled by row on the global side, so the reads are
//    bank-conflict free) against token rows held in registers for the whole
//    task (the next task's rows load during the unit before the switch);
//  * a unit's eight partial tiles are written to LDS after its last stage and
//    reduced, in fixed wave order, after the next stage barrier (by threads
//    of alternating waves from unit to unit).
// One 1024-thread workgroup per CU; persistent workgroups take their units
// from a device-wide counter (below), and the MFMA waves load the next
// task's token rows behind the current unit's MFMAs.  Rounding as in
// moe_stream.hip.
#include "common.h"
#include "moe_internal.h"
#include "moe_route_dev.h"

#define MOE_CONST __attribute__((address_space(4)))

namespace moe {

namespace {

constexpr int kConsumers = 8;
constexpr int kDownRows = 64;
constexpr int kLoaders = 8;
constexpr int kThreads = (kConsumers + kLoaders) * kWave;
// Weight rows per unit: gate/up 16 gate + 16 up rows; down kDownRows rows
// with 16-row tasks, 32 with 32-row tasks (whose partials take twice the LDS).
template <int KIND, int MT>
constexpr int kRowsOf = KIND == 1 && MT == 1 ? kDownRows : 32;
constexpr int kWaitVmcntZero = (7 << 4) | (15 << 8);

template <typename T>
__device__ __forceinline__ const MOE_CONST T *as_const(const T *p) {
  return (const MOE_CONST T *)p;
}

__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Loader barrier: no fence (a release fence would wait for the loader's own
// LDS loads, which is exactly what the ring must not do); compiler barriers
// keep the loads on their side of it.
__device__ __forceinline__ void loader_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Planning prologue (PLAN): the task list and grouped-row -> token table stay
// in LDS for the whole launch.
constexpr int kPlanTaskMax = route_dev::kMaxExperts + route_dev::kSmallPlanRoutes / 16;
constexpr int kPlanBytes = kPlanTaskMax * 16 + (route_dev::kSmallPlanRoutes + 64) * 4 + 16;

// Work distribution.  Workgroup b first takes units A b .. A b + A - 1; every
// later unit comes from a device-wide counter, kChunkOf consecutive units per
// atomic add, so a workgroup that streams faster takes more units (static
// blocks of equal size measured a 20 us spread of finish times at T = 17, and
// T = 193 gate/up 145 -> 135 us with the counter).  MFMA wave 0 takes the
// unit A units ahead of the one it starts, and publishes it one unit later in
// an LDS ring that the loaders read when they set that unit up.  The counter
// pair {units handed out, workgroups finished} is reset by the last
// workgroup to finish, so it is zero at every launch.
constexpr int kSeqRing = 8;
// Units per counter step: pairs of consecutive units (fewer task switches)
// measured 2-8 us faster per launch than single units at T = 17 and 193, and
// than larger blocks, which leave longer tails; the 32-row units of down
// with 32-row tasks go in fours (T = 300-480: down 3-7 us faster than pairs).
// The last G counter-served units go out one per step: a pair taken at the
// very end held its workgroup ~8 us (two 128 KiB units) past the others
// (per-workgroup stamps at BF16 T = 17: median end 86 us, last 92.7 us).
// With PLAN (routing in the prologue) the first unit of workgroup b is named
// before routing (see the kernel) and its stages load during the prologue.
template <int KIND, int MT>
constexpr int kChunkOf = KIND == 1 && MT == 2 ? 4 : 2;

// The finishing add also carries the workgroup's unit count (bits 12 and
// up; grids stay below 4096 workgroups), so the last workgroup knows how many
// units the launch ran.  Anything but exactly `total` means the counters were
// not zero at launch (a workspace that was not zeroed, a launch that did not
// complete): units were skipped or run twice, and the launch latches
// MOE_STATUS_DIRTY_COUNTERS into status[0] instead of returning a wrong
// result with a clean status.
__device__ __forceinline__ void finish_units(int32_t *w, int G, int units, int total, uint32_t *status) {
  const uint32_t old = (uint32_t)atomicAdd(w + 1, 1 + (units << 12));
  if ((old & 0xfffu) == (uint32_t)G - 1u) {
    if ((int)(old >> 12) + units != total) atomicOr(status, kStatusDirtyCounters);
    atomicExch(w, 0);
    atomicExch(w + 1, 0);
  }
}

template <int KIND, int MT, bool PLAN = false>
struct DmaCfg {
  static constexpr int ROWS = kRowsOf<KIND, MT>;
  static constexpr int NRB = ROWS / 16;                   // 16-row MFMA blocks per unit
  static constexpr int KC = KIND == 0 ? 512 : 256;      // K per stage
  static constexpr int STAGE = ROWS * KC * 2;             // bytes
  static constexpr int KKS = KC / kConsumers / 32;        // k-steps per wave per stage
  // Partial tiles of one unit, reduced after the first stage barrier of the
  // next unit.  One buffer suffices because every unit has two or more
  // stages (checked in the kernel): the next unit writes its partials only
  // after its second stage barrier, which every wave reaches after its part
  // of the reduction.
  static constexpr int PAR = 1;
  static constexpr int RED = PAR * kConsumers * NRB * MT * kWave * 16;
  static constexpr int PLANB = PLAN ? kPlanBytes : 0;
  static constexpr int SEQB = kSeqRing * 4;
  static constexpr int NS0 = (int)((kMaxLds - RED - PLANB - SEQB) / STAGE);
  // Ring depth: at most five stages for down (with 16 KiB stages, four ahead
  // measured 0.5 us faster than seven); its 64-row units' 32 KiB stages fit
  // three beside the partials and the unit ring.  Gate/up keeps all it fits.
  static constexpr int NSMAX = KIND == 1 ? 5 : 8;
  static constexpr int NS = NS0 > NSMAX ? NSMAX : NS0;
  static constexpr int PER = STAGE / 1024 / kLoaders;     // 1 KiB loads per stage per loader
  static_assert(NS >= 3, "at least two stages ahead");
  static_assert((NS - 2) * PER < 64, "vmcnt range");
  static constexpr int LDS = NS * STAGE + RED + PLANB + SEQB;
};

// Units taken ahead: a unit taken at the start of unit k is published at the
// start of unit k + 1 and must be visible (one barrier later) when the
// loaders set up its first stage, NS - 1 stages ahead of the MFMA waves:
// (A - 1) SPU >= NS.  A is also how many units a workgroup holds when the
// counter runs out, so it is kept at that minimum (one more unit ahead
// measured 10 us slower at T = 17).
template <int NS, int SPU>
constexpr int kAheadOf = 1 + (NS + SPU - 1) / SPU;

// Byte offset in a stage of 16-byte chunk c of stage row R (rows of KC elements).
template <int KC>
__device__ __forceinline__ int stage_off(int R, int c) {
  return R * (KC * 2) + ((c ^ (R & 15)) << 4);
}

// PLAN (gate/up, 16-row tasks, T <= 32 router-fused shapes): every workgroup
// first routes all tokens and plans in LDS (route_dev::route_token and
// plan_small), and workgroup 0 also writes the routing results and the global
// plan arrays for the down and combine launches; the separate planner launch
// is then not needed.
template <int KIND, int MT, int SPU, bool PLAN = false>
__global__ __launch_bounds__(kThreads) void dma_kernel(ExpertArgs a, RouteArgs ra) {
  using C = DmaCfg<KIND, MT, PLAN>;
  static_assert(!PLAN || (KIND == 0 && MT == 1), "planning prologue: 16-row gate/up");
  static_assert(SPU >= 2, "one partial buffer needs two or more stages per unit");
  constexpr int KC = C::KC, KKS = C::KKS, NS = C::NS, PER = C::PER;
  constexpr int NRB = C::NRB, ROWS = C::ROWS;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  f32x4 *s_red = (f32x4 *)(smem + NS * C::STAGE);  // [2][kConsumers][NRB][MT][64]

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & (kWave - 1);
  const int H = a.H, I = a.I;
  const int K = KIND == 0 ? H : I;  // == SPU * KC (checked on the host)
  const int ncb = KIND == 0 ? I / 16 : H / ROWS;  // units per task
  const int4 *l_tasks = nullptr;
  const int *l_row_token = nullptr;
  int ntasks = 0;
  const int G = gridDim.x;
  int32_t *const wcnt = a.counters + 2 * KIND;
  int *const seq = (int *)(smem + NS * C::STAGE + C::RED);
  // PLAN: speculative first unit.  Workgroup b < C0 E (C0 = G / E column
  // blocks per expert) starts with column block b / E of expert b % E, which
  // it can name before routing.  Its loader waves that route no token stream
  // that unit's first NS - 1 stages into the stage ring while the workgroup
  // routes and plans (HBM is otherwise idle then).  After planning the unit
  // is kept when the expert is active and has a single task (then the units
  // with column block < C0 of every task are exactly the workgroups' first
  // units), and the prefetched stages are discarded otherwise.  Every other
  // unit comes from the counter.
  constexpr int kPrefetch = NS - 1 < SPU ? NS - 1 : SPU;  // stages of unit 0 prefetched
  int spec_u = -1;      // the kept speculative unit (PLAN)
  bool spec_pf = false; // this wave issued prefetch loads (PLAN loaders)
  int nsc = 0;          // column blocks per task taken by first units (PLAN)
  int c_first = 0;      // wave 0, lane 0: the first counter chunk (PLAN)
  if constexpr (PLAN) {
    using namespace route_dev;
    uint8_t *pa = smem + NS * C::STAGE + C::RED + C::SEQB;
    int4 *p_tasks = (int4 *)pa;
    int *p_row = (int *)(pa + kPlanTaskMax * 16);
    int *p_nt = p_row + kSmallPlanRoutes + 64;
    const int E = ra.E;
    const int C0 = min(G / E, ncb);
    const bool spec_wg = (int)blockIdx.x < C0 * E;
    const int se = (int)blockIdx.x % E, scb = (int)blockIdx.x / E;
    const bool half = ra.fuse_router == 2;
    const int nroute = min(kConsumers + kLoaders, half ? (ra.T + 1) / 2 : ra.T);  // routing waves
    const int free0 = max(kConsumers, nroute);  // loader waves >= free0 route no token
    if (spec_wg && wave >= free0) {
      // Stage s, piece p (stage row p * RPI + lane / LPR, 16-byte chunk
      // lane % LPR, XOR-swizzled as the loaders place it), the free loader
      // waves' pieces in turn.
      constexpr int RPI = 1024 / (KC * 2), LPR = kWave / RPI, NP = C::STAGE / 1024;
      const int nfree = kConsumers + kLoaders - free0, fi = wave - free0;
      const int lrow = lane / LPR, lch = lane % LPR;
      for (int q = fi; q < kPrefetch * NP; q += nfree) {
        const int st = q / NP, pc = q - st * NP;
        const int R = pc * RPI + lrow;
        const size_t grow = (size_t)se * 2 * I + (R < 16 ? scb * 16 + R : I + scb * 16 + R - 16);
        const uint16_t *src = a.gate_up + grow * K + (lch ^ (R & 15)) * 8 + st * KC;
        __builtin_amdgcn_global_load_lds((const void *)src,
                                         (__attribute__((address_space(3))) void *)(smem + st * C::STAGE + pc * 1024),
                                         16, 0, 0);
      }
      spec_pf = true;
    }
    // The first counter chunk: requested by the last wave (which routes a
    // token only from T = 31 on) after its prefetch loads, used after
    // planning; it passes through the last unit-ring slot.
    if (wave == kConsumers + kLoaders - 1 && lane == 0) seq[kSeqRing - 1] = atomicAdd(wcnt, 1);
    // Scratch in the last stage buffer (the prefetch fills the others).
    uint8_t *scr = smem + (NS - 1) * C::STAGE;
    static_assert(12 * kSmallPlanRoutes + 4 * kSmallPlanWaves * kMaxExperts + 12 * kMaxExperts + 8 <= C::STAGE,
                  "planning scratch fits one stage");
    int *x_ids = (int *)scr;
    float *x_w = (float *)(scr + 4 * kSmallPlanRoutes);
    int *x_wcnt = (int *)(scr + 8 * kSmallPlanRoutes);
    int *x_cnt = x_wcnt + kSmallPlanWaves * kMaxExperts;
    int *x_off = x_cnt + kMaxExperts;
    int *x_toff = x_off + kMaxExperts;
    uint32_t *x_flags = (uint32_t *)(x_toff + kMaxExperts + 1);
    // One token per wave (fuse_router 1) or half-wave (2); logits first.
    // (16 lanes per token measured 0.4 us slower here: the sixteen waves
    // route up to 32 tokens in one pass either way.)
    const int ft = half ? 2 * wave + (lane >> 5) : wave;
    const bool fwave = half ? 2 * wave < ra.T : wave < ra.T;  // wave-uniform
    float raw[4];
    if (fwave) {  // waves that route no token skip the loads (and their waits)
      if (half) load_token_logits<true>(ra.logits, ft, ft < ra.T, ra.E, raw);
      else load_token_logits<false>(ra.logits, ft, ft < ra.T, ra.E, raw);
    }
    for (int i = tid; i < kSmallPlanWaves * ra.E; i += kThreads) x_wcnt[i] = 0;
    if (tid == 0) *x_flags = 0;
    const bool g0 = blockIdx.x == 0;
    uint32_t flags = 0;
    if (fwave) {
      int32_t *ids_g = g0 ? (int32_t *)ra.ids : nullptr;
      float *w_g = g0 ? ra.weights : nullptr;
      if (half)
        route_token<true>(raw, ft, ft < ra.T, ra.E, ra.K, ra.renormalize, ids_g, w_g, flags, x_ids, x_w);
      else
        route_token<false>(raw, ft, true, ra.E, ra.K, ra.renormalize, ids_g, w_g, flags, x_ids, x_w);
    }
    // LDS-only barrier: a full one would make the prefetching waves wait for
    // their stage loads.
    lds_sync();
    const SmallPlanLds L{x_ids, x_w, x_wcnt, x_cnt, x_off, x_toff, p_tasks, p_row, p_nt, x_flags};
    const SmallPlanOut O{ra.counts, ra.offsets, ra.ranks, ra.map, ra.row_route, ra.row_token,
                         ra.tasks, ra.num_tasks, ra.status};
    plan_small(L, O, g0, ra.R, ra.E, ra.K, 16, flags);
    ntasks = *p_nt;
    l_tasks = p_tasks;
    l_row_token = p_row;
    // First units are kept when every active expert has one task (always
    // below 17 tokens): then the counter hands out column blocks >= C0.
    bool one_task = true;
    for (int e = lane; e < E; e += kWave) one_task &= x_cnt[e] <= 16;
    one_task = __builtin_amdgcn_readfirstlane((int)(__ballot(!one_task) == 0)) != 0;
    nsc = one_task && C0 > 0 ? C0 : 0;
    if (nsc > 0 && spec_wg && x_cnt[se] > 0) spec_u = x_toff[se] * ncb + scb;
  }
  // The planning gate/up launch is the first of its forward: it zeroes the
  // down launch's counters (which start only after this launch ends).
  if (PLAN && blockIdx.x == 0 && tid < 2) a.counters[2 + tid] = 0;
  const int total = (PLAN ? ntasks : *as_const(a.num_tasks)) * ncb;
  constexpr int A = kAheadOf<NS, SPU>;
  static_assert(A + 1 <= kSeqRing, "unit ring");
  constexpr int CH = kChunkOf<KIND, MT>;
  // Units taken without the counter.  Without PLAN: S consecutive ones per
  // workgroup (static shares up to 7/8 of the work, the rest from the
  // counter, measured slower: the per-workgroup streaming rate varies too
  // much).  With PLAN: the kept first unit, then the counter from the start
  // (MFMA wave 0 takes the first A units after planning and publishes them in
  // the unit ring).
  constexpr int S = PLAN ? 0 : A;
  const int ub = (int)blockIdx.x * S;  // this workgroup's first unit
  // Counter-served units: value v -> unit v + S G, or with PLAN (task
  // v / (ncb - nsc), column block nsc + v % (ncb - nsc)); total_v in all.
  const int ncv = ncb - nsc;
  const int total_v = PLAN ? ntasks * ncv : max(0, total - S * G);
  auto unit_of_v = [&](int v) -> int {
    if (v < 0 || v >= total_v) return total;
    if (!PLAN) return v + S * G;
    const int t = v / ncv;
    return t * ncb + nsc + (v - t * ncv);
  };
  // Counter value c hands out CH consecutive values while c < cs, then one
  // value each: the last round of units goes out singly, so that no
  // workgroup takes a long chunk at the very end (the launch's tail).
  const int cs = max(0, (total_v - G) / CH);
  auto chunk_of = [&](int c, int &base, int &size) {
    if (c < cs) {
      base = CH * c;
      size = CH;
    } else {
      base = CH * cs + (c - cs);
      size = 1;
    }
  };
  // Wave 0, lane 0: the counter walk -- value of the unit taken last, the
  // current chunk (base, size; size < 0 while its add is in flight in
  // `cpend`) and the values of it used.
  int taken = 0, tbase = 0, tsize = 0, tpos = 0, cpend = 0;
  if constexpr (PLAN) {
    if (wave == 0 && lane == 0) {
      c_first = seq[kSeqRing - 1];
      chunk_of(c_first, tbase, tsize);
      int k = 0;
      if (spec_u >= 0) seq[k++] = spec_u;
      for (; k < A; ++k) {
        if (tpos == tsize) {
          chunk_of(atomicAdd(wcnt, 1), tbase, tsize);
          tpos = 0;
        }
        taken = tbase + tpos++;
        seq[k] = unit_of_v(taken);
      }
    }
    __syncthreads();
    if (seq[0] >= total) {
      if (spec_pf) wait_vmcnt<0>();
      if (tid == 0) finish_units(wcnt, G, 0, total, a.status);
      return;
    }
  } else if (ub >= total) {
    if (tid == 0) finish_units(wcnt, G, 0, total, a.status);
    return;
  }
  const MOE_CONST int32_t *tasks = as_const((const int32_t *)a.tasks);

  if (wave >= kConsumers) {
    // ---- loaders ------------------------------------------------------------
    const int lw = wave - kConsumers;
    // Load j of this wave covers stage rows R0 .. R0 + RPI - 1, RPI = 1024 / (2 KC)
    // rows per 1 KiB; lane l writes LDS byte 16 l of the piece.
    constexpr int RPI = 1024 / (KC * 2);
    constexpr int LPR = kWave / RPI;  // lanes per row
    const int lrow = lane / LPR, lch = lane % LPR;
    int cur = -1;
    const uint16_t *src[PER];
    // The task's expert: from LDS with PLAN through an instruction the compiler
    // cannot see (a visible LDS access after global -> LDS loads makes it
    // wait for every such load in flight).
    auto expert_of = [&](int t) -> int {
      if constexpr (PLAN) {
        uint32_t v;
        asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)"
                     : "=v"(v)
                     : "v"((uint32_t)(size_t)(const __attribute__((address_space(3))) int4 *)(l_tasks + t))
                     : "memory");
        return __builtin_amdgcn_readfirstlane(v);
      } else {
        return tasks[4 * t];
      }
    };
    auto setup = [&](int u, int e) {
      const int t = u / ncb, cb = u - t * ncb;
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const int R = (lw * PER + j) * RPI + lrow;  // stage row
        size_t grow;
        if (KIND == 0) grow = (size_t)e * 2 * I + (R < 16 ? cb * 16 + R : I + cb * 16 + R - 16);
        else grow = (size_t)e * H + cb * ROWS + R;
        const int c = lch ^ (R & 15);  // the chunk that belongs at LDS chunk lch
        src[j] = (KIND == 0 ? a.gate_up : a.down) + grow * K + c * 8;
      }
    };
    // Unit k of this workgroup (k >= A: published by MFMA wave 0, read
    // through an instruction the compiler cannot see).
    auto unit_at = [&](int k) -> int {
      if (!PLAN && k < S) return ub + k;
      uint32_t v;
      asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)"
                   : "=v"(v)
                   : "v"((uint32_t)(size_t)(const __attribute__((address_space(3))) int *)(seq + k % kSeqRing))
                   : "memory");
      return __builtin_amdgcn_readfirstlane(v);
    };
    int issued = 0;
    bool ended = false;
    // Issues stage `issued` unless its unit is past the end.
    auto issue = [&]() {
      const int st = issued;
      const int i = st / SPU, s = st - (st / SPU) * SPU;
      if (i != cur) {
        const int u = unit_at(i);
        if (u >= total) {
          ended = true;
          return;
        }
        setup(u, expert_of(u / ncb));
        cur = i;
      }
      uint8_t *buf = smem + (st % NS) * C::STAGE;
#pragma unroll
      for (int j = 0; j < PER; ++j)
        __builtin_amdgcn_global_load_lds(
            (const void *)(src[j] + s * KC),
            (__attribute__((address_space(3))) void *)(buf + (lw * PER + j) * 1024), 16, 0, 0);
      ++issued;
    };
    if (PLAN && spec_pf) {
      // The prefetched stages have landed (issued before routing); they are
      // unit 0's first kPrefetch stages when the speculative unit was kept.
      wait_vmcnt<0>();
      if (spec_u >= 0) {
        setup(spec_u, expert_of(spec_u / ncb));
        cur = 0;
        issued = kPrefetch;
      }
    }
    while (issued < NS - 1 && !ended) issue();
    for (int st = 0; st < issued; ++st) {
      // Stage st has landed once at most the loads issued after it remain.
      const int later = issued - 1 - st;
      switch (later) {
        case 0: wait_vmcnt<0>(); break;
        case 1: wait_vmcnt<PER>(); break;
        case 2: wait_vmcnt<(NS > 3 ? 2 : 0) * PER>(); break;
        case 3: wait_vmcnt<(NS > 4 ? 3 : 0) * PER>(); break;
        case 4: wait_vmcnt<(NS > 5 ? 4 : 0) * PER>(); break;
        case 5: wait_vmcnt<(NS > 6 ? 5 : 0) * PER>(); break;
        default: wait_vmcnt<(NS > 7 ? 6 : 0) * PER>(); break;
      }
      loader_barrier();
      // Buffer (st - 1) % NS was last read before this barrier.
      if (!ended) issue();
    }
    loader_barrier();  // the MFMA waves' last reduction barrier
    return;
  }

  // ---- MFMA waves: wave w owns K-slice [w * KC / 8, +KC / 8) of every stage --
  const int r = lane & 15, g = lane >> 4;
  struct Meta {
    int task, cb, row0, rows;
    int idxv;  // lane k < 32: token (gate/up) or route (down) of row k
  };
  const int32_t *row_vec = KIND == 0 ? a.row_token : a.row_route;
  auto meta_of = [&](int u) {
    Meta m;
    m.task = u / ncb;
    m.cb = u - m.task * ncb;
    if constexpr (PLAN) {
      const int4 tk = l_tasks[m.task];
      m.row0 = __builtin_amdgcn_readfirstlane(tk.y);
      m.rows = __builtin_amdgcn_readfirstlane(tk.z);
      m.idxv = l_row_token[m.row0 + (lane & 31)];
    } else {
      m.row0 = tasks[4 * m.task + 1];
      m.rows = tasks[4 * m.task + 2];
      m.idxv = row_vec[m.row0 + (lane & 31)];
    }
    return m;
  };

  // Token rows of the task: fragment [mt][s * KKS + kk] = row mt*16 + r,
  // K = s*KC + wave*KC/8 + kk*32 + 8g .. +8.  Rows past the task's end are
  // zero (columns the epilogue never stores).
  // The next task's rows load behind the current unit's MFMAs when a second
  // set fits in registers (else at the switch, with a wait).
  constexpr bool PREF = MT * SPU * KKS * 4 <= 32;
  u32x4 bfr[MT][SPU * KKS], bnext[MT][SPU * KKS];
  auto load_b = [&](const Meta &m, u32x4(&dst)[MT][SPU * KKS]) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int j = mt * 16 + r;
      const bool ok = j < m.rows;
      const int q = __shfl(m.idxv, j, kWave);
      size_t row;
      if (KIND == 0) row = (size_t)q * H;
      else row = (size_t)(m.row0 + j) * I;
      const uint16_t *b = (KIND == 0 ? a.x : a.act) + row + wave * (KC / 8) + g * 8;
#pragma unroll
      for (int s = 0; s < SPU; ++s)
#pragma unroll
        for (int kk = 0; kk < KKS; ++kk)
          dst[mt][s * KKS + kk] = ok ? *(const u32x4 *)(b + s * KC + kk * 32) : u32x4{0u, 0u, 0u, 0u};
    }
  };

  auto epilogue = [&](const Meta &m, int parity, int rot) {
    const f32x4 *red = s_red + (size_t)parity * kConsumers * NRB * MT * kWave;
    if (KIND == 0) {
      // The threads of the epilogue rotate over the MFMA waves from unit to unit.
      constexpr int EN = MT * 4 * kWave;
      const int et = tid - (rot % (kConsumers * kWave / EN)) * EN;
      if (et >= 0 && et < EN) {
        const int l = et & 63, i = (et >> 6) & 3, mt = et >> 8;
        const int j = mt * 16 + (l & 15);
        const float *redf = (const float *)red;
        auto part = [&](int w, int rb) { return redf[((((w * NRB + rb) * MT + mt) * 4 + i) * kWave + l)]; };
        float sg = part(0, 0), su = part(0, 1);
#pragma unroll
        for (int w = 1; w < kConsumers; ++w) {
          sg += part(w, 0);
          su += part(w, 1);
        }
        const float gt = bf16_round(sg);
        const float up = bf16_round(su);
        const float v = gt / (1.0f + expf(-gt)) * up;
        if (j < m.rows)
          a.act[(size_t)(m.row0 + j) * I + m.cb * 16 + 4 * (l >> 4) + i] =
              (uint16_t)(pack_bf16x2(v, 0.f) & 0xffffu);
      }
    } else {
      constexpr int EN = NRB * MT * kWave;
      const int et = tid - (rot % (kConsumers * kWave / EN)) * EN;
      if (et >= 0 && et < EN) {
        const int rb = et / (MT * kWave);
        const int mt = (et >> 6) % MT, l = et & 63;
        const int j = mt * 16 + (l & 15);
        f32x4 sm = red[(rb * MT + mt) * kWave + l];
#pragma unroll
        for (int w = 1; w < kConsumers; ++w) sm += red[((w * NRB + rb) * MT + mt) * kWave + l];
        const int q = __shfl(m.idxv, j, kWave);
        u32x2 packed;
        packed[0] = pack_bf16x2(sm[0], sm[1]);
        packed[1] = pack_bf16x2(sm[2], sm[3]);
        if (j < m.rows)
          *(u32x2 *)(a.routed + (size_t)q * H + m.cb * ROWS + rb * 16 + 4 * (l >> 4)) = packed;
      }
    }
  };

  // Unit k of this workgroup, k >= A: published by MFMA wave 0 at the start
  // of unit k - A + 1 (visible to every wave one barrier later).
  auto unit_at = [&](int k) -> int { return k < S ? ub + k : seq[k % kSeqRing]; };
  Meta prev, cur = meta_of(unit_at(0)), next;
  load_b(cur, bfr);
  int done_units = 0;  // units this workgroup ran (known when its loop ends)
  bool taking = true;  // wave 0: the units taken so far are all in range
  bool pending = false;
  int st = 0;
  for (int i = 0;; ++i) {
    int un = total;  // unit i + 1
    f32x4 acc[NRB][MT];
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[rb][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < SPU; ++s, ++st) {
      lds_barrier();  // stage st published; unit i-1's partials published
      if (s == 0) {
        if (i > 0) epilogue(prev, (i - 1) % C::PAR, (i - 1) & 1);
        if (wave == 0) {
          if (pending) {  // unit i - 1 + A, taken at the start of unit i - 1
            if (lane == 0 && tsize < 0) {  // a new chunk: its add has returned by now
              chunk_of(cpend, tbase, tsize);
              taken = tbase;
              tpos = 1;
            }
            const int u = unit_of_v(__builtin_amdgcn_readfirstlane(taken));
            if (lane == 0) seq[(i - 1 + A) % kSeqRing] = u;
            taking = u < total;  // (a corrupted counter ends the workgroup's units)
            pending = false;
          }
          if (taking) {  // unit i + A
            if (lane == 0) {
              if (tsize > 0 && tpos < tsize) {
                taken = tbase + tpos++;
              } else {
                cpend = atomicAdd(wcnt, 1);
                tsize = -1;
              }
            }
            pending = true;
          }
        }
      }
      if (s == 1) {
        // The next unit; its token rows load behind this unit's MFMAs when
        // it belongs to another task.
        un = unit_at(i + 1);
        if (un < total) {
          next = meta_of(un);
          if (PREF && next.task != cur.task) load_b(next, bnext);
        }
      }
      const uint8_t *buf = smem + (st % NS) * C::STAGE;
      u32x4 af[KKS][NRB];
#pragma unroll
      for (int kk = 0; kk < KKS; ++kk)
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {
          const int c = wave * (KC / 64) + kk * 4 + g;
          af[kk][rb] = *(const u32x4 *)(buf + stage_off<KC>(rb * 16 + r, c));
        }
#pragma unroll
      for (int kk = 0; kk < KKS; ++kk)
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            acc[rb][mt] = mfma16(af[kk][rb], bfr[mt][s * KKS + kk], acc[rb][mt]);
    }
    // Partials of unit i (buffer i % PAR), reduced after the next barrier.
    f32x4 *red = s_red + (size_t)(i % C::PAR) * kConsumers * NRB * MT * kWave;
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if constexpr (KIND == 0) {
          // component-major: the epilogue's one-output-per-thread reads are
          // consecutive floats across lanes (no LDS bank conflicts)
          float *rf = (float *)red + (((wave * NRB + rb) * MT + mt) * 4) * kWave + lane;
#pragma unroll
          for (int c = 0; c < 4; ++c) rf[c * kWave] = acc[rb][mt][c];
        } else {
          red[((wave * NRB + rb) * MT + mt) * kWave + lane] = acc[rb][mt];
        }
      }
    prev = cur;
    if (un >= total) {
      lds_barrier();
      epilogue(prev, i % C::PAR, i & 1);
      done_units = i + 1;
      break;
    }
    if (next.task != cur.task) {
      if constexpr (PREF) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int j = 0; j < SPU * KKS; ++j) bfr[mt][j] = bnext[mt][j];
      } else {
        load_b(next, bfr);
      }
    }
    cur = next;
  }
  // Every unit this workgroup took has been read back (or is waited for
  // here) before it counts itself finished.
  if (wave == 0) {
    __builtin_amdgcn_s_waitcnt(kWaitVmcntZero);
    if (lane == 0) finish_units(wcnt, G, done_units, total, a.status);
  }
}

template <int KIND, int MT, int SPU, bool PLAN = false>
hipError_t launch_one(const ExpertArgs &a, int num_cus, hipStream_t s, const RouteArgs *ra = nullptr) {
  using C = DmaCfg<KIND, MT, PLAN>;
  auto k = dma_kernel<KIND, MT, SPU, PLAN>;
  const size_t lds = C::LDS;
  static const bool attr = hipFuncSetAttribute((const void *)k,
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)lds) == hipSuccess;
  if (!attr) return hipErrorInvalidValue;
  RouteArgs none{};
  if (num_cus >= 4096) return hipErrorInvalidValue;  // finish_units packs the grid size in 12 bits
  hipLaunchKernelGGL(k, dim3(num_cus > 0 ? num_cus : 1), dim3(kThreads), lds, s, a, ra ? *ra : none);
  return hipGetLastError();
}

}  // namespace

// gate/up: K = H in 2 or 4 stages of 512 (8 with 16-row tasks); down: K = I
// in 2, 3 or 4 stages of 256.
bool dma_shape_ok(int H, int I, int token_block) {
  return (H == 1024 || H == 2048 || (H == 4096 && token_block == 16)) &&
         (I == 512 || I == 768 || I == 1024);
}

namespace {
template <int KIND, int MT>
hipError_t launch_spu(const ExpertArgs &a, int spu, int num_cus, hipStream_t s) {
  if (spu == 2) return launch_one<KIND, MT, 2>(a, num_cus, s);
  if (spu == 4) return launch_one<KIND, MT, 4>(a, num_cus, s);
  if constexpr (KIND == 1) {
    if (spu == 3) return launch_one<KIND, MT, 3>(a, num_cus, s);
  } else if constexpr (MT == 1) {
    if (spu == 8) return launch_one<KIND, MT, 8>(a, num_cus, s);
  }
  return hipErrorInvalidValue;
}
}  // namespace

hipError_t launch_dma_gate_up(const ExpertArgs &a, int token_block, int num_cus, hipStream_t s) {
  const int spu = a.H / 512;
  return token_block == 16 ? launch_spu<0, 1>(a, spu, num_cus, s) : launch_spu<0, 2>(a, spu, num_cus, s);
}

hipError_t launch_dma_down(const ExpertArgs &a, int token_block, int num_cus, hipStream_t s) {
  const int spu = a.I / 256;
  return token_block == 16 ? launch_spu<1, 1>(a, spu, num_cus, s) : launch_spu<1, 2>(a, spu, num_cus, s);
}

// gate/up with the routing and planning prologue: 16-row tasks, H = 1024 or
// 2048, at most 1024 routes, the router shapes the planner fuses (one token
// per wave up to 16 tokens, per half-wave up to 32 with E <= 128).
bool dma_plan_ok(int H, int I, int T, int K, int E, int fuse_router) {
  return dma_shape_ok(H, I, 16) && (H == 1024 || H == 2048) && fuse_router != 0 &&
         T * K <= route_dev::kSmallPlanRoutes && E <= route_dev::kMaxExperts &&
         E + (T * K + 15) / 16 <= kPlanTaskMax;
}

hipError_t launch_dma_gate_up_planned(const ExpertArgs &a, const RouteArgs &ra, int num_cus,
                                      hipStream_t s) {
  if (a.H == 1024) return launch_one<0, 1, 2, true>(a, num_cus, s, &ra);
  if (a.H == 2048) return launch_one<0, 1, 4, true>(a, num_cus, s, &ra);
  return hipErrorInvalidValue;
}

}  // namespace moe
