// Routing and dispatch for the MoE forward on gfx950.
//
//  * router:  softmax(fp32) -> top-k -> renormalise, one wave64 per token
//             (semantics of scripts/capture_qwen3_moe_layer0.py:583-586).
//  * planner: one 1024-thread workgroup computes the status word, per-expert
//             counts, canonical expert-local ranks, the exclusive scan, the
//             route->row map, its inverse and the GEMM task list.  It replaces
//             _reset / _rank_histogram / _prefix / the MAP half of
//             _rank_dispatch (moe.py:13-43, moe_ranked.py:18-65).
//
// Ranks are canonical: rank[q] = #{q' < q : id[q'] == id[q]}.  They are
// computed with wave ballots (a radix "match" over the ID bits) instead of
// the reference's relaxed atomics, so the permutation is deterministic and
// bit-identical from run to run.
#include "common.h"
#include "moe_internal.h"
#include "moe_route_dev.h"

namespace moe {

namespace {

constexpr int kPlanThreads = 1024;
constexpr int kPlanWaves = kPlanThreads / kWave;
using namespace route_dev;

__global__ __launch_bounds__(256) void router_kernel(RouteArgs a) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  uint32_t flags = 0;
  if (t < a.T) {
    float raw[4];
    load_token_logits<false>(a.logits, t, true, a.E, raw);
    route_token<false>(raw, t, true, a.E, a.K, a.renormalize, (int32_t *)a.ids, a.weights, flags,
                       nullptr, nullptr);
  }
  if (flags && (threadIdx.x & 63) == 0) atomicOr(&a.status[1], flags);
}

// Routes held in LDS by the planner (covers T = 1024 at top-8).
constexpr int kLdsRoutes = 8192;
static_assert(32 * 32 <= kLdsRoutes, "fused router (T <= 32, K <= 32) must fit the LDS routes");

// LDS of the planner, carved by hand so the route arrays exist only when the
// routes fit (R <= kLdsRoutes).
struct PlanShared {
  // Per-round per-wave expert counts, turned into exclusive prefixes in place;
  // two tables by round parity so the next round's table is cleared while the
  // current one is read.
  int wcnt[2][kPlanWaves][kMaxExperts];
  int run[kMaxExperts];
  int off[kMaxExperts];
  int toff[kMaxExperts + 1];
  uint32_t status;
};

template <typename IdT, bool LDSR>
__global__ __launch_bounds__(kPlanThreads) void route_plan_kernel(RouteArgs a) {
  __shared__ PlanShared sh;
  // LDSR: ids, weights (fused router only) and ranks stay on chip.
  __shared__ int s_ids[LDSR ? kLdsRoutes : 1];
  __shared__ int s_rank[LDSR ? kLdsRoutes : 1];
  __shared__ float s_w[LDSR ? kLdsRoutes : 1];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & (kWave - 1);
  const int E = a.E;
  const int nbits = id_bits(E);
  // Fused router: one token per wave (mode 1, T <= 16) or per half-wave
  // (mode 2, T <= 32, E <= 128); the logits are requested before the set-up.
  const int fmode = LDSR && a.route_logits ? a.fuse_router : 0;
  const int ft = fmode == 2 ? 2 * wave + (lane >> 5) : wave;
  const bool fwave = fmode == 2 ? 2 * wave < a.T : wave < a.T;  // wave-uniform
  float raw[4];
  if (fmode == 2) load_token_logits<true>(a.logits, ft, ft < a.T, E, raw);
  else if (fmode == 1) load_token_logits<false>(a.logits, ft, ft < a.T, E, raw);
  if (tid == 0) sh.status = 0;
  // The planner runs before both streaming GEMMs: their work counters start
  // at zero even on a workspace an earlier, aborted forward left dirty.
  if (tid < 4) a.counters[tid] = 0;
  for (int e = tid; e < E; e += kPlanThreads) sh.run[e] = 0;
  for (int i = tid; i < kPlanWaves * kMaxExperts; i += kPlanThreads) (&sh.wcnt[0][0][0])[i] = 0;
  uint32_t flags = 0;

  bool ids_in_lds = false;
  if (a.route_logits) {
    if (fmode == 2) {
      if (fwave)
        route_token<true>(raw, ft, ft < a.T, E, a.K, a.renormalize, (int32_t *)a.ids, a.weights,
                          flags, s_ids, s_w);
      ids_in_lds = true;
    } else if (fmode == 1) {
      if (fwave)
        route_token<false>(raw, ft, true, E, a.K, a.renormalize, (int32_t *)a.ids, a.weights,
                           flags, s_ids, s_w);
      ids_in_lds = true;
    } else if (tid == 0) {
      flags |= a.status[1];  // written by router_kernel earlier on this stream
      a.status[1] = 0;
    }
  }
  // The router's results become visible to the whole workgroup here (they
  // are read back from LDS when the routes fit there; otherwise from global
  // memory, which needs the stronger fence).
  if (LDSR && a.route_logits && a.fuse_router) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  } else {
    __threadfence_block();
    __syncthreads();
  }

  const IdT *ids = (const IdT *)a.ids;
  auto id_of = [&](int q) -> long long {
    if (LDSR && ids_in_lds) return s_ids[q];
    return (long long)ids[q];
  };
  // Pass 1 with the routes in global memory: canonical ranks, 1024 routes per
  // round, two barriers per round.
  auto rank_round = [&](int r, long long idv, float wv) __attribute__((always_inline)) {
    int (*cnt)[kMaxExperts] = sh.wcnt[r & 1];
    int *next = &sh.wcnt[(r + 1) & 1][0][0];
    const int q = r * kPlanThreads + tid;
    const bool valid = q < a.R;
    const bool ok = valid && idv >= 0 && idv < E;
    if (valid && !ok) flags |= 1u;
    if (valid && !isfinite(wv)) flags |= 2u;
    const int id = ok ? (int)idv : 0;
    uint64_t match = __ballot(ok);
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
      if (bit >= nbits) break;  // every id is below 2^nbits
      const bool set = (id >> bit) & 1;
      const uint64_t b = __ballot(ok && set);
      match &= set ? b : ~b;
    }
    const int lrank = __popcll(match & lanemask_lt());
    if (ok && lrank == 0) cnt[wave][id] = __popcll(match);
    __syncthreads();
    // Counts -> exclusive prefixes over (earlier rounds, earlier waves); the
    // other table, last read before this round's first barrier, is cleared.
    for (int e = tid; e < E; e += kPlanThreads) {
      int c = sh.run[e];
#pragma unroll
      for (int w = 0; w < kPlanWaves; ++w) {
        const int t = cnt[w][e];
        cnt[w][e] = c;
        c += t;
      }
      sh.run[e] = c;
    }
    for (int i = tid; i < kPlanWaves * kMaxExperts; i += kPlanThreads) next[i] = 0;
    __syncthreads();
    const int rank = ok ? cnt[wave][id] + lrank : -1;
    if (valid) a.ranks[q] = rank;
  };
  // Chunk of routes each wave ranks on its own (LDSR pass 1): a multiple of
  // 64 so a wave's sub-rounds are whole waves.
  const int CH = ((a.R + kPlanWaves - 1) / kPlanWaves + kWave - 1) / kWave * kWave;
  if constexpr (LDSR) {
    // Pass 1 with the routes on chip: wave w ranks routes [w*CH, (w+1)*CH)
    // in 64-route sub-rounds against its own per-expert counters, with no
    // workgroup barrier; one prefix over the waves (below) then turns the
    // chunk-local ranks into canonical ones: rank[q] = #{q' < q : id[q'] ==
    // id[q]} = (routes of that expert in earlier chunks) + (earlier in this
    // chunk).
    int *cnt = sh.wcnt[0][wave];
    // Every sub-round's id and weight are requested before the first one.
    constexpr int kSub = kLdsRoutes / kPlanWaves / kWave;  // CH <= kSub * 64
    long long pid[kSub];
    float pw[kSub];
#pragma unroll
    for (int j = 0; j < kSub; ++j) {
      const int q = wave * CH + j * kWave + lane;
      const bool valid = j * kWave < CH && q < a.R;
      pid[j] = valid ? id_of(q) : -1;
      pw[j] = valid ? (ids_in_lds ? s_w[q] : a.weights[q]) : 0.f;
    }
#pragma unroll
    for (int j = 0; j < kSub; ++j) {
      if (j * kWave >= CH) break;
      const int q = wave * CH + j * kWave + lane;
      const bool valid = q < a.R;
      const long long idv = pid[j];
      const float wv = pw[j];
      const bool ok = valid && idv >= 0 && idv < E;
      if (valid && !ok) flags |= 1u;
      if (valid && !isfinite(wv)) flags |= 2u;
      const int id = ok ? (int)idv : 0;
      uint64_t match = __ballot(ok);
#pragma unroll
      for (int bit = 0; bit < 8; ++bit) {
        if (bit >= nbits) break;
        const bool set = (id >> bit) & 1;
        const uint64_t bb = __ballot(ok && set);
        match &= set ? bb : ~bb;
      }
      const int lrank = __popcll(match & lanemask_lt());
      // Every lane of a group reads the counter before its first lane (the
      // only writer) updates it: one wave's LDS operations run in order.
      const int before = ok ? cnt[id] : 0;
      if (ok && lrank == 0) cnt[id] = before + __popcll(match);
      if (valid) {
        s_rank[q] = ok ? before + lrank : -1;
        if (!ids_in_lds) s_ids[q] = ok ? id : -1;
      }
    }
    __syncthreads();
    for (int e = tid; e < E; e += kPlanThreads) {
      int c = 0;
#pragma unroll
      for (int w = 0; w < kPlanWaves; ++w) {
        const int t = sh.wcnt[0][w][e];
        sh.wcnt[0][w][e] = c;
        c += t;
      }
      sh.run[e] = c;
    }
    __syncthreads();
  } else {
    for (int r = 0; r * kPlanThreads < a.R; ++r) {
      const int q = r * kPlanThreads + tid;
      rank_round(r, q < a.R ? id_of(q) : -1, q < a.R ? a.weights[q] : 0.f);
    }
  }

  // Pass 2: exclusive scans of counts and of per-expert task counts (wave 0,
  // four experts per lane).
  if (wave == 0) {
    const int tb = a.token_block;
    int c[4], nt[4], csum = 0, tsum = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane * 4 + j;
      c[j] = e < E ? sh.run[e] : 0;
      nt[j] = (c[j] + tb - 1) / tb;
      csum += c[j];
      tsum += nt[j];
    }
    const int cinc = wave_incl_scan(csum), tinc = wave_incl_scan(tsum);
    int crun = cinc - csum, trun = tinc - tsum;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane * 4 + j;
      if (e < E) {
        sh.off[e] = crun;
        sh.toff[e] = trun;
        a.counts[e] = c[j];
        a.offsets[e] = crun;
      }
      crun += c[j];
      trun += nt[j];
    }
    if (lane == kWave - 1) sh.toff[E] = trun;
  }
  __syncthreads();

  // Pass 3: map / inverse map.
  int valid_rows = 0;
  if (E > 0) valid_rows = sh.off[E - 1] + sh.run[E - 1];
  for (int q = tid; q < a.R; q += kPlanThreads) {
    long long idv;
    int rank;
    if (LDSR) {
      idv = s_ids[q];
      rank = s_rank[q];
      if (rank >= 0) {
        rank += sh.wcnt[0][q / CH][idv];
        a.ranks[q] = rank;
      } else {
        a.ranks[q] = -1;
      }
    } else {
      idv = (long long)ids[q];
      rank = a.ranks[q];  // written by this thread in pass 1
    }
    if (idv >= 0 && idv < E) {
      const int p = sh.off[idv] + rank;
      a.map[q] = p;
      a.row_route[p] = q;
      a.row_token[p] = q / a.K;
    } else {
      a.map[q] = -1;
    }
  }
  for (int p = valid_rows + tid; p < a.R; p += kPlanThreads) {
    a.row_route[p] = -1;
    a.row_token[p] = 0;
  }

  // Pass 4: task list, expert-major.
  for (int e = tid; e < E; e += kPlanThreads) {
    const int c = sh.run[e];
    const int tb = a.token_block;
    int t0 = sh.toff[e];
    for (int r0 = 0; r0 < c; r0 += tb, ++t0)
      a.tasks[t0] = make_int4(e, sh.off[e] + r0, min(tb, c - r0), 0);
  }
  if (flags) atomicOr(&sh.status, flags);
  __syncthreads();
  if (tid == 0) {
    *a.num_tasks = sh.toff[E];
    a.status[0] = sh.status;
  }
}

// ---- multi-workgroup router + planner --------------------------------------
//
// For every shape the single-workgroup planner does not route itself (T > 32
// with logits, or any fixed-route shape), one launch of W workgroups routes
// and plans: workgroup w owns tokens [w*TPW, (w+1)*TPW) (16 tokens, one per
// wave, with the router; 1024 / K tokens with fixed routes) and
//  1. routes its tokens (router mode) or loads their ids and weights,
//  2. ranks its routes canonically within its chunk (wave-ballot match, then
//     a prefix over its waves) and counts them per expert,
//  3. publishes its per-expert counts and status bits to the other
//     workgroups as 32-bit words tagged with this launch's epoch in the high
//     half (agent-scope stores; the readers re-read a word until its tag is
//     the epoch, so no fence or barrier orders the exchange),
//  4. reads every workgroup's counts: base[e] = routes of expert e in earlier
//     chunks, total[e] = routes of expert e; offsets and task offsets are
//     exclusive scans of the totals, and rank[q] = base[e] + chunk rank, which
//     is the canonical rank #{q' < q : id[q'] == e} because chunks are in
//     route order;
//  5. writes ranks, map, row_route and row_token of its routes; workgroup 0
//     also writes counts, offsets, the task list, num_tasks and status, and
//     finally advances the epoch (every other workgroup read it before
//     publishing, and workgroup 0 has seen every publication).
// All W <= CU count workgroups are resident at once (one launch, nothing else
// on the stream), so every awaited word is being produced; a wait that still
// exceeds its spin bound sets status bit MOE_STATUS_STALLED instead of hanging.
constexpr int kMultiThreads = 1024;
constexpr int kMultiWaves = kMultiThreads / kWave;
constexpr int kMultiBatch = 16;  // published words read per thread per round trip

__device__ __forceinline__ uint32_t coherent_load(const uint32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coherent_store(uint32_t *p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Tag of the epoch value e: never 0, so a zeroed word is never taken as published.
__device__ __forceinline__ uint32_t epoch_tag(uint32_t e) { return (e & 0x7fffu) | 0x8000u; }

template <typename IdT, bool ROUTER>
__global__ __launch_bounds__(kMultiThreads) void route_plan_multi_kernel(RouteArgs a) {
  __shared__ int s_ids[kMultiThreads];
  __shared__ float s_w[kMultiThreads];
  __shared__ int s_lrank[kMultiThreads];
  __shared__ int s_wcnt[kMultiWaves][kMaxExperts];
  __shared__ int s_base[kMaxExperts], s_tot[kMaxExperts], s_off[kMaxExperts], s_toff[kMaxExperts + 1];
  __shared__ uint32_t s_flags, s_all_flags;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & (kWave - 1);
  const int E = a.E, K = a.K, W = gridDim.x, w = blockIdx.x;
  const int tpw = a.plan_tpw;
  const int t0 = w * tpw, t1 = min(a.T, t0 + tpw);
  const int q0 = t0 * K, nq = (t1 - t0) * K;  // <= kMultiThreads
  uint32_t *const part = (uint32_t *)a.partials;

  // 1. routes of this chunk into LDS.  The logits are requested before the
  // epoch word, whose device-coherent load is another memory round trip:
  // the two overlap instead of the logits waiting behind it.  With E <= 128
  // each token is routed by a half-wave, so the chunk's 16 tokens take 8
  // waves; else one token per wave.  (16 lanes per token, with 16, 32 or 64
  // tokens per workgroup, measured 0.3-2 us slower at T = 193 and no faster
  // at T = 1024: this launch is bound by latency, not by issue.)
  const bool half = ROUTER && E <= 128;
  float raw[4];
  const int rt = half ? t0 + 2 * wave + (lane >> 5) : t0 + wave;
  if (ROUTER) {
    if (half) load_token_logits<true>(a.logits, rt, rt < t1, E, raw);
    else load_token_logits<false>(a.logits, rt, rt < t1, E, raw);
  }
  const uint32_t epoch = coherent_load(a.status + 2);
  // status[1]: bits of a separate router launch earlier on this stream, read
  // now so the last workgroup's final writes wait on no load.
  const uint32_t router_bits = !ROUTER && tid == 0 ? a.status[1] : 0u;
  if (tid == 0) {
    s_flags = 0;
    s_all_flags = 0;
  }
  for (int i = tid; i < kMultiWaves * kMaxExperts; i += kMultiThreads) (&s_wcnt[0][0])[i] = 0;
  uint32_t flags = 0;
  if constexpr (ROUTER) {
    if (half) {
      if (t0 + 2 * wave < t1)
        route_token<true>(raw, rt, rt < t1, E, K, a.renormalize, (int32_t *)a.ids, a.weights, flags,
                          s_ids - q0, s_w - q0);
    } else if (rt < t1) {
      route_token<false>(raw, rt, true, E, K, a.renormalize, (int32_t *)a.ids, a.weights, flags,
                         s_ids - q0, s_w - q0);
    }
  } else {
    if (tid < nq) {
      const long long idv = (long long)((const IdT *)a.ids)[q0 + tid];
      s_ids[tid] = idv >= 0 && idv < E ? (int)idv : -1;
      s_w[tid] = a.weights[q0 + tid];
    }
  }
  __syncthreads();
  const uint32_t tag = epoch_tag(__builtin_amdgcn_readfirstlane(epoch));

  // 2. chunk-local canonical ranks and per-expert counts.
  const bool valid = tid < nq;
  const int idv = valid ? s_ids[tid] : -1;
  const bool ok = idv >= 0;
  if (valid && !ok) flags |= 1u;
  if (valid && !isfinite(s_w[tid])) flags |= 2u;
  const int id = ok ? idv : 0;
  uint64_t match = __ballot(ok);
  const int nbits = id_bits(E);
#pragma unroll
  for (int bit = 0; bit < 8; ++bit) {
    if (bit >= nbits) break;
    const bool set = (id >> bit) & 1;
    const uint64_t b = __ballot(ok && set);
    match &= set ? b : ~b;
  }
  const int lrank = __popcll(match & lanemask_lt());
  if (ok && lrank == 0) s_wcnt[wave][id] = __popcll(match);
  if (flags) atomicOr(&s_flags, flags);
  __syncthreads();
  for (int e = tid; e < E; e += kMultiThreads) {
    int run = 0;
#pragma unroll
    for (int v = 0; v < kMultiWaves; ++v) {
      const int c = s_wcnt[v][e];
      s_wcnt[v][e] = run;
      run += c;
    }
    // 3. publish the chunk's count of expert e.
    if (w != a.plan_hold_wg) coherent_store(part + (size_t)w * (E + 1) + e, (tag << 16) | (uint32_t)run);
  }
  if (tid == 0 && w != a.plan_hold_wg) coherent_store(part + (size_t)w * (E + 1) + E, (tag << 16) | s_flags);
  __syncthreads();
  if (ok) s_lrank[tid] = s_wcnt[wave][id] + lrank;

  // 4. every chunk's counts.  The W x (E + 1) published words are spread over
  // the workgroup's threads, kMultiBatch per request batch: all of a batch's
  // loads are in flight before any tag is checked (one memory round trip per
  // batch, not per word; 64 router workgroups x 129 words at T = 1024 fit one
  // batch of 16 per thread, where 8 per thread needed a second round trip).
  // Integer sums, so the order of the LDS additions does not matter.
  for (int e = tid; e < E; e += kMultiThreads) {
    s_base[e] = 0;
    s_tot[e] = 0;
  }
  __syncthreads();
  bool stalled = false;
  {
    const int nwords = W * (E + 1);
    uint32_t fl = 0;
    for (int j0 = 0; j0 < nwords; j0 += kMultiBatch * kMultiThreads) {
      uint32_t v[kMultiBatch];
      // The whole batch is re-read (all its loads in flight again) until
      // every tag has arrived.
      for (int n = 0;; ++n) {
#pragma unroll
        for (int i = 0; i < kMultiBatch; ++i) {
          const int j = j0 + i * kMultiThreads + tid;
          v[i] = j < nwords ? coherent_load(part + j) : (tag << 16);
        }
        bool all = true;
#pragma unroll
        for (int i = 0; i < kMultiBatch; ++i) all &= (v[i] >> 16) == tag;
        if (all) break;
        if (n >= a.plan_spin_cap) {
          stalled = true;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
#pragma unroll
      for (int i = 0; i < kMultiBatch; ++i) {
        const int j = j0 + i * kMultiThreads + tid;
        if (j >= nwords) continue;
        const uint32_t c = v[i] & 0xffffu;
        const int src = j / (E + 1), e = j - src * (E + 1);
        // A word that cannot have been published by workgroup src (a count
        // above its route count, unknown flag bits) marks the plan invalid,
        // so no index is ever formed from it.
        const int src_routes = (min(a.T, (src + 1) * tpw) - src * tpw) * K;
        if (e == E) {
          if (c & ~7u) stalled = true;
          fl |= c & 7u;
        } else if ((int)c > src_routes) {
          stalled = true;
        } else if (c) {
          atomicAdd(&s_tot[e], (int)c);
          if (src < w) atomicAdd(&s_base[e], (int)c);
        }
      }
    }
    if (stalled) fl |= kStatusStalled;
    if (fl) atomicOr(&s_all_flags, fl);
  }
  __syncthreads();
  if (wave == 0) {
    const int tb = a.token_block;
    int c[4], nt[4], csum = 0, tsum = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane * 4 + j;
      c[j] = e < E ? s_tot[e] : 0;
      nt[j] = (c[j] + tb - 1) / tb;
      csum += c[j];
      tsum += nt[j];
    }
    int crun = wave_incl_scan(csum) - csum, trun = wave_incl_scan(tsum) - tsum;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane * 4 + j;
      if (e < E) {
        s_off[e] = crun;
        s_toff[e] = trun;
        if (w == 0) {
          a.counts[e] = c[j];
          a.offsets[e] = crun;
        }
      }
      crun += c[j];
      trun += nt[j];
    }
    if (lane == kWave - 1) {
      s_toff[E] = trun;
      // Totals above R (possible only from words that were never published
      // in this launch) would place rows past the arrays.
      if (crun > a.R) atomicOr(&s_all_flags, kStatusStalled);
    }
  }
  __syncthreads();

  // 5. this chunk's rows; workgroup 0 the expert-level arrays.  A workgroup
  // whose view is incomplete (a wait ran out, or a word failed its bounds)
  // writes nothing.  Every workgroup then arrives on one counter, carrying
  // whether its view was complete; the last to arrive is the only writer of
  // status[0], num_tasks and the epoch: the task count when every view was
  // complete, else no tasks and MOE_STATUS_STALLED, so the GEMMs never read
  // rows a workgroup did not write.  It runs after every workgroup of the
  // launch has read the epoch (each reads it before it arrives), so no
  // workgroup of this launch can see the advanced value, and words left by
  // this launch never carry the next launch's tag.
  const uint32_t all_flags = s_all_flags;
  const bool bad = (all_flags & kStatusStalled) != 0;
  uint32_t *const arrive = part + (size_t)W * (E + 1);
  uint32_t before = 0;
  if (tid == 0)
    before = __hip_atomic_fetch_add(arrive, 1u + (bad ? 1u << 16 : 0u), __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
  if (!bad) {
    if (valid) {
      const int q = q0 + tid;
      if (ok) {
        const int rank = s_base[id] + s_lrank[tid];
        const int p = s_off[id] + rank;
        a.ranks[q] = rank;
        a.map[q] = p;
        a.row_route[p] = q;
        a.row_token[p] = q / K;
      } else {
        a.ranks[q] = -1;
        a.map[q] = -1;
      }
    }
    if (w == 0) {
      const int valid_rows = s_off[E - 1] + s_tot[E - 1];
      for (int p = valid_rows + tid; p < a.R; p += kMultiThreads) {
        a.row_route[p] = -1;
        a.row_token[p] = 0;
      }
      const int tb = a.token_block;
      for (int e = tid; e < E; e += kMultiThreads) {
        const int c = s_tot[e];
        int tt = s_toff[e];
        for (int r0 = 0; r0 < c; r0 += tb, ++tt) a.tasks[tt] = make_int4(e, s_off[e] + r0, min(tb, c - r0), 0);
      }
      if (tid == 0) a.counters[0] = a.counters[1] = a.counters[2] = a.counters[3] = 0;
    }
  }
  if (tid == 0 && (before & 0xffffu) == (uint32_t)W - 1u) {
    const bool any_bad = bad || (before >> 16) != 0;
    uint32_t st = router_bits | (any_bad ? (all_flags & 7u) | kStatusStalled : all_flags);
    a.status[0] = st;
    a.status[1] = 0;
    *a.num_tasks = any_bad ? 0 : s_toff[E];
    coherent_store(arrive, 0u);
    coherent_store(a.status + 2, epoch + 1u);  // every workgroup read this epoch
  }
}

}  // namespace

hipError_t launch_router(const RouteArgs &a, hipStream_t s) {
  if (a.T == 0) return hipSuccess;
  hipLaunchKernelGGL(router_kernel, dim3((a.T + 3) / 4), dim3(256), 0, s, a);
  return hipGetLastError();
}

bool multi_plan_ok(int T, int K, int E, bool router, int num_cus) {
  const int tpw = multi_plan_tokens(K, E, router);
  return T > 0 && tpw > 0 && (T + tpw - 1) / tpw <= num_cus && num_cus <= 4096;
}

// Tokens per planner workgroup: with the router 16 (one per wave or
// half-wave); fixed routes 1024 / K (one route per thread).
int multi_plan_tokens(int K, int E, bool router) {
  (void)E;
  if (router) return K <= kMultiThreads / kMultiWaves ? kMultiWaves : 0;
  return K <= kMultiThreads ? kMultiThreads / K : 0;
}

hipError_t launch_route_plan_multi(const RouteArgs &a, hipStream_t s) {
  const int W = (a.T + a.plan_tpw - 1) / a.plan_tpw;
  if (W <= 0) return hipSuccess;
#define MOE_MPLAN(T, R) \
  hipLaunchKernelGGL((route_plan_multi_kernel<T, R>), dim3(W), dim3(kMultiThreads), 0, s, a)
  if (a.route_logits) MOE_MPLAN(int32_t, true);
  else if (a.id64) MOE_MPLAN(long long, false);
  else MOE_MPLAN(int32_t, false);
#undef MOE_MPLAN
  return hipGetLastError();
}

hipError_t launch_route_plan(const RouteArgs &a, hipStream_t s) {
  const bool lds = a.R <= kLdsRoutes;
#define MOE_PLAN(T, L) hipLaunchKernelGGL((route_plan_kernel<T, L>), dim3(1), dim3(kPlanThreads), 0, s, a)
  if (a.id64) {
    if (lds) MOE_PLAN(long long, true); else MOE_PLAN(long long, false);
  } else {
    if (lds) MOE_PLAN(int32_t, true); else MOE_PLAN(int32_t, false);
  }
#undef MOE_PLAN
  return hipGetLastError();
}

}  // namespace moe
