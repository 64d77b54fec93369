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

}  // namespace

hipError_t launch_router(const RouteArgs &a, hipStream_t s) {
  if (a.T == 0) return hipSuccess;
  hipLaunchKernelGGL(router_kernel, dim3((a.T + 3) / 4), dim3(256), 0, s, a);
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
