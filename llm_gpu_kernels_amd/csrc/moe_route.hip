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

namespace moe {

namespace {

constexpr int kPlanThreads = 1024;
constexpr int kPlanWaves = kPlanThreads / kWave;
constexpr int kMaxExperts = 256;

// Wave-wide reductions from DPP row permutes (quad xor 1, quad xor 2, half-row
// mirror, row mirror) and four v_readlane: every lane gets the result.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xf, 0xf, false);
}
#define MOE_DPP_REDUCE(T, OP, TOBITS, FROMBITS)                                   \
  v = OP(v, FROMBITS(dpp_u<0xb1>(TOBITS(v))));                                     \
  v = OP(v, FROMBITS(dpp_u<0x4e>(TOBITS(v))));                                     \
  v = OP(v, FROMBITS(dpp_u<0x141>(TOBITS(v))));                                    \
  v = OP(v, FROMBITS(dpp_u<0x140>(TOBITS(v))));                                    \
  {                                                                               \
    const T a0 = FROMBITS((uint32_t)__builtin_amdgcn_readlane((int)TOBITS(v), 0));  \
    const T a1 = FROMBITS((uint32_t)__builtin_amdgcn_readlane((int)TOBITS(v), 16)); \
    const T a2 = FROMBITS((uint32_t)__builtin_amdgcn_readlane((int)TOBITS(v), 32)); \
    const T a3 = FROMBITS((uint32_t)__builtin_amdgcn_readlane((int)TOBITS(v), 48)); \
    v = OP(OP(a0, a1), OP(a2, a3));                                               \
  }
#define MOE_ID(x) (x)
__device__ __forceinline__ uint32_t umax_(uint32_t a, uint32_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint32_t umin_(uint32_t a, uint32_t b) { return a < b ? a : b; }
__device__ __forceinline__ float fadd_(float a, float b) { return a + b; }
__device__ __forceinline__ uint32_t wave_umax(uint32_t v) {
  MOE_DPP_REDUCE(uint32_t, umax_, MOE_ID, MOE_ID)
  return v;
}
__device__ __forceinline__ uint32_t wave_umin(uint32_t v) {
  MOE_DPP_REDUCE(uint32_t, umin_, MOE_ID, MOE_ID)
  return v;
}
__device__ __forceinline__ float wave_fsum(float v) {
  MOE_DPP_REDUCE(float, fadd_, __float_as_uint, __uint_as_float)
  return v;
}
#undef MOE_DPP_REDUCE
#undef MOE_ID

// Order-preserving map of a float to uint32 (NaN -> 0, below -inf).
__device__ __forceinline__ uint32_t float_key(float f) {
  if (isnan(f)) return 0u;
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_float(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// One wave routes token t.  Expert e lives in lane e % 64, slot e / 64.
// Selection is by logit (softmax is monotone): K rounds of a DPP wave max
// over the remaining keys; the lowest expert holding the max is the first
// set bit of the first non-empty per-slot ballot (slot j holds experts
// 64j + lane), all scalar.  Lane k keeps the key and expert of slot k and
// the probabilities are formed once, after the loop.  NaN logits rank below
// every number and set the logit flag.  Results go to global memory and,
// when `lds_ids` is given, to LDS for the planner.
__device__ void route_token(const float *__restrict__ logits, int t, int E, int K,
                            int renormalize, int32_t *__restrict__ ids_out,
                            float *__restrict__ w_out, uint32_t &flags, int *lds_ids,
                            float *lds_w) {
  const int lane = threadIdx.x & (kWave - 1);
  float raw[4];
  uint32_t key[4];
  bool bad = false;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + kWave * j;
    raw[j] = e < E ? logits[(size_t)t * E + e] : -INFINITY;
    bad |= e < E && !isfinite(raw[j]);
    key[j] = e < E ? float_key(raw[j]) : 0u;
  }
  if (__any(bad)) flags |= 4u;
  const uint32_t top = umax_(umax_(key[0], key[1]), umax_(key[2], key[3]));
  const float m = key_float(wave_umax(top));
  float z = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (lane + kWave * j < E) z += expf(raw[j] - m);
  z = wave_fsum(z);

  uint32_t taken = 0, my_key = 0;
  int my_id = 0;
  for (int k = 0; k < K; ++k) {
    uint32_t best = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (!((taken >> j) & 1)) best = umax_(best, key[j]);
    const uint32_t M = wave_umax(best);
    int idx = kMaxExperts;
#pragma unroll
    for (int j = 3; j >= 0; --j) {  // lowest slot wins: scan from the top down
      const uint64_t hit = __ballot(lane + kWave * j < E && !((taken >> j) & 1) && key[j] == M);
      idx = hit ? kWave * j + (int)__builtin_ctzll(hit) : idx;
    }
    if ((idx & (kWave - 1)) == lane) taken |= 1u << (idx / kWave);
    if (lane == k) {
      my_key = M;
      my_id = idx;
    }
  }
  const float p = lane < K ? expf(key_float(my_key) - m) / z : 0.f;
  float psum = 0.f;
  for (int k = 0; k < K; ++k) psum += __shfl(p, k, kWave);  // slot order, every lane alike
  if (lane < K) {
    const int q = t * K + lane;
    const float w = renormalize ? p / psum : p;
    ids_out[q] = my_id;
    w_out[q] = w;
    if (lds_ids) {
      lds_ids[q] = my_id;
      lds_w[q] = w;
    }
  }
}

// Half-wave reductions: every lane gets the result over its 32-lane half
// (DPP within each 16-lane row, then the gfx950 row-pair swap).
__device__ __forceinline__ uint32_t half_umax(uint32_t v) {
  v = umax_(v, dpp_u<0xb1>(v));
  v = umax_(v, dpp_u<0x4e>(v));
  v = umax_(v, dpp_u<0x141>(v));
  v = umax_(v, dpp_u<0x140>(v));
  const auto q = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return umax_(q[0], q[1]);
}
__device__ __forceinline__ float half_fsum(float x) {
  uint32_t v = __float_as_uint(x);
  v = __float_as_uint(__uint_as_float(v) + __uint_as_float(dpp_u<0xb1>(v)));
  v = __float_as_uint(__uint_as_float(v) + __uint_as_float(dpp_u<0x4e>(v)));
  v = __float_as_uint(__uint_as_float(v) + __uint_as_float(dpp_u<0x141>(v)));
  v = __float_as_uint(__uint_as_float(v) + __uint_as_float(dpp_u<0x140>(v)));
  const auto q = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// route_token for two tokens per wave (E <= 128): half h = lane / 32 routes
// token t of its own; expert e lives in lane 32h + e % 32, slot e / 32.  The
// same selection (by logit, ties to the lower expert) and probabilities; a
// half with live == false computes on -inf logits and stores nothing.
__device__ void route_token_half(const float *__restrict__ logits, int t, bool live, int E, int K,
                                 int renormalize, int32_t *__restrict__ ids_out,
                                 float *__restrict__ w_out, uint32_t &flags, int *lds_ids,
                                 float *lds_w) {
  const int lane = threadIdx.x & (kWave - 1);
  const int h = lane & 31;
  const bool upper = lane >= 32;
  float raw[4];
  uint32_t key[4];
  bool bad = false;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = h + 32 * j;
    const bool ok = live && e < E;
    raw[j] = ok ? logits[(size_t)t * E + e] : -INFINITY;
    bad |= ok && !isfinite(raw[j]);
    key[j] = ok ? float_key(raw[j]) : 0u;
  }
  if (__any(bad)) flags |= 4u;
  const uint32_t top = umax_(umax_(key[0], key[1]), umax_(key[2], key[3]));
  const float m = key_float(half_umax(top));
  float z = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (live && h + 32 * j < E) z += expf(raw[j] - m);
  z = half_fsum(z);

  uint32_t taken = 0, my_key = 0;
  int my_id = 0;
  for (int k = 0; k < K; ++k) {
    uint32_t best = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (!((taken >> j) & 1)) best = umax_(best, key[j]);
    const uint32_t M = half_umax(best);
    int idx_lo = kMaxExperts, idx_hi = kMaxExperts;
#pragma unroll
    for (int j = 3; j >= 0; --j) {  // lowest slot wins: scan from the top down
      const uint64_t hit = __ballot(live && h + 32 * j < E && !((taken >> j) & 1) && key[j] == M);
      const uint32_t lo = (uint32_t)hit, hi = (uint32_t)(hit >> 32);
      idx_lo = lo ? 32 * j + (int)__builtin_ctz(lo) : idx_lo;
      idx_hi = hi ? 32 * j + (int)__builtin_ctz(hi) : idx_hi;
    }
    const int idx = upper ? idx_hi : idx_lo;
    if ((idx & 31) == h) taken |= 1u << (idx / 32);
    if (h == k) {
      my_key = M;
      my_id = idx;
    }
  }
  const float p = h < K ? expf(key_float(my_key) - m) / z : 0.f;
  float psum = 0.f;
  const int base = upper ? 32 : 0;
  for (int k = 0; k < K; ++k) psum += __shfl(p, base + k, kWave);  // slot order
  if (live && h < K) {
    const int q = t * K + h;
    const float w = renormalize ? p / psum : p;
    ids_out[q] = my_id;
    w_out[q] = w;
    if (lds_ids) {
      lds_ids[q] = my_id;
      lds_w[q] = w;
    }
  }
}

__global__ __launch_bounds__(256) void router_kernel(RouteArgs a) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  uint32_t flags = 0;
  if (t < a.T)
    route_token(a.logits, t, a.E, a.K, a.renormalize, (int32_t *)a.ids, a.weights, flags,
                nullptr, nullptr);
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
  if (tid == 0) sh.status = 0;
  for (int e = tid; e < E; e += kPlanThreads) sh.run[e] = 0;
  for (int i = tid; i < kPlanWaves * kMaxExperts; i += kPlanThreads) (&sh.wcnt[0][0][0])[i] = 0;
  uint32_t flags = 0;

  bool ids_in_lds = false;
  if (a.route_logits) {
    if (LDSR && a.fuse_router == 2) {  // T <= 32, E <= 128: two tokens per wave
      const int t = 2 * wave + (lane >> 5);
      if (2 * wave < a.T)
        route_token_half(a.logits, t, t < a.T, E, a.K, a.renormalize, (int32_t *)a.ids,
                         a.weights, flags, s_ids, s_w);
      ids_in_lds = true;
    } else if (LDSR && a.fuse_router) {  // T <= 16: one token per wave
      for (int t = wave; t < a.T; t += kPlanWaves)
        route_token(a.logits, t, E, a.K, a.renormalize, (int32_t *)a.ids, a.weights, flags,
                    s_ids, s_w);
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
    int cinc = csum, tinc = tsum;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int cu = __shfl_up(cinc, o, kWave);
      const int tu = __shfl_up(tinc, o, kWave);
      if (lane >= o) {
        cinc += cu;
        tinc += tu;
      }
    }
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
    a.counters[0] = 0;
    a.counters[1] = 0;
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
