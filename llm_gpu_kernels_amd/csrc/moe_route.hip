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
// Selection is by logit (softmax is monotone): K rounds of a wave max over
// the remaining keys, then the lowest expert index holding that key, so the
// top-k come out in slot order with ties to the lower index.  NaN logits
// rank below every number and set the logit flag.
__device__ void route_token(const float *__restrict__ logits, int t, int E, int K,
                            int renormalize, int32_t *__restrict__ ids_out,
                            float *__restrict__ w_out, uint32_t &flags) {
  const int lane = threadIdx.x & (kWave - 1);
  float raw[4];
  uint32_t key[4];
  bool bad = false;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + kWave * j;
    raw[j] = e < E ? logits[(size_t)t * E + e] : -INFINITY;
    bad |= (e < E) && !isfinite(raw[j]);
    key[j] = e < E ? float_key(raw[j]) : 0u;
  }
  if (__any(bad)) flags |= 4u;
  uint32_t top = umax_(umax_(key[0], key[1]), umax_(key[2], key[3]));
  const float m = key_float(wave_umax(top));
  float z = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (lane + kWave * j < E) z += expf(raw[j] - m);
  z = wave_fsum(z);

  uint32_t taken = 0;
  float my_p = 0.f, psum = 0.f;
  int my_id = 0;
  for (int k = 0; k < K; ++k) {
    uint32_t best = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (!((taken >> j) & 1)) best = umax_(best, key[j]);
    const uint32_t M = wave_umax(best);
    uint32_t cand = 0xffffu;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane + kWave * j;
      if (e < E && !((taken >> j) & 1) && key[j] == M) cand = umin_(cand, (uint32_t)e);
    }
    const int idx = (int)wave_umin(cand);
    if ((idx & (kWave - 1)) == lane) taken |= 1u << (idx / kWave);
    const float p = expf(key_float(M) - m) / z;
    psum += p;
    if (lane == k) {
      my_p = p;
      my_id = idx;
    }
  }
  if (lane < K) {
    ids_out[(size_t)t * K + lane] = my_id;
    w_out[(size_t)t * K + lane] = renormalize ? my_p / psum : my_p;
  }
}

__global__ __launch_bounds__(256) void router_kernel(RouteArgs a) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  uint32_t flags = 0;
  if (t < a.T)
    route_token(a.logits, t, a.E, a.K, a.renormalize, (int32_t *)a.ids, a.weights, flags);
  if (flags && (threadIdx.x & 63) == 0) atomicOr(&a.status[1], flags);
}

template <typename IdT>
__global__ __launch_bounds__(kPlanThreads) void route_plan_kernel(RouteArgs a) {
  __shared__ int s_wcnt[kPlanWaves][kMaxExperts];
  __shared__ int s_run[kMaxExperts];
  __shared__ int s_off[kMaxExperts];
  __shared__ int s_toff[kMaxExperts + 1];
  __shared__ uint32_t s_status;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & (kWave - 1);
  const int E = a.E;
  if (tid == 0) s_status = 0;
  for (int e = tid; e < E; e += kPlanThreads) s_run[e] = 0;
  uint32_t flags = 0;

  if (a.route_logits) {
    if (a.fuse_router) {
      for (int t = wave; t < a.T; t += kPlanWaves)
        route_token(a.logits, t, E, a.K, a.renormalize, (int32_t *)a.ids, a.weights, flags);
    } else if (tid == 0) {
      flags |= a.status[1];  // written by router_kernel earlier on this stream
      a.status[1] = 0;
    }
  }
  // The router's global writes become visible to the whole workgroup here.
  __threadfence_block();
  __syncthreads();

  const IdT *ids = (const IdT *)a.ids;
  // Pass 1: canonical ranks, 1024 routes per round.
  for (int base = 0; base < a.R; base += kPlanThreads) {
    for (int i = tid; i < kPlanWaves * kMaxExperts; i += kPlanThreads) (&s_wcnt[0][0])[i] = 0;
    __syncthreads();
    const int q = base + tid;
    const bool valid = q < a.R;
    long long idv = -1;
    float wv = 0.f;
    if (valid) {
      idv = (long long)ids[q];
      wv = a.weights[q];
    }
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
    if (ok && lrank == 0) s_wcnt[wave][id] = __popcll(match);
    __syncthreads();
    if (ok) {
      int r = s_run[id] + lrank;
      for (int w = 0; w < wave; ++w) r += s_wcnt[w][id];
      a.ranks[q] = r;
    } else if (valid) {
      a.ranks[q] = -1;
    }
    __syncthreads();
    for (int e = tid; e < E; e += kPlanThreads) {
      int c = 0;
      for (int w = 0; w < kPlanWaves; ++w) c += s_wcnt[w][e];
      s_run[e] += c;
    }
    __syncthreads();
  }

  // Pass 2: exclusive scans of counts and of per-expert task counts (wave 0,
  // four experts per lane).
  if (wave == 0) {
    const int tb = a.token_block;
    int c[4], nt[4], csum = 0, tsum = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane * 4 + j;
      c[j] = e < E ? s_run[e] : 0;
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
        s_off[e] = crun;
        s_toff[e] = trun;
        a.counts[e] = c[j];
        a.offsets[e] = crun;
      }
      crun += c[j];
      trun += nt[j];
    }
    if (lane == kWave - 1) s_toff[E] = trun;
  }
  __syncthreads();

  // Pass 3: map / inverse map (each thread rereads the ranks it wrote).
  int valid_rows = 0;
  if (E > 0) valid_rows = s_off[E - 1] + s_run[E - 1];
  for (int q = tid; q < a.R; q += kPlanThreads) {
    const long long idv = (long long)ids[q];
    if (idv >= 0 && idv < E) {
      const int p = s_off[idv] + a.ranks[q];
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
    const int c = s_run[e];
    const int tb = a.token_block;
    int t0 = s_toff[e];
    for (int r0 = 0; r0 < c; r0 += tb, ++t0)
      a.tasks[t0] = make_int4(e, s_off[e] + r0, min(tb, c - r0), 0);
  }
  if (flags) atomicOr(&s_status, flags);
  __syncthreads();
  if (tid == 0) {
    *a.num_tasks = s_toff[E];
    a.status[0] = s_status;
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
  if (a.id64)
    hipLaunchKernelGGL(route_plan_kernel<long long>, dim3(1), dim3(kPlanThreads), 0, s, a);
  else
    hipLaunchKernelGGL(route_plan_kernel<int32_t>, dim3(1), dim3(kPlanThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace moe
