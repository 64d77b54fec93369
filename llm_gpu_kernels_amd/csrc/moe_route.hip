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

// One wave routes token t.  Expert e lives in lane e % 64, slot e / 64.
// Selection is by logit (softmax is monotone), largest first, ties to the
// lower expert index; NaN logits sort below every number.
__device__ void route_token(const float *__restrict__ logits, int t, int E, int K,
                            int renormalize, int32_t *__restrict__ ids_out,
                            float *__restrict__ w_out, uint32_t &flags) {
  const int lane = threadIdx.x & (kWave - 1);
  float raw[4], key[4];
  bool bad = false;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + kWave * j;
    if (e < E) {
      const float v = logits[(size_t)t * E + e];
      bad |= !isfinite(v);
      raw[j] = v;
      key[j] = isnan(v) ? -INFINITY : v;
    } else {
      raw[j] = -INFINITY;
      key[j] = -INFINITY;
    }
  }
  float m = fmaxf(fmaxf(key[0], key[1]), fmaxf(key[2], key[3]));
  m = wave_max(m);
  float z = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (lane + kWave * j < E) z += expf(raw[j] - m);
  z = wave_sum(z);
  if (__any(bad)) flags |= 4u;

  uint32_t taken = 0;
  float my_p = 0.f;
  int my_id = 0;
  float psum = 0.f;
  for (int k = 0; k < K; ++k) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane + kWave * j;
      if (e < E && !(taken & (1u << j)) && (key[j] > bv || (key[j] == bv && e < bi))) {
        bv = key[j];
        bi = e;
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, kWave);
      const int oi = __shfl_xor(bi, o, kWave);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if ((bi & (kWave - 1)) == lane) taken |= 1u << (bi / kWave);
    const float rv = __shfl(raw[0], bi & (kWave - 1), kWave);
    const float rv1 = __shfl(raw[1], bi & (kWave - 1), kWave);
    const float rv2 = __shfl(raw[2], bi & (kWave - 1), kWave);
    const float rv3 = __shfl(raw[3], bi & (kWave - 1), kWave);
    const int slot = bi / kWave;
    const float xv = slot == 0 ? rv : slot == 1 ? rv1 : slot == 2 ? rv2 : rv3;
    const float p = expf(xv - m) / z;
    psum += p;
    if (lane == k) {
      my_p = p;
      my_id = bi;
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
    } else {
      a.map[q] = -1;
    }
  }
  for (int p = valid_rows + tid; p < a.R; p += kPlanThreads) a.row_route[p] = -1;

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
