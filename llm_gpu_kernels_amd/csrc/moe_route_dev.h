// Device-side routing helpers shared by the planner (moe_route.hip) and the
// streaming gate/up kernel that plans in its prologue (moe_dma.hip):
// wave-level reductions, the softmax -> top-k -> renormalise router for one
// token per wave or half-wave, and a prefix scan.
#pragma once

#include "common.h"

namespace moe {
namespace route_dev {

constexpr int kMaxExperts = 256;

// DPP row permute of one dword (quad xor 1 = 0xb1, quad xor 2 = 0x4e, half-row
// mirror = 0x141, row mirror = 0x140).
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xf, 0xf, false);
}

// Order-preserving map of a float to uint32 (NaN -> 0, below -inf).
__device__ __forceinline__ uint32_t float_key(float f) {
  if (isnan(f)) return 0u;
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_float(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Reductions over the L lanes routing one token (L = 64, 32 or 16): DPP
// within 16-lane rows, then gfx950's row-pair and half swaps; every lane of
// the group gets the result.  The float sum adds rows as (r0 + r1) + (r2 + r3).
template <int L>
__device__ __forceinline__ float group_fsum_l(float x) {
  static_assert(L == 16 || L == 32 || L == 64, "lanes per token");
  uint32_t v = __float_as_uint(x);
  v = __float_as_uint(__uint_as_float(v) + __uint_as_float(dpp_u<0xb1>(v)));
  v = __float_as_uint(__uint_as_float(v) + __uint_as_float(dpp_u<0x4e>(v)));
  v = __float_as_uint(__uint_as_float(v) + __uint_as_float(dpp_u<0x141>(v)));
  v = __float_as_uint(__uint_as_float(v) + __uint_as_float(dpp_u<0x140>(v)));
  if (L >= 32) {
    const auto q = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = __float_as_uint(__uint_as_float(q[0]) + __uint_as_float(q[1]));
  }
  if (L == 64) {
    const auto h = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    v = __float_as_uint(__uint_as_float(h[0]) + __uint_as_float(h[1]));
  }
  return __uint_as_float(v);
}
template <bool HALF>
__device__ __forceinline__ float group_fsum(float x) {
  return group_fsum_l<HALF ? 32 : 64>(x);
}
// Inclusive prefix sum over the wave: DPP row shifts, then row broadcasts
// (lane 15 into rows 1 and 3, lane 31 into rows 2 and 3).
template <int CTRL, int ROWS = 0xf, int BANKS = 0xf>
__device__ __forceinline__ int dpp_add(int v, int src) {
  return v + __builtin_amdgcn_update_dpp(0, src, CTRL, ROWS, BANKS, false);
}
__device__ __forceinline__ int wave_incl_scan(int x) {
  int v = dpp_add<0x111>(x, x);           // row_shr:1
  v = dpp_add<0x112>(v, x);               // row_shr:2
  v = dpp_add<0x113>(v, x);               // row_shr:3
  v = dpp_add<0x114, 0xf, 0xe>(v, v);     // row_shr:4, banks 1-3
  v = dpp_add<0x118, 0xf, 0xc>(v, v);     // row_shr:8, banks 2-3
  v = dpp_add<0x142, 0xa, 0xf>(v, v);     // row_bcast:15 into rows 1, 3
  v = dpp_add<0x143, 0xc, 0xf>(v, v);     // row_bcast:31 into rows 2, 3
  return v;
}

template <int L, bool MAX>
__device__ __forceinline__ uint32_t group_uext_l(uint32_t v) {
  static_assert(L == 16 || L == 32 || L == 64, "lanes per token");
  auto op = [](uint32_t a, uint32_t b) { return MAX ? (a > b ? a : b) : (a < b ? a : b); };
  v = op(v, dpp_u<0xb1>(v));
  v = op(v, dpp_u<0x4e>(v));
  v = op(v, dpp_u<0x141>(v));
  v = op(v, dpp_u<0x140>(v));
  if (L >= 32) {
    const auto q = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = op(q[0], q[1]);
  }
  if (L == 64) {
    const auto h = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    v = op(h[0], h[1]);
  }
  return v;
}
template <bool HALF, bool MAX>
__device__ __forceinline__ uint32_t group_uext(uint32_t v) {
  return group_uext_l<HALF ? 32 : 64, MAX>(v);
}

// Logits of token t for one lane: expert e = h + L j (j < KPL) with L lanes
// per token, h = lane % L: L = 64 or 32 with four logits per lane (E <= 256
// and E <= 128), L = 16 with eight (E <= 128).  Issued early so the
// planner's set-up hides their latency.
template <int L>
constexpr int kKeysPerLane = L == 16 ? 8 : 4;
template <int L>
__device__ __forceinline__ void load_token_logits_l(const float *__restrict__ logits, int t, bool live,
                                                    int E, float (&raw)[kKeysPerLane<L>]) {
  const int h = threadIdx.x & (L - 1);
#pragma unroll
  for (int j = 0; j < kKeysPerLane<L>; ++j) {
    const int e = h + L * j;
    raw[j] = live && e < E ? logits[(size_t)t * E + e] : -INFINITY;
  }
}
template <bool HALF>
__device__ __forceinline__ void load_token_logits(const float *__restrict__ logits, int t, bool live,
                                                  int E, float (&raw)[4]) {
  load_token_logits_l<HALF ? 32 : 64>(logits, t, live, E, raw);
}

// The lanes of one token route it from its logits (raw, as loaded above).
// Selection is by logit (softmax is monotone): K rounds of a group max over
// each lane's best remaining key, then a group min over the experts holding
// that key (equal logits go to the lower expert), whose lane drops it.  Keys
// are offset by one so a dropped or absent expert (0) ranks below a NaN
// logit (1).  Lane k keeps the key and expert of slot k and the
// probabilities are formed once, after the loop.  NaN logits rank below
// every number and set the logit flag.  Results go to global memory and,
// when `lds_ids` is given, to LDS for the planner (global memory only when
// `ids_out` is non-null).  A group with live ==
// false computes on nothing and stores nothing.
template <int L, int NT>
__device__ void route_tokens(const float (&raw)[NT][kKeysPerLane<L>], const int (&t)[NT], const bool (&live)[NT], int E,
                             int K, int renormalize, int32_t *__restrict__ ids_out,
                             float *__restrict__ w_out, uint32_t &flags, int *lds_ids, float *lds_w) {
  // NT tokens per lane group, their dependency chains interleaved step by
  // step (every loop below runs over the tokens innermost), so a group
  // routing two tokens takes about the latency of one.
  constexpr int KPL = kKeysPerLane<L>;
  const int h = threadIdx.x & (L - 1);
  uint32_t key[NT][KPL];
  bool bad = false;
#pragma unroll
  for (int n = 0; n < NT; ++n)
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
      const bool ok = live[n] && h + L * j < E;
      bad |= ok && !isfinite(raw[n][j]);
      key[n][j] = ok ? float_key(raw[n][j]) + 1u : 0u;
    }
  if (__any(bad)) flags |= 4u;
  auto top4 = [&](int n) {  // the lane's best remaining key (pairwise tree)
    uint32_t v[KPL];
#pragma unroll
    for (int j = 0; j < KPL; ++j) v[j] = key[n][j];
#pragma unroll
    for (int w = KPL / 2; w > 0; w /= 2)
#pragma unroll
      for (int j = 0; j < w; ++j) v[j] = v[j] > v[j + w] ? v[j] : v[j + w];
    return v[0];
  };
  float m[NT], z[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) m[n] = key_float(group_uext_l<L, true>(top4(n)) - 1u);
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    z[n] = 0.f;
#pragma unroll
    for (int j = 0; j < KPL; ++j)
      if (live[n] && h + L * j < E) z[n] += expf(raw[n][j] - m[n]);
  }
#pragma unroll
  for (int n = 0; n < NT; ++n) z[n] = group_fsum_l<L>(z[n]);

  uint32_t my_key[NT];
  int my_id[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    my_key[n] = 1;
    my_id[n] = kMaxExperts;
  }
  for (int k = 0; k < K; ++k) {
    uint32_t M[NT], c[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) M[n] = group_uext_l<L, true>(top4(n));
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      c[n] = kMaxExperts;
#pragma unroll
      for (int j = KPL - 1; j >= 0; --j)
        if (M[n] != 0 && key[n][j] == M[n]) c[n] = h + L * j;
    }
    int idx[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) idx[n] = (int)group_uext_l<L, false>(c[n]);
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      if (idx[n] < kMaxExperts && (idx[n] & (L - 1)) == h) {
#pragma unroll
        for (int j = 0; j < KPL; ++j)
          if (idx[n] / L == j) key[n][j] = 0;
      }
      if (h == k) {
        my_key[n] = M[n];
        my_id[n] = idx[n];
      }
    }
  }
  float p[NT], psum[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) p[n] = h < K ? expf(key_float(my_key[n] - 1u) - m[n]) / z[n] : 0.f;
#pragma unroll
  for (int n = 0; n < NT; ++n) psum[n] = group_fsum_l<L>(p[n]);
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    if (live[n] && h < K) {
      const int q = t[n] * K + h;
      const float w = renormalize ? p[n] / psum[n] : p[n];
      if (ids_out) {
        ids_out[q] = my_id[n];
        w_out[q] = w;
      }
      if (lds_ids) {
        lds_ids[q] = my_id[n];
        lds_w[q] = w;
      }
    }
  }
}

template <bool HALF>
__device__ __forceinline__ void route_token(const float (&raw)[4], int t, bool live, int E, int K,
                                            int renormalize, int32_t *__restrict__ ids_out,
                                            float *__restrict__ w_out, uint32_t &flags, int *lds_ids,
                                            float *lds_w) {
  const float (&r1)[1][4] = *reinterpret_cast<const float(*)[1][4]>(&raw);
  const int t1[1] = {t};
  const bool l1[1] = {live};
  route_tokens<HALF ? 32 : 64, 1>(r1, t1, l1, E, K, renormalize, ids_out, w_out, flags, lds_ids, lds_w);
}


// ---- planning from routes held in LDS, for R <= 1024 routes ----------------
//
// The planner of moe_route.hip restated for one 1024-thread workgroup that
// has just routed every token into LDS (one route per thread): status bits,
// per-expert counts, canonical ranks rank[q] = #{q' < q : id[q'] == id[q]}
// (wave-ballot match over the ID bits, then a prefix over the waves),
// exclusive scans, the grouped-row -> token table and the task list, all in
// LDS; with `write_global` the global plan arrays too (the same values the
// planner kernel writes).
constexpr int kSmallPlanRoutes = 1024;
constexpr int kSmallPlanWaves = 16;

struct SmallPlanLds {
  const int *ids;    // [R] expert of route q
  const float *w;    // [R] routing weight of route q
  int *wcnt;         // [NT / 64][E] zeroed before the call; per-wave counts -> prefixes
  int *cnt, *off;    // [E]
  int *toff;         // [E + 1]
  int4 *tasks;       // task list
  int *row_token;    // [R + 64] token of grouped row p (0 past the last row)
  int *ntasks;       // [1]
  uint32_t *flags;   // [1] zeroed before the call; OR of the status bits
};
struct SmallPlanOut {
  int32_t *counts, *offsets, *ranks, *map, *row_route, *row_token;
  int4 *tasks;
  int32_t *num_tasks;
  uint32_t *status;
};

// Workgroup barrier ordering LDS only.  __syncthreads() is also a release
// fence for global memory, which waits for every load the workgroup has in
// flight -- the streaming gate/up requests its first weights before planning.
__device__ __forceinline__ void lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Bits of an expert id below E (E <= 256).
__device__ __forceinline__ int id_bits(int E) { return E <= 1 ? 1 : 32 - __builtin_clz((unsigned)(E - 1)); }

// Called by all NT threads of the workgroup (R <= NT routes, one per thread;
// NT / 64 per-wave count rows in wcnt) after the routes are visible in LDS.
template <int NT = kSmallPlanRoutes>
__device__ inline void plan_small(const SmallPlanLds &s, const SmallPlanOut &go, bool write_global,
                                  int R, int E, int K, int tb, uint32_t flags) {
  const SmallPlanOut *g = write_global ? &go : nullptr;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & (kWave - 1);
  const int q = tid;
  const bool valid = q < R;
  const int idv = valid ? s.ids[q] : -1;
  const float wv = valid ? s.w[q] : 0.f;
  const bool ok = valid && idv >= 0 && idv < E;
  if (valid && !ok) flags |= 1u;
  if (valid && !isfinite(wv)) flags |= 2u;
  const int id = ok ? idv : 0;
  uint64_t match = __ballot(ok);
  const int nbits = id_bits(E);
#pragma unroll
  for (int bit = 0; bit < 8; ++bit) {
    if (bit >= nbits) break;  // every id is below 2^nbits
    const bool set = (id >> bit) & 1;
    const uint64_t b = __ballot(ok && set);
    match &= set ? b : ~b;
  }
  const int lrank = __popcll(match & lanemask_lt());
  if (ok && lrank == 0) s.wcnt[wave * E + id] = __popcll(match);
  lds_sync();
  if (wave == 0) {
    // Per expert (four per lane): counts of the waves holding routes ->
    // exclusive prefixes in place, then exclusive scans of the counts and
    // task counts over the experts.
    const int nw = (R + kWave - 1) / kWave;
    int c[4], nt[4], csum = 0, tsum = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane * 4 + j;
      int run = 0;
      if (e < E) {
        for (int w = 0; w < nw; ++w) {
          const int t = s.wcnt[w * E + e];
          s.wcnt[w * E + e] = run;
          run += t;
        }
        s.cnt[e] = run;
      }
      c[j] = run;
      nt[j] = (c[j] + tb - 1) / tb;
      csum += c[j];
      tsum += nt[j];
    }
    int crun = wave_incl_scan(csum) - csum, trun = wave_incl_scan(tsum) - tsum;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane * 4 + j;
      if (e < E) {
        s.off[e] = crun;
        s.toff[e] = trun;
        if (g) {
          g->counts[e] = c[j];
          g->offsets[e] = crun;
        }
      }
      crun += c[j];
      trun += nt[j];
    }
    if (lane == kWave - 1) {
      s.toff[E] = trun;
      *s.ntasks = trun;
    }
  }
  lds_sync();
  const int valid_rows = s.off[E - 1] + s.cnt[E - 1];
  if (ok) {
    const int rank = s.wcnt[wave * E + id] + lrank;
    const int p = s.off[id] + rank;
    s.row_token[p] = q / K;
    if (g) {
      g->ranks[q] = rank;
      g->map[q] = p;
      g->row_route[p] = q;
      g->row_token[p] = q / K;
    }
  } else if (valid && g) {
    g->ranks[q] = -1;
    g->map[q] = -1;
  }
  for (int p = valid_rows + tid; p < R + 64; p += NT) {
    s.row_token[p] = 0;
    if (g && p < R) {
      g->row_route[p] = -1;
      g->row_token[p] = 0;
    }
  }
  for (int e = tid; e < E; e += NT) {
    const int c = s.cnt[e];
    int t0 = s.toff[e];
    for (int r0 = 0; r0 < c; r0 += tb, ++t0) {
      const int4 t = make_int4(e, s.off[e] + r0, min(tb, c - r0), 0);
      s.tasks[t0] = t;
      if (g) g->tasks[t0] = t;
    }
  }
  if (flags) atomicOr(s.flags, flags);
  lds_sync();
  if (g && tid == 0) {
    *g->num_tasks = s.toff[E];
    // Write-through: a later workgroup of the same launch may OR a bit into
    // this word from another XCD (the work-accounting check of the GEMMs).
    __hip_atomic_store(g->status, *s.flags, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace route_dev
}  // namespace moe
