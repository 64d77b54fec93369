// Weight-streaming grouped GEMMs of the MoE forward on gfx950 (CDNA4).
//
// gate/up + SwiGLU (reference: _dynamic_grouped_gate_up_swiglu,
// moe_fused.py:18-73; cuda_gate_up_bf16, cuda_gate_up.cu:53-131; W4:
// cuda_gate_up_w4_sync, cuda_w4_gate_up.cu:46-100) and the down projection
// (_dynamic_grouped, moe.py:69-95) for the regime of every BASELINE
// configuration: few grouped rows per expert, so the expert weights are the
// only large operand and the kernel is bound by HBM bandwidth.
//
// Work unit = (task, column block): a task is an expert and up to 16*MT of
// its grouped rows; a column block is 16 intermediate columns (gate/up
// kernel: 16 gate rows + 16 up rows of weights) or 32 hidden columns (down).
//
//  * Split-K across the 8 waves of a workgroup: wave w owns k-steps
//    [w*SPW, (w+1)*SPW).  It loads its K-slice of the unit's token rows (MFMA
//    B operand) straight from global memory into registers -- x rows are
//    gathered through the route list, no permuted copy of x exists -- and
//    streams the weights (MFMA A operand, one 128-bit load per lane per
//    16x16x32 MFMA) from HBM.  The eight partial tiles are summed through LDS
//    in fixed wave order (deterministic) and the epilogue applies the
//    reference's rounding stages.
//  * Persistent workgroups, one per CU slot, each take a block of
//    consecutive units (balanced to one unit): the token rows are loaded once
//    per task, and the next units' weights are in flight while the current
//    unit multiplies.  The loop body is straight-line: k-slices are
//    compile-time, invalid rows load a clamped address, and all unit
//    metadata comes through scalar loads, so the only vector-memory wait
//    before the MFMAs is for the current unit's weights.
//  * W4G128: the 16-byte load of a lane holds 32 int4 of one row (a whole
//    128-K group, 4 MFMA k-steps) and is decoded in registers by
//    w4_decode8, bit-exact with the reference dequantisation.
#include <type_traits>

#include "common.h"
#include "moe_internal.h"
#include "moe_route_dev.h"

#define MOE_CONST __attribute__((address_space(4)))

namespace moe {

namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
constexpr int kWaitVmcntZero = (7 << 4) | (15 << 8);  // s_waitcnt vmcnt(0) only (gfx9 encoding)


template <typename T>
__device__ __forceinline__ const MOE_CONST T *as_const(const T *p) {
  return (const MOE_CONST T *)p;
}

// Workgroup barrier ordering LDS only.  __syncthreads() also orders global
// memory, which makes every wave wait for its in-flight weight prefetch.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// KIND 0: gate/up + SwiGLU.  A = gate rows cb*16.. and up rows I+cb*16..,
//         K = H, B = x rows of the task's tokens.
// KIND 1: down.  A = rows cb*32 + 16*rb (rb < 2), K = I, B = act rows.
// FOLD (W4 only): the folded decode (w4_fold8): token fragments as the MFMA
// A operand in the folded K order, weights (136 + q) as B, and each group's
// fp32 sum scaled by the lane's own weight-row scale after subtracting 136 x
// the group's token sums; effective weights q * scale exactly.
// PLAN (W4 gate/up, 16-row tasks, router-fused shapes with R <= 512): every
// workgroup first routes all tokens and plans in LDS (route_dev::route_token
// and plan_small), workgroup 0 also writes the routing results, the global
// plan arrays for the down and combine launches and zeroes the work counters
// (as the planner launch would), and the units' tasks and token rows come
// from LDS; the separate planner launch is then not needed.
constexpr int kPlanTasks = route_dev::kMaxExperts + kThreads / 16;  // E + R / 16 bound
constexpr int kPlanLds = kPlanTasks * 16 + (kThreads + 64) * 4 + 16;

template <int KIND, int MT, int SPW, bool W4, bool FOLD>
constexpr size_t stream_lds(bool plan) {
  return (size_t)2 * kWaves * 2 * MT * kWave * sizeof(f32x4) +
         (FOLD ? (size_t)kWaves * (SPW / 4) * MT * 16 * sizeof(float) : 0) + (plan ? kPlanLds : 0);
}

template <int KIND, int MT, int SPW, bool W4, bool FOLD, bool PLAN = false>
__global__ __launch_bounds__(kThreads, FOLD ? 4 : 1) void stream_kernel(ExpertArgs a, RouteArgs ra) {
  constexpr int NRB = 2;
  extern __shared__ f32x4 s_red[];  // [2][kWaves][NRB][MT][64]
  static_assert(!PLAN || (KIND == 0 && MT == 1 && W4), "planning prologue: 16-row W4 gate/up");

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar address math
  const int lane = tid & (kWave - 1);
  const int r = lane & 15, g = lane >> 4;
  const int H = a.H, I = a.I;
  const int s0 = wave * SPW;
  const int ncb = KIND == 0 ? I / 16 : H / 32;
  const int4 *l_tasks = nullptr;
  const int *l_row = nullptr;
  int ntasks = 0;
  if constexpr (PLAN) {
    using namespace route_dev;
    uint8_t *pl = (uint8_t *)s_red + stream_lds<KIND, MT, SPW, W4, FOLD>(false);
    int4 *p_tasks = (int4 *)pl;
    int *p_row = (int *)(pl + kPlanTasks * 16);
    int *p_nt = p_row + kThreads + 64;
    // Scratch in the partial-sum buffers (idle until the first unit's sums).
    int *x_ids = (int *)s_red;
    float *x_w = (float *)((uint8_t *)s_red + 4 * kThreads);
    int *x_wcnt = (int *)((uint8_t *)s_red + 8 * kThreads);
    int *x_cnt = x_wcnt + kWaves * kMaxExperts;
    int *x_off = x_cnt + kMaxExperts;
    int *x_toff = x_off + kMaxExperts;
    uint32_t *x_flags = (uint32_t *)(x_toff + kMaxExperts + 1);
    // Routing: with E <= 128 and K <= 16, 16 lanes per token (eight logits
    // per lane), so the eight waves route up to 32 tokens in one pass; the
    // prologue's routing is bound by instruction issue (every workgroup routes
    // every token), and 16-lane groups need about 2.4x fewer wave
    // instructions than half-waves over two rounds.  Otherwise one token per
    // wave (T <= 16), two per wave interleaved.  All logits are requested
    // before the LDS set-up.
    const bool quarter = ra.E <= 128 && ra.K <= 16;
    const bool half = !quarter && ra.fuse_router == 2;  // K > 16, T <= 32: 32 lanes per token
    const int per_pass = half ? 2 * kWaves : kWaves;
    float rq[1][8];
    float raw[2][4];
    int ft[2];
    if (quarter) {
      ft[0] = 4 * wave + (lane >> 4);
      load_token_logits_l<16>(ra.logits, ft[0], ft[0] < ra.T, ra.E, rq[0]);
    } else {
#pragma unroll
      for (int rd = 0; rd < 2; ++rd) {
        ft[rd] = rd * per_pass + (half ? 2 * wave + (lane >> 5) : wave);
        if (half) load_token_logits<true>(ra.logits, ft[rd], ft[rd] < ra.T, ra.E, raw[rd]);
        else load_token_logits<false>(ra.logits, ft[rd], ft[rd] < ra.T, ra.E, raw[rd]);
      }
    }
    for (int i = tid; i < kWaves * ra.E; i += kThreads) x_wcnt[i] = 0;
    if (tid == 0) *x_flags = 0;
    const bool g0 = blockIdx.x == 0;
    if (g0 && tid < 4) ra.counters[tid] = 0;
    uint32_t flags = 0;
    int32_t *ids_g = g0 ? (int32_t *)ra.ids : nullptr;
    float *w_g = g0 ? ra.weights : nullptr;
    if (quarter) {
      if (4 * wave < ra.T) {  // wave-uniform: the wave's first token exists
        const int t1[1] = {ft[0]};
        const bool l1[1] = {ft[0] < ra.T};
        route_tokens<16, 1>(rq, t1, l1, ra.E, ra.K, ra.renormalize, ids_g, w_g, flags, x_ids, x_w);
      }
    } else {
      // Up to two tokens per wave (or half-wave), routed in one interleaved pass.
      const int first = half ? 2 * wave : wave;  // wave-uniform
      const bool live2[2] = {ft[0] < ra.T, ft[1] < ra.T};
      if (first + per_pass < ra.T) {
        if (half) route_tokens<32, 2>(raw, ft, live2, ra.E, ra.K, ra.renormalize, ids_g, w_g, flags, x_ids, x_w);
        else route_tokens<64, 2>(raw, ft, live2, ra.E, ra.K, ra.renormalize, ids_g, w_g, flags, x_ids, x_w);
      } else if (first < ra.T) {
        if (half) route_token<true>(raw[0], ft[0], live2[0], ra.E, ra.K, ra.renormalize, ids_g, w_g, flags, x_ids, x_w);
        else route_token<false>(raw[0], ft[0], true, ra.E, ra.K, ra.renormalize, ids_g, w_g, flags, x_ids, x_w);
      }
    }
    __syncthreads();
    const SmallPlanLds L{x_ids, x_w, x_wcnt, x_cnt, x_off, x_toff, p_tasks, p_row, p_nt, x_flags};
    const SmallPlanOut O{ra.counts, ra.offsets, ra.ranks, ra.map, ra.row_route, ra.row_token,
                         ra.tasks, ra.num_tasks, ra.status};
    plan_small<kThreads>(L, O, g0, ra.R, ra.E, ra.K, 16, flags);
    ntasks = *p_nt;
    l_tasks = p_tasks;
    l_row = p_row;
  }
  const int total = (PLAN ? ntasks : *as_const(a.num_tasks)) * ncb;
  // Each workgroup takes a block of consecutive units, i.e. mostly one
  // task, so the token rows (B) stay in registers from unit to unit and are
  // reloaded only when the task changes (round-robin units, B reloaded per
  // unit behind the weight loads of later units, measured 5-18 us slower).
  const int G = gridDim.x;
  const int c = (total + G - 1) / G;
  const int b0 = (int)blockIdx.x * c;
  const int count = b0 < total ? min(c, total - b0) : 0;
  if (count <= 0) return;
  auto unit_at = [&](int i) { return b0 + i; };

  const MOE_CONST int32_t *tasks = as_const((const int32_t *)a.tasks);

  // Unit metadata: scalars, plus one VGPR whose lane k < ROWS holds the
  // token (gate/up) or route (down) of the task's row k (one vector load; the
  // index arrays carry 64 ints of slack past the last row).
  const int32_t *row_vec = KIND == 0 ? a.row_token : a.row_route;
  struct Meta {
    int unit, task, cb, expert, row0, rows;
    int idxv;
  };
  auto meta_of = [&](int u) {
    Meta m;
    m.unit = u;
    const int t = u / ncb;
    m.task = t;
    m.cb = u - t * ncb;
    if constexpr (PLAN) {
      const int4 tk = l_tasks[t];
      m.expert = __builtin_amdgcn_readfirstlane(tk.x);
      m.row0 = __builtin_amdgcn_readfirstlane(tk.y);
      m.rows = __builtin_amdgcn_readfirstlane(tk.z);
      m.idxv = l_row[m.row0 + (lane & 31)];
    } else {
      m.expert = tasks[4 * t];
      m.row0 = tasks[4 * t + 1];
      m.rows = tasks[4 * t + 2];
      m.idxv = row_vec[m.row0 + (lane & 31)];
    }
    return m;
  };

  // B operand: [MT][SPW] fragments of this wave's K-slice.  Rows past the
  // task's end load row 0 of x (gate/up) or of act (down) instead, finite
  // data that is never zeroed: an MFMA output column depends only on its own
  // B column and the epilogue never stores those columns.
  u32x4 bfr[MT][SPW];
  // FOLD: the MFMA operands are swapped (token fragments A, weights B), so
  // the output lane holds its own weight row (one scale per lane) and tokens
  // 4g .. 4g + 3; xs holds -136 x (each group's sum of the 128 x values of
  // those tokens), computed once per task.
  static_assert(W4 || !FOLD, "the folded decode is a W4 mode");
  constexpr int AWX = W4 ? SPW / 4 : 1;
  // -136 x group sums per wave, [group][token], read back as f32x4 per group
  // (in LDS rather than registers: the kernel is at its 128-VGPR budget).
  float *s_xs = (float *)(s_red + 2 * kWaves * 2 * MT * kWave);  // after the partials
  auto prep_b = [&]() {
    if constexpr (FOLD) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int q = 0; q < AWX; ++q) {
          float t = 0.f;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            t += bf16x8_sum(bfr[mt][4 * q + j]);
            bfr[mt][4 * q + j] = w4_fold_b(bfr[mt][4 * q + j]);
          }
          t += __shfl_xor(t, 16, kWave);
          t += __shfl_xor(t, 32, kWave);  // token r's group sum, in every lane of column r
          if (g == 0) s_xs[(wave * AWX + q) * MT * 16 + mt * 16 + r] = -136.0f * t;
        }
    }
  };
  auto load_b = [&](const Meta &m) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int j = mt * 16 + r;
      const bool ok = j < m.rows;
      size_t row;
      if (KIND == 0)
        row = (size_t)(ok ? __shfl(m.idxv, j, kWave) : 0) * H;
      else
        row = (size_t)(ok ? m.row0 + j : 0) * I;
      const uint16_t *src = (KIND == 0 ? a.x : a.act) + row + s0 * 32 + g * 8;
#pragma unroll
      for (int i = 0; i < SPW; ++i) bfr[mt][i] = *(const u32x4 *)(src + i * 32);
    }
  };

  // A operand: bf16 -> [NRB][SPW] fragments; W4 -> [NRB][SPW/4] words + scales.
  // A ring of S unit slots keeps S-1 units of weights in flight (W4 units are
  // 4x smaller, so they need a deeper ring; three slots keep the kernel within
  // 128 VGPRs, i.e. two workgroups per CU).  Slots are compile-time indices
  // of an unrolled loop: copying a register whose load is still in flight
  // would make the wave wait for it.
  constexpr int AW = W4 ? SPW / 4 : SPW;
  constexpr int S = W4 && !FOLD ? 3 : 2;
  u32x4 aq[S][NRB][AW];
  using ScaleT = uint32_t;  // the scale of the lane's own weight row
  ScaleT sq[S][NRB][AW];
  Meta mq[S];
  // m.unit < 0 marks a ring slot past the end: it reads the first unit of the
  // weights (expert 0, column block 0), which every such slot shares through
  // the cache, with the normal lane offsets -- so every address is a scalar
  // base plus a fixed per-lane offset and the loads need no vector math.
  const uint32_t lane_a = KIND == 0 ? (uint32_t)(r * H + g * 8) * 2u : (uint32_t)(r * I + g * 8) * 2u;
  auto load_a = [&](const Meta &m, u32x4 (&buf)[NRB][AW], ScaleT (&sc)[NRB][AW]) {
    const bool live = m.unit >= 0;
    const int ex = live ? m.expert : 0, cb = live ? m.cb : 0;
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
      if constexpr (W4) {
        const int G4 = H >> 7;
        const size_t rbi = (size_t)ex * (2 * I / 16) + cb + (rb ? I / 16 : 0);
#pragma unroll
        for (int i = 0; i < AW; ++i) {
          const size_t unit = rbi * G4 + (s0 >> 2) + i;
          buf[rb][i] = ((const u32x4 *)a.w4_words)[unit * kWave + lane];
          sc[rb][i] = a.w4_scales[unit * 16 + r];
        }
      } else {
        const uint16_t *base;
        if (KIND == 0)
          base = a.gate_up + ((size_t)ex * 2 * I + (rb ? I : 0) + cb * 16) * H + s0 * 32;
        else
          base = a.down + ((size_t)ex * H + cb * 32 + rb * 16) * I + s0 * 32;
        const uint8_t *lb = (const uint8_t *)base + lane_a;
#pragma unroll
        for (int i = 0; i < AW; ++i) buf[rb][i] = *(const u32x4 *)(lb + i * 64);
      }
    }
  };

  // Prologue: positions p < S (clamped to a valid unit) into slots p.
#pragma unroll
  for (int p = 0; p < S; ++p) {
    mq[p] = meta_of(unit_at(p < count ? p : 0));
    if (p >= count) mq[p].unit = -1;
    load_a(mq[p], aq[p], sq[p]);
    if (p == 0) {
      load_b(mq[0]);
      // B is never in flight at a step boundary (see the task switch below).
      __builtin_amdgcn_s_waitcnt(kWaitVmcntZero);
      prep_b();
    }
  }
  int btask = mq[0].task;

  int i = 0;
  int parity = 0;
  // One unit in ring slot SL; returns whether another unit follows.
  auto step = [&](auto slot_tag) -> bool {
    constexpr int SL = decltype(slot_tag)::value;
    const Meta &cur = mq[SL];
    // New task: its token rows, waited for here, so no step boundary has a
    // B load in flight (a B load outstanding across the loop would make
    // every step wait for the weight loads issued after it).
    if (cur.task != btask) {
      load_b(cur);
      __builtin_amdgcn_s_waitcnt(kWaitVmcntZero);
      prep_b();
      btask = cur.task;
    }
    f32x4 acc[NRB][MT];
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[rb][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
      if constexpr (FOLD) {
#pragma unroll
        for (int i = 0; i < AW; ++i) {
          f32x4 tg[MT];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const u32x4 af = w4_fold8(aq[SL][rb][i][j]);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
              tg[mt] = j == 0 ? mfma16(bfr[mt][i * 4 + j], af, f32x4{0.f, 0.f, 0.f, 0.f})
                              : mfma16(bfr[mt][i * 4 + j], af, tg[mt]);
          }
          const float sc = bf16_bits_to_f32(sq[SL][rb][i]);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const f32x4 xo = *(const f32x4 *)(s_xs + (wave * AWX + i) * MT * 16 + mt * 16 + 4 * g);
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[rb][mt][c] = __builtin_fmaf(sc, tg[mt][c] + xo[c], acc[rb][mt][c]);
          }
        }
      } else if constexpr (W4) {
#pragma unroll
        for (int i = 0; i < AW; ++i) {
          const W4Scale ks = w4_scale(bf16_bits_to_f32(sq[SL][rb][i]));
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const u32x4 af = w4_decode8(aq[SL][rb][i][j], ks);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[rb][mt] = mfma16(af, bfr[mt][i * 4 + j], acc[rb][mt]);
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < SPW; ++i)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) acc[rb][mt] = mfma16(aq[SL][rb][i], bfr[mt][i], acc[rb][mt]);
      }
    }

    // Partial sums alternate between two LDS buffers from step to step (the
    // epilogue of one unit may still read its buffer while fast waves write
    // the next unit's partials).
    f32x4 *red = s_red + (size_t)(parity & 1) * kWaves * NRB * MT * kWave;
    ++parity;
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

    lds_barrier();

    // Epilogue of cur: fixed-order sum of the eight K-slices.
    if (KIND == 0) {
      // One output per thread (4 waves per token block), so no single wave
      // carries the epilogue's latency into the next unit's barrier.
      // The threads of the epilogue rotate over the waves from unit to unit.
      constexpr int EN = MT * 4 * kWave;
      const int et = tid - ((i & 1) % (kThreads / EN)) * EN;
      if (et >= 0 && et < EN) {
        const int l = et & 63, ii = (et >> 6) & 3, mt = et >> 8;
        // FOLD: partial tiles are [token][weight row] (token 4(l/16) + ii,
        // feature l%16); otherwise [weight row][token].
        const int j = FOLD ? mt * 16 + 4 * (l >> 4) + ii : mt * 16 + (l & 15);
        const int feat = FOLD ? (l & 15) : 4 * (l >> 4) + ii;
        const float *redf = (const float *)red;
        auto part = [&](int w, int rb) { return redf[((((w * NRB + rb) * MT + mt) * 4 + ii) * kWave + l)]; };
        float sg = part(0, 0), su = part(0, 1);
#pragma unroll
        for (int w = 1; w < kWaves; ++w) {
          sg += part(w, 0);
          su += part(w, 1);
        }
        const float gt = bf16_round(sg);
        const float up = bf16_round(su);
        const float v = gt / (1.0f + expf(-gt)) * up;
        if (j < cur.rows)
          a.act[(size_t)(cur.row0 + j) * I + cur.cb * 16 + feat] =
              (uint16_t)(pack_bf16x2(v, 0.f) & 0xffffu);
      }
    } else {
      constexpr int EN = NRB * MT * kWave;
      const int et = tid - ((i & 1) % (kThreads / EN)) * EN;
      if (et >= 0 && et < EN) {
        const int rb = et / (MT * kWave);
        const int mt = (et >> 6) % MT, l = et & 63;
        const int j = mt * 16 + (l & 15);
        f32x4 sm = red[(rb * MT + mt) * kWave + l];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) sm += red[((w * NRB + rb) * MT + mt) * kWave + l];
        const int q = __shfl(cur.idxv, j, kWave);
        u32x2 packed;
        packed[0] = pack_bf16x2(sm[0], sm[1]);
        packed[1] = pack_bf16x2(sm[2], sm[3]);
        if (j < cur.rows)
          *(u32x2 *)(a.routed + (size_t)q * H + cur.cb * 32 + rb * 16 + 4 * (l >> 4)) = packed;
      }
    }

    // Refill this slot with the unit S positions ahead.
    const int ip = i + S;
    mq[SL] = meta_of(unit_at(ip < count ? ip : i));
    if (ip >= count) mq[SL].unit = -1;
    load_a(mq[SL], aq[SL], sq[SL]);
    ++i;
    return i < count;
  };

  using std::integral_constant;
  while (true) {
    if (!step(integral_constant<int, 0>{})) break;
    if (!step(integral_constant<int, 1>{})) break;
    if constexpr (S >= 3) {
      if (!step(integral_constant<int, 2>{})) break;
    }
    if constexpr (S >= 4) {
      if (!step(integral_constant<int, 3>{})) break;
    }
  }
}

template <int KIND, int MT, int SPW, bool W4, bool FOLD = false, bool PLAN = false>
hipError_t launch_one(const ExpertArgs &a, int units_bound, int num_cus, hipStream_t s,
                      const RouteArgs *ra = nullptr) {
  auto k = stream_kernel<KIND, MT, SPW, W4, FOLD, PLAN>;
  const size_t lds = stream_lds<KIND, MT, SPW, W4, FOLD>(PLAN);
  static int per_cu = [&] {
    int n = 1;
    (void)hipFuncSetAttribute((const void *)k, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)kMaxLds);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, (const void *)k, kThreads, lds) !=
            hipSuccess || n < 1)
      n = 1;
    // Two resident workgroups per CU overlap one's barrier and epilogue with
    // the other's MFMA phase; a third only adds HBM contention (the bf16
    // kernels already stream at the practical HBM rate with two).
    return n < 2 ? n : 2;
  }();
  int grid = num_cus * per_cu;
  if (grid > units_bound) grid = units_bound;
  if (grid < 1) grid = 1;
  RouteArgs none{};
  hipLaunchKernelGGL(k, dim3(grid), dim3(kThreads), lds, s, a, ra ? *ra : none);
  return hipGetLastError();
}

template <int KIND, int MT, bool W4>
hipError_t launch_spw(const ExpertArgs &a, int spw, int units, int num_cus, hipStream_t s) {
  if constexpr (W4) {
    if (a.w4_fold) {
      switch (spw) {
        case 4: return launch_one<KIND, MT, 4, true, true>(a, units, num_cus, s);
        case 8: return launch_one<KIND, MT, 8, true, true>(a, units, num_cus, s);
        default: return hipErrorInvalidValue;
      }
    }
    switch (spw) {
      case 4: return launch_one<KIND, MT, 4, true>(a, units, num_cus, s);
      case 8: return launch_one<KIND, MT, 8, true>(a, units, num_cus, s);
      default: return hipErrorInvalidValue;
    }
  } else {
    switch (spw) {
      case 1: return launch_one<KIND, MT, 1, false>(a, units, num_cus, s);
      case 2: return launch_one<KIND, MT, 2, false>(a, units, num_cus, s);
      case 3: return launch_one<KIND, MT, 3, false>(a, units, num_cus, s);
      case 4: return launch_one<KIND, MT, 4, false>(a, units, num_cus, s);
      case 6: return launch_one<KIND, MT, 6, false>(a, units, num_cus, s);
      case 8: return launch_one<KIND, MT, 8, false>(a, units, num_cus, s);
      default: return hipErrorInvalidValue;
    }
  }
}

bool spw_ok(int dim, bool w4) {
  if (dim % 256) return false;
  const int spw = dim / 256;
  if (w4) return spw == 4 || spw == 8;
  return spw == 1 || spw == 2 || spw == 3 || spw == 4 || spw == 6 || spw == 8;
}

}  // namespace

bool stream_shape_ok(int H, int I, bool w4) { return spw_ok(H, w4) && spw_ok(I, false); }

hipError_t launch_stream_gate_up(const ExpertArgs &a, int task_capacity, int token_block, bool w4,
                                 int num_cus, hipStream_t s) {
  const int units = task_capacity * (a.I / 16);
  const int spw = a.H / 256;
  if (token_block == 16)
    return w4 ? launch_spw<0, 1, true>(a, spw, units, num_cus, s)
              : launch_spw<0, 1, false>(a, spw, units, num_cus, s);
  return w4 ? launch_spw<0, 2, true>(a, spw, units, num_cus, s)
            : launch_spw<0, 2, false>(a, spw, units, num_cus, s);
}

bool stream_plan_ok(int H, int I, int T, int K, int E, int fuse_router) {
  return stream_shape_ok(H, I, true) && H / 256 == 8 && fuse_router != 0 && T * K <= kThreads &&
         E <= route_dev::kMaxExperts && T <= 32;
}

hipError_t launch_stream_gate_up_planned(const ExpertArgs &a, const RouteArgs &ra, int task_capacity,
                                         int num_cus, hipStream_t s) {
  const int units = task_capacity * (a.I / 16);
  if (a.H != 2048) return hipErrorInvalidValue;
  if (a.w4_fold) return launch_one<0, 1, 8, true, true, true>(a, units, num_cus, s, &ra);
  return launch_one<0, 1, 8, true, false, true>(a, units, num_cus, s, &ra);
}

hipError_t launch_stream_down(const ExpertArgs &a, int task_capacity, int token_block,
                              int num_cus, hipStream_t s) {
  const int units = task_capacity * (a.H / 32);
  const int spw = a.I / 256;
  if (token_block == 16) return launch_spw<1, 1, false>(a, spw, units, num_cus, s);
  return launch_spw<1, 2, false>(a, spw, units, num_cus, s);
}

}  // namespace moe
