// MFMA grouped GEMMs of the MoE forward for shapes outside the tuned kernels
// (reference semantics as in moe_stream.hip: _dynamic_grouped_gate_up_swiglu,
// moe_fused.py:18-73, W4 cuda_w4_gate_up.cu:46-100; down _dynamic_grouped,
// moe.py:69-95).
//
// The streaming, LDS-streaming and tiled kernels fix K per stage at compile
// time (H, I in {512 .. 4096} at fixed steps).  Here K is a run-time multiple
// of 32 (bf16) or of 128 (W4G128, the format's group), so any such shape --
// H = 2880 or 7168, I = 1536 -- runs on the matrix cores:
//
//  * one workgroup of 8 waves per unit (task, column block): 16 act columns
//    (gate rows cb*16.. and up rows I + cb*16..) for gate/up, 32 hidden
//    columns (two 16-row blocks) for down;
//  * wave w takes the K-steps w, w + 8, ... (32 wide; W4: one 128-wide group
//    per step, one 16-byte load per lane of the tiled layout) and loads the
//    weight fragments (MFMA A operand) and token-row fragments (B operand)
//    straight from global memory into a register ring kFlexRing steps ahead;
//  * the eight partial tiles are summed through LDS in fixed wave order and
//    the epilogue applies the reference's rounding stages.
//
// With few K-steps (e.g. the down projection of one GPU's share I = 96 under
// tensor parallelism) splitting K would leave waves idle and cost a cross-wave
// sum per unit, so the waves split the columns instead: a unit is (task, eight
// column blocks), wave w takes column block 8 g + w over the whole K and
// stores its own outputs (no LDS, no barrier).  Which split is faster depends
// on K and on the rows per task (measured over H, I in 320 .. 2880 with 16-
// and 64-row tasks): columns up to K = 384 / 768 / 1536 for 16 / 32 / 64-row
// tasks, K beyond.
#include "common.h"
#include "moe_internal.h"

namespace moe {

namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;

// Steps of the register ring: bf16 4 (2 + MT fragments per step), W4 2
// (2 words + 4 MT token fragments per group).
template <bool W4>
constexpr int kFlexRing = W4 ? 2 : 4;

// K at or below which the waves split the columns instead of K, by token
// blocks per task.
constexpr int column_k(int MT) { return MT == 1 ? 384 : MT == 2 ? 768 : 1536; }

template <int KIND, int MT, bool W4, bool SPLIT>
__global__ __launch_bounds__(kThreads) void flex_kernel(ExpertArgs a) {
  static_assert(!W4 || KIND == 0, "W4G128 holds the gate/up weights only");
  constexpr int NRB = 2;
  constexpr int D = kFlexRing<W4>;
  constexpr int KPS = W4 ? 4 : 1;  // 32-wide MFMA k-steps per ring step
  extern __shared__ f32x4 s_red[];  // [kWaves][NRB][MT][64]

  const int H = a.H, I = a.I;
  const int ncb = KIND == 0 ? I / 16 : H / 32;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & (kWave - 1);
  const int r = lane & 15, g = lane >> 4;
  // Unit of this workgroup: (task, column block) or, without the K split,
  // (task, group of kWaves column blocks).
  const int per_task = SPLIT ? ncb : (ncb + kWaves - 1) / kWaves;
  const int task = blockIdx.x / per_task, ub = blockIdx.x - task * per_task;
  const int cb = SPLIT ? ub : ub * kWaves + wave;
  if (task >= *a.num_tasks || cb >= ncb) return;  // no barrier follows without the split
  const int4 tk = a.tasks[task];
  const int expert = tk.x, row0 = tk.y, rows = tk.z;

  const int K = KIND == 0 ? H : I;
  const int nsteps = W4 ? K / 128 : K / 32;
  // K-steps of this wave: w, w + 8, ... with the split, all of them without.
  const int mine = SPLIT ? (wave < nsteps ? (nsteps - 1 - wave) / kWaves + 1 : 0) : nsteps;
  const int sfirst = SPLIT ? wave : 0, sstride = SPLIT ? kWaves : 1;

  // Token blocks holding rows of this task (wave-uniform); the loads and
  // MFMAs of the others are skipped.
  const int nmt = __builtin_amdgcn_readfirstlane((rows + 15) >> 4);
  // Token rows of this lane's B fragments (rows past the task's end read the
  // task's first row: finite data in columns the epilogue never stores).
  const uint16_t *brow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int j = mt * 16 + r;
    const int jj = j < rows ? j : 0;
    brow[mt] = KIND == 0 ? a.x + (size_t)a.row_token[row0 + jj] * H + g * 8
                         : a.act + (size_t)(row0 + jj) * I + g * 8;
  }
  // Weight rows of this lane's A fragments.
  const uint16_t *arow[NRB];
  size_t w4unit[NRB];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb) {
    if constexpr (W4) {
      w4unit[rb] = ((size_t)expert * (2 * I / 16) + cb + (rb ? I / 16 : 0)) * (size_t)(H / 128);
    } else {
      const size_t wr = KIND == 0 ? (size_t)expert * 2 * I + (rb ? I : 0) + cb * 16 + r
                                  : (size_t)expert * H + cb * 32 + rb * 16 + r;
      arow[rb] = (KIND == 0 ? a.gate_up : a.down) + wr * K + g * 8;
    }
  }

  u32x4 ra[D][NRB], rbuf[D][MT][KPS];
  uint32_t rs[D][NRB];
  auto load = [&](int j, int d) __attribute__((always_inline)) {
    const int st = sfirst + j * sstride;
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
      if constexpr (W4) {
        const size_t u = w4unit[rb] + st;
        ra[d][rb] = load_u128_at((const uint8_t *)a.w4_words + u * (kWave * 16), (uint32_t)lane * 16u);
        rs[d][rb] = load_u16_at((const uint8_t *)a.w4_scales + u * 32, (uint32_t)r * 2u);
      } else {
        ra[d][rb] = *(const u32x4 *)(arow[rb] + st * 32);
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if (mt > 0 && mt >= nmt) break;  // token blocks past the task's last row
#pragma unroll
      for (int ks = 0; ks < KPS; ++ks)
        rbuf[d][mt][ks] = *(const u32x4 *)(brow[mt] + (size_t)(st * KPS + ks) * 32);
    }
  };

  f32x4 acc[NRB][MT];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[rb][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int d) __attribute__((always_inline)) {
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
      if constexpr (W4) {
        const W4Scale ks = w4_scale(bf16_bits_to_f32(rs[d][rb]));
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const u32x4 af = w4_decode8(ra[d][rb][q], ks);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            if (mt > 0 && mt >= nmt) break;
            acc[rb][mt] = mfma16(af, rbuf[d][mt][q], acc[rb][mt]);
          }
        }
      } else {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          if (mt > 0 && mt >= nmt) break;
          acc[rb][mt] = mfma16(ra[d][rb], rbuf[d][mt][0], acc[rb][mt]);
        }
      }
    }
  };

#pragma unroll
  for (int d = 0; d < D; ++d)
    if (d < mine) load(d, d);
  for (int j0 = 0; j0 < mine; j0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int j = j0 + d;
      if (j < mine) {
        compute(d);
        if (j + D < mine) load(j + D, d);
      }
    }
  }

  if constexpr (!SPLIT) {
    // Output (rb, mt, i) of this lane: weight row 16 rb + 4 g + i of the
    // block, token row mt * 16 + r of the task; four consecutive columns,
    // one 8-byte store.
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int j = mt * 16 + r;
      if (j >= rows) continue;
      if constexpr (KIND == 0) {
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float gt = bf16_round(acc[0][mt][i]);
          const float up = bf16_round(acc[1][mt][i]);
          v[i] = gt / (1.0f + expf(-gt)) * up;
        }
        u32x2 packed;
        packed[0] = pack_bf16x2(v[0], v[1]);
        packed[1] = pack_bf16x2(v[2], v[3]);
        *(u32x2 *)(a.act + (size_t)(row0 + j) * I + cb * 16 + 4 * g) = packed;
      } else {
        const size_t q = (size_t)a.row_route[row0 + j];
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {
          u32x2 packed;
          packed[0] = pack_bf16x2(acc[rb][mt][0], acc[rb][mt][1]);
          packed[1] = pack_bf16x2(acc[rb][mt][2], acc[rb][mt][3]);
          *(u32x2 *)(a.routed + q * H + cb * 32 + rb * 16 + 4 * g) = packed;
        }
      }
    }
    return;
  }

  // Fixed-order sum of the eight K-slices.
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) s_red[((wave * NRB + rb) * MT + mt) * kWave + lane] = acc[rb][mt];
  __syncthreads();
  // Output (rb, mt, lane, i): weight row 16 rb + 4 (lane / 16) + i of the
  // block, token row mt * 16 + lane % 16 of the task.
  if constexpr (KIND == 0) {
    for (int o = tid; o < MT * kWave * 4; o += kThreads) {
      const int i = o & 3, l = (o >> 2) & 63, mt = o >> 8;
      const int j = mt * 16 + (l & 15);
      float sg = 0.f, su = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        sg += s_red[((w * NRB + 0) * MT + mt) * kWave + l][i];
        su += s_red[((w * NRB + 1) * MT + mt) * kWave + l][i];
      }
      const float gt = bf16_round(sg);
      const float up = bf16_round(su);
      const float v = gt / (1.0f + expf(-gt)) * up;
      if (j < rows)
        a.act[(size_t)(row0 + j) * I + cb * 16 + 4 * (l >> 4) + i] = (uint16_t)(pack_bf16x2(v, 0.f) & 0xffffu);
    }
  } else {
    for (int o = tid; o < NRB * MT * kWave * 4; o += kThreads) {
      const int i = o & 3, l = (o >> 2) & 63, mt = (o >> 8) % MT, rb = (o >> 8) / MT;
      const int j = mt * 16 + (l & 15);
      float sm = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) sm += s_red[((w * NRB + rb) * MT + mt) * kWave + l][i];
      if (j < rows)
        a.routed[(size_t)a.row_route[row0 + j] * H + cb * 32 + rb * 16 + 4 * (l >> 4) + i] =
            (uint16_t)(pack_bf16x2(sm, 0.f) & 0xffffu);
    }
  }
}

template <int KIND, int MT, bool W4>
hipError_t launch_mt(const ExpertArgs &a, int task_capacity, hipStream_t s) {
  const int ncb = KIND == 0 ? a.I / 16 : a.H / 32;
  if ((KIND == 0 ? a.H : a.I) <= column_k(MT)) {
    const long long grid = (long long)task_capacity * ((ncb + kWaves - 1) / kWaves);
    if (grid <= 0) return hipSuccess;
    hipLaunchKernelGGL((flex_kernel<KIND, MT, W4, false>), dim3((unsigned)grid), dim3(kThreads), 0, s, a);
    return hipGetLastError();
  }
  const long long grid = (long long)task_capacity * ncb;
  if (grid <= 0) return hipSuccess;
  const size_t lds = (size_t)kWaves * 2 * MT * kWave * sizeof(f32x4);
  auto k = flex_kernel<KIND, MT, W4, true>;
  static const bool attr = hipFuncSetAttribute((const void *)k,
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)lds) == hipSuccess;
  if (!attr) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(kThreads), lds, s, a);
  return hipGetLastError();
}

template <int KIND, bool W4>
hipError_t launch_tb(const ExpertArgs &a, int task_capacity, int token_block, hipStream_t s) {
  switch (token_block) {
    case 16: return launch_mt<KIND, 1, W4>(a, task_capacity, s);
    case 32: return launch_mt<KIND, 2, W4>(a, task_capacity, s);
    case 64: return launch_mt<KIND, 4, W4>(a, task_capacity, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool flex_shape_ok(int H, int I, bool w4) {
  if (w4) return H % 128 == 0 && I % 32 == 0;  // W4G128 groups along H; down K = I
  return H % 32 == 0 && I % 32 == 0;
}

hipError_t launch_flex_gate_up(const ExpertArgs &a, int task_capacity, int token_block, bool w4,
                               hipStream_t s) {
  return w4 ? launch_tb<0, true>(a, task_capacity, token_block, s)
            : launch_tb<0, false>(a, task_capacity, token_block, s);
}

hipError_t launch_flex_down(const ExpertArgs &a, int task_capacity, int token_block, hipStream_t s) {
  return launch_tb<1, false>(a, task_capacity, token_block, s);
}

}  // namespace moe
