// LDS-tiled grouped GEMMs of the MoE forward on gfx950 for large row counts.
//
// When experts receive many rows (T = 1024, Zipf-skewed routing: a few
// experts take ~1000 rows), streaming each weight byte once per 16/32-row task
// would re-read the hot experts' weights dozens of times.  Here a task holds
// up to BM = 64 grouped rows and a work unit is (task, n-tile of BN weight
// rows); units are numbered expert-major and n-tile-major within an expert,
// and that sequence is cut into one contiguous chunk per XCD, so the tasks of
// an expert that share a weight tile, and the n-tiles of a task that share its
// token rows, are read through one XCD's L2 (HBM reads at T = 1024 Zipf:
// gate/up 765 -> 661 MB, down 382 -> 312 MB, against 4-task blocks dealt
// round-robin).
//
// Per unit: a K loop over BK-wide stages.  Each stage's weight tile [BN][BK]
// and token tile [BM][BK] go global -> LDS (the warp-specialised kernel
// below), 16-byte chunks XOR-swizzled by row so that the MFMA operand reads
// are bank-conflict free, then 8 waves (4 along N x 2 along M) run 16x16x32
// bf16 MFMAs.  (W4G128 gate/up with many rows per expert runs in
// the wave kernel of moe_wave.hip, which decodes each weight once into MFMA
// registers; the down weights are bf16 in both formats.)
//
// Epilogues match the streaming kernels: gate/up round to bf16, SwiGLU in
// fp32, bf16 act rows; down rounds to bf16 and scatters rows to route order.
#include "common.h"
#include "moe_internal.h"

#define MOE_CONST __attribute__((address_space(4)))

namespace moe {

namespace {

constexpr int BM = 64;

template <typename T>
__device__ __forceinline__ const MOE_CONST T *as_const(const T *p) {
  return (const MOE_CONST T *)p;
}

__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Byte offset of 16-byte chunk c of row `row` in a [rows][BK] bf16 tile.
template <int BK>
__device__ __forceinline__ int swz(int row, int c) {
  if constexpr (BK == 64) return row * 128 + ((c ^ ((row >> 1) & 7)) << 4);
  else return row * 256 + ((c ^ (row & 15)) << 4);
}


template <int KIND>
struct TileCfg {
  static constexpr int BN = 256;  // weight rows per tile
  static constexpr int BK = 64;
  static constexpr int WNT = BN / 4 / 16;                   // 16-row tiles per wave
  static constexpr int A_BYTES = BN * BK * 2;
  static constexpr int B_BYTES = BM * BK * 2;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int OUT_COLS = KIND == 0 ? BN / 2 : BN;  // output columns per n-tile
};

// ---- warp-specialised kernel ---------------------------------------------------
// The K stages move by global -> LDS direct loads (16 bytes per lane, gfx950)
// into a ring of kWsStages LDS stages, kWsStages - 1 stages ahead of the
// matrix cores.  Four loader waves
// issue every load and carry every vector-memory wait; the eight MFMA waves
// only read LDS.  One workgroup barrier per stage publishes that stage (the
// loaders waited for it) and frees the oldest buffer (every MFMA wave has
// finished reading it).  One 768-thread workgroup per CU owns all 160 KB of
// LDS.
constexpr int kWsConsumers = 8;
constexpr int kWsLoaders = 4;
constexpr int kWsThreads = (kWsConsumers + kWsLoaders) * 64;
constexpr int kWsStages = 4;

// s_waitcnt with only the vector-memory counter bounded (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <int KIND>
__global__ __launch_bounds__(kWsThreads) void tile_ws_kernel(ExpertArgs a) {
  using C = TileCfg<KIND>;
  constexpr int BN = C::BN, BK = C::BK, WNT = C::WNT;
  constexpr int KS = BK / 32;
  static_assert(BK == 64, "one 128-byte row piece per stage");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int H = a.H, I = a.I;
  const int Kdim = KIND == 0 ? H : I;
  const int KT = Kdim / BK;
  const int ntiles = (KIND == 0 ? I : H) / C::OUT_COLS;
  const int num_tasks = *as_const(a.num_tasks);
  const int total = num_tasks * ntiles;
  const MOE_CONST int32_t *tasks = as_const((const int32_t *)a.tasks);
  const int G = gridDim.x;
  // XCD-affine order: the unit sequence, expert-major and n-tile-major
  // within an expert (every task of the expert on one n-tile, then the next
  // n-tile), is cut into eight contiguous chunks, one per XCD (consecutive
  // workgroup IDs go round-robin over the XCDs), and the workgroups of an XCD
  // walk their chunk together.  So an expert's weight tile and its tasks'
  // token rows are read from one XCD's L2, except at the seven chunk edges.
  const bool xcd_mode = G % 8 == 0 && G >= 8;
  const int P = xcd_mode ? G / 8 : G;            // workgroups per XCD
  const int xcd = xcd_mode ? (int)blockIdx.x % 8 : 0;
  const int p = xcd_mode ? (int)blockIdx.x / 8 : (int)blockIdx.x;
  const int CH = xcd_mode ? (total + 7) / 8 : total;  // units per chunk
  const int c_end = min(CH, total - xcd * CH);
  const int nu = p < c_end ? (c_end - p + P - 1) / P : 0;
  const MOE_CONST int32_t *cnts = as_const(a.counts);
  const MOE_CONST int32_t *offs = as_const(a.offsets);
  const int nstages = nu * KT;

  struct Unit {
    int e, row0, rows, nt;
  };
  auto unit_of = [&](int i) {
    const int L = xcd * CH + p + i * P;
    const int T = L / ntiles;  // the task whose expert owns unit L
    const int e = tasks[4 * T];
    const int t0 = T - (tasks[4 * T + 1] - offs[e]) / BM;  // the expert's first task
    const int m = (cnts[e] + BM - 1) / BM;                 // and its task count
    const int local = L - ntiles * t0;
    Unit un;
    un.nt = local / m;
    const int t = t0 + (local - un.nt * m);
    un.e = e;
    un.row0 = tasks[4 * t + 1];
    un.rows = tasks[4 * t + 2];
    return un;
  };

  if (wave >= kWsConsumers) {
    // ---- loaders: wave lw moves tile rows [lw*64, +64) of the weights and
    // [lw*16, +16) of the tokens, 8 rows (1 KiB of LDS) per instruction.
    const int lw = wave - kWsConsumers;
    constexpr int A_PER = BN / kWsLoaders / 8;
    constexpr int B_PER = BM / kWsLoaders / 8;
    constexpr int PER = A_PER + B_PER;  // instructions per stage per loader wave
    static_assert(kWsStages == 4 && 2 * PER < 64, "wait counts below assume 4 stages");
    const uint16_t *asrc[A_PER];
    const uint16_t *bsrc[B_PER];
    int cur = -1;
    auto setup = [&](int i) {
      const Unit un = unit_of(i);
#pragma unroll
      for (int j = 0; j < A_PER; ++j) {
        const int row = lw * (BN / kWsLoaders) + j * 8 + lane / 8;  // tile row
        const int c = (lane % 8) ^ ((row >> 1) & 7);  // logical chunk of LDS chunk lane%8
        size_t wrow;
        if (KIND == 0)
          wrow = (size_t)un.e * 2 * I +
                 (row < BN / 2 ? un.nt * (BN / 2) + row : I + un.nt * (BN / 2) + row - BN / 2);
        else
          wrow = (size_t)un.e * H + un.nt * BN + row;
        asrc[j] = (KIND == 0 ? a.gate_up : a.down) + wrow * Kdim + c * 8;
      }
      // Token of each B row through scalar loads (the loaders' vector-memory
      // counter then holds only their LDS loads, so nothing here waits on
      // them); rows past the task's end take the task's first token.
      constexpr int BR = BM / kWsLoaders;  // B rows of this loader wave
      int tokv[BR];
      if (KIND == 0) {
        const MOE_CONST int32_t *rt = as_const(a.row_token) + un.row0;
        const int t0 = rt[0];
#pragma unroll
        for (int k = 0; k < BR; ++k) tokv[k] = lw * BR + k < un.rows ? rt[lw * BR + k] : t0;
      }
#pragma unroll
      for (int j = 0; j < B_PER; ++j) {
        const int row = lw * BR + j * 8 + lane / 8;
        const int c = (lane % 8) ^ ((row >> 1) & 7);
        size_t off;
        if (KIND == 0) {
          int tok = tokv[j * 8];
#pragma unroll
          for (int k = 1; k < 8; ++k) tok = lane / 8 == k ? tokv[j * 8 + k] : tok;
          off = (size_t)tok * H;
        } else {
          off = (size_t)(un.row0 + (row < un.rows ? row : 0)) * I;
        }
        bsrc[j] = (KIND == 0 ? a.x : a.act) + off + c * 8;
      }
    };
    auto issue = [&](int st) {
      const int i = st / KT, kt = st - (st / KT) * KT;
      if (i != cur) {
        setup(i);
        cur = i;
      }
      uint8_t *buf = smem + (st % kWsStages) * C::STAGE_BYTES;
#pragma unroll
      for (int j = 0; j < A_PER; ++j)
        __builtin_amdgcn_global_load_lds(
            (const void *)(asrc[j] + kt * BK),
            (__attribute__((address_space(3))) void *)(buf + (lw * (BN / kWsLoaders) + j * 8) * 128),
            16, 0, 0);
#pragma unroll
      for (int j = 0; j < B_PER; ++j)
        __builtin_amdgcn_global_load_lds(
            (const void *)(bsrc[j] + kt * BK),
            (__attribute__((address_space(3))) void *)(buf + C::A_BYTES +
                                                       (lw * (BM / kWsLoaders) + j * 8) * 128),
            16, 0, 0);
    };
    for (int st = 0; st < kWsStages - 1 && st < nstages; ++st) issue(st);
    for (int st = 0; st < nstages; ++st) {
      // Stage st has landed once at most the loads issued after it remain.
      const int later = min(kWsStages - 2, nstages - 1 - st);
      if (later >= 2) wait_vmcnt<2 * PER>();
      else if (later == 1) wait_vmcnt<PER>();
      else wait_vmcnt<0>();
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      // Buffer (st - 1) % stages was last read before this barrier.
      if (st + kWsStages - 1 < nstages) issue(st + kWsStages - 1);
    }
    return;
  }

  // ---- MFMA waves: (wn, wm) = 64 weight rows x 32 tokens ------------------
  const int wn = wave & 3, wm = wave >> 2;
  auto a_row = [&](int i) {
    if (KIND == 0) {
      constexpr int HALF_T = WNT / 2;
      return (i < HALF_T ? 0 : BN / 2) + wn * HALF_T * 16 + (i % HALF_T) * 16;
    }
    return wn * WNT * 16 + i * 16;
  };
  int st = 0;
  for (int i = 0; i < nu; ++i) {
    const Unit un = unit_of(i);
    f32x4 acc[WNT][2];
#pragma unroll
    for (int q = 0; q < WNT; ++q) acc[q][0] = acc[q][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int kt = 0; kt < KT; ++kt, ++st) {
      lds_barrier();  // stage st published; every read of stage st - 1 is done
      const uint8_t *abuf = smem + (st % kWsStages) * C::STAGE_BYTES;
      const uint8_t *bbuf = abuf + C::A_BYTES;
      const int r = lane & 15, g = lane >> 4;
      // Every fragment of the stage is requested before the first MFMA, so
      // the stage costs one LDS round trip.
      u32x4 bf[KS][2], af[KS][WNT];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int c = 4 * ks + g;
        bf[ks][0] = *(const u32x4 *)(bbuf + swz<BK>(wm * 32 + r, c));
        bf[ks][1] = *(const u32x4 *)(bbuf + swz<BK>(wm * 32 + 16 + r, c));
#pragma unroll
        for (int q = 0; q < WNT; ++q) af[ks][q] = *(const u32x4 *)(abuf + swz<BK>(a_row(q) + r, c));
      }
      __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the MFMAs
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int q = 0; q < WNT; ++q) {
          acc[q][0] = mfma16(af[ks][q], bf[ks][0], acc[q][0]);
          acc[q][1] = mfma16(af[ks][q], bf[ks][1], acc[q][1]);
        }
    }
    // Epilogue (registers only, no LDS): lane holds rows 4*(l/16)+k of its
    // 16-row weight tile for token l%16.
    const int g = lane >> 4;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int tok = wm * 32 + mt * 16 + (lane & 15);
      if (KIND == 0) {
        constexpr int HALF_T = WNT / 2;
#pragma unroll
        for (int q = 0; q < HALF_T; ++q) {
          const f32x4 sg = acc[q][mt], su = acc[q + HALF_T][mt];
          float v[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const float gt = bf16_round(sg[k]);
            const float up = bf16_round(su[k]);
            v[k] = gt / (1.0f + expf(-gt)) * up;
          }
          u32x2 packed;
          packed[0] = pack_bf16x2(v[0], v[1]);
          packed[1] = pack_bf16x2(v[2], v[3]);
          const int col = un.nt * (BN / 2) + wn * HALF_T * 16 + q * 16 + 4 * g;
          if (tok < un.rows) *(u32x2 *)(a.act + (size_t)(un.row0 + tok) * I + col) = packed;
        }
      } else {
        const int q0 = tok < un.rows ? a.row_route[un.row0 + tok] : 0;
#pragma unroll
        for (int q = 0; q < WNT; ++q) {
          u32x2 packed;
          packed[0] = pack_bf16x2(acc[q][mt][0], acc[q][mt][1]);
          packed[1] = pack_bf16x2(acc[q][mt][2], acc[q][mt][3]);
          const int col = un.nt * BN + wn * WNT * 16 + q * 16 + 4 * g;
          if (tok < un.rows) *(u32x2 *)(a.routed + (size_t)q0 * H + col) = packed;
        }
      }
    }
  }
}

template <int KIND>
hipError_t launch_tile_ws(const ExpertArgs &a, int units_bound, int num_cus, hipStream_t s) {
  using C = TileCfg<KIND>;
  auto k = tile_ws_kernel<KIND>;
  const size_t lds = (size_t)kWsStages * C::STAGE_BYTES;
  static bool attr = [&] {
    return hipFuncSetAttribute((const void *)k, hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)lds) == hipSuccess;
  }();
  if (!attr) return hipErrorInvalidValue;
  int grid = num_cus;
  if (grid > units_bound) grid = units_bound;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL(k, dim3(grid), dim3(kWsThreads), lds, s, a);
  return hipGetLastError();
}

}  // namespace

bool tile_shape_ok(int H, int I, bool w4) {
  // down (both formats): K = I in 64-wide stages (even count), H in 256-row tiles.
  if (I % 128 || H % 256) return false;
  // gate/up: bf16 here, K = H in 64-wide stages (even count), act columns in
  // 128-column tiles; W4 in the wave kernel.
  return w4 ? wave_w4_shape_ok(H, I, 64) : H % 128 == 0;
}

hipError_t launch_tile_gate_up(const ExpertArgs &a, int task_capacity, int num_cus, hipStream_t s) {
  return launch_tile_ws<0>(a, task_capacity * (a.I / 128), num_cus, s);
}

hipError_t launch_tile_down(const ExpertArgs &a, int task_capacity, int num_cus, hipStream_t s) {
  return launch_tile_ws<1>(a, task_capacity * (a.H / 256), num_cus, s);
}

}  // namespace moe
