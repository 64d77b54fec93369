// W4A16 gate/up + SwiGLU for tasks with several rows per expert on gfx950
// (reference: cuda_gate_up_w4_sync, cuda_w4_gate_up.cu:46-100; semantics of
// _dynamic_grouped_gate_up_swiglu, moe_fused.py:18-73).
//
// Unit = (task, 16 intermediate columns): 16 gate + 16 up weight rows against
// the task's 16*MT token rows.  One unit per wave over the whole K:
//
//  * The int4 weights stream from HBM straight into MFMA A registers (one
//    16-byte load per lane = 32 int4 of one row = a whole 128-K group, from
//    the tiled layout where each such load is 1 KiB contiguous) through a
//    ring of D4 groups, and each fragment is decoded once (w4_decode8,
//    bit-exact with the reference dequantisation) and used by MT MFMAs: at
//    MT = 4 the decode and the matrix cores carry comparable work instead of
//    the decode being paid once per 16 tokens.
//  * A workgroup = one task and 8 adjacent column blocks (8 waves).  The
//    task's token rows (MFMA B operand, gathered through the route list) are
//    staged in LDS in K-chunks of 32 KiB, double buffered: the next chunk is
//    loaded into registers while the current one is multiplied, so the only
//    workgroup barrier is one per chunk.  64 KiB of LDS per workgroup and at
//    most 128 VGPRs keep two workgroups per CU.
//  * The epilogue is in-wave (gate and up of a (feature, token) sit in the
//    same lane) with the reference's rounding stages.
#include <type_traits>

#include "common.h"
#include "moe_internal.h"

#define MOE_CONST __attribute__((address_space(4)))

namespace moe {

namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
constexpr int D4 = 2;                    // int4 groups in flight per wave (ring slots)
constexpr int kChunkBytes = 32 * 1024;   // one B buffer

template <typename T>
__device__ __forceinline__ const MOE_CONST T *as_const(const T *p) {
  return (const MOE_CONST T *)p;
}

// Calls f(integral_constant<int, d>) for d = 0, 1, ... in order.
template <class F, int... d>
__device__ __forceinline__ void unroll_seq(F &&f, std::integer_sequence<int, d...>) {
  (f(std::integral_constant<int, d>{}), ...);
}

// Byte offset of 16-byte chunk c of row `row` in a staged [rows][KC] chunk.
template <int KC>
__device__ __forceinline__ uint32_t b_off(int row, int c) {
  return (uint32_t)row * (KC * 2) + (uint32_t)((c ^ (row & 15)) << 4);
}

// MT = 1, 2: at most 128 VGPRs (4 waves per SIMD, two workgroups per CU): the
// decode is VALU-bound and one wave issues a VALU op only every few cycles.
// MT = 4 does four MFMAs per decoded fragment and keeps 2 waves per SIMD.
template <int MT>
__global__ __launch_bounds__(kThreads, 4) void wave_w4_kernel(ExpertArgs a) {
  constexpr int NRB = 2;
  constexpr int ROWS = 16 * MT;
  constexpr int KC = kChunkBytes / (ROWS * 2);  // K per chunk: 1024, 512, 256
  constexpr int GPC = KC / 128;                 // int4 groups per chunk: 8, 4, 2
  constexpr int BPT = kChunkBytes / 16 / kThreads;  // 16-byte B pieces per thread per chunk
  static_assert(GPC % D4 == 0, "a chunk holds whole ring rounds");
  __shared__ __attribute__((aligned(16))) uint8_t s_b[2][kChunkBytes];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & (kWave - 1);
  const int r = lane & 15, g = lane >> 4;
  const int H = a.H, I = a.I;
  const int nunits = I / 16;
  const int groups = (nunits + kWaves - 1) / kWaves;
  const int task = blockIdx.x / groups;
  if (task >= *as_const(a.num_tasks)) return;
  const int unit = (blockIdx.x - task * groups) * kWaves + wave;
  const bool active = unit < nunits;
  const int cb = active ? unit : 0;

  const MOE_CONST int32_t *tk = as_const((const int32_t *)a.tasks) + 4 * task;
  const int expert = tk[0], row0 = tk[1], rows = tk[2];

  // ---- weight ring (A operand) ---------------------------------------------
  const int NS = H >> 7;  // int4 groups along K
  size_t rbi[NRB];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb)
    rbi[rb] = ((size_t)expert * (2 * I / 16) + cb + (rb ? I / 16 : 0)) * NS;
  u32x4 ring[D4][NRB];
  uint32_t sring[D4][NRB];
  auto load_group = [&](int s, u32x4 (&slot)[NRB], uint32_t (&sslot)[NRB])
                        __attribute__((always_inline)) {
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
      const size_t u = rbi[rb] + s;
      slot[rb] = load_u128_at((const uint8_t *)a.w4_words + u * (kWave * 16), (uint32_t)lane * 16u);
      sslot[rb] = load_u16_at((const uint8_t *)a.w4_scales + u * 32, (uint32_t)r * 2u);
    }
  };
  if (active) {
#pragma unroll
    for (int d = 0; d < D4; ++d) load_group(d, ring[d], sring[d]);
  }

  // ---- token rows (B operand), K-chunked and double buffered ---------------
  // Thread piece i covers row (i*512 + tid) / (KC/8), 16-byte chunk
  // (i*512 + tid) % (KC/8) of every K-chunk; rows past the task's end load
  // row 0 (finite data in columns the epilogue never stores).
  const uint16_t *bsrc[BPT];
  uint32_t bdst[BPT];
#pragma unroll
  for (int i = 0; i < BPT; ++i) {
    const int idx = i * kThreads + tid;
    const int row = idx / (KC / 8), c = idx % (KC / 8);
    const int rr = row < rows ? row : 0;
    bsrc[i] = a.x + (size_t)a.row_token[row0 + rr] * H + 8 * c;
    bdst[i] = b_off<KC>(row, c);
  }
  u32x4 breg[BPT];
  auto bload = [&](int c) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < BPT; ++i) breg[i] = *(const u32x4 *)(bsrc[i] + (size_t)c * KC);
  };
  auto bstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < BPT; ++i) *(u32x4 *)(s_b[buf] + bdst[i]) = breg[i];
  };

  const int NCH = H / KC;
  bload(0);
  bstore(0);
  if (NCH > 1) bload(1);
  __syncthreads();

  f32x4 acc[NRB][MT];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[rb][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Token blocks holding rows of this task (wave-uniform).
  const int nmt = __builtin_amdgcn_readfirstlane((rows + 15) >> 4);
  // Group s (ring slot d) against chunk buffer `buf`, whose first group is s0c.
  auto step = [&](int s, auto d_tag, int buf, int s0c) __attribute__((always_inline)) {
    constexpr int d = decltype(d_tag)::value;
    const uint8_t *bb = s_b[buf];
    // Both row blocks (gate, up) are decoded before the token fragments are
    // read, so each B fragment comes out of LDS once for two MFMAs.
    const W4Scale ks0 = w4_scale(bf16_bits_to_f32(sring[d][0]));
    const W4Scale ks1 = w4_scale(bf16_bits_to_f32(sring[d][1]));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u32x4 af0 = w4_decode8(ring[d][0][j], ks0);
      const u32x4 af1 = w4_decode8(ring[d][1][j], ks1);
      const int c = 4 * (4 * (s - s0c) + j) + g;  // 16-byte chunk of k-step within the chunk
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if (mt > 0 && mt >= nmt) break;  // 16-row blocks past the task's last row
        const u32x4 bf = *(const u32x4 *)(bb + b_off<KC>(mt * 16 + r, c));
        acc[0][mt] = mfma16(af0, bf, acc[0][mt]);
        acc[1][mt] = mfma16(af1, bf, acc[1][mt]);
      }
    }
    if (s + D4 < NS) load_group(s + D4, ring[d], sring[d]);
  };
  using std::integral_constant;
  // One ring round = D4 consecutive groups in slots 0 .. D4-1, starting at
  // group s0 (a multiple of D4) of the chunk that starts at group s0c.
  auto ring_round = [&](int s0, int buf, int s0c) __attribute__((always_inline)) {
    unroll_seq([&](auto dt) __attribute__((always_inline)) {
      step(s0 + decltype(dt)::value, dt, buf, s0c);
    }, std::make_integer_sequence<int, D4>{});
  };
  for (int c = 0; c < NCH; ++c) {
    const int buf = c & 1;
    if (active) {
      const int s0c = c * GPC;
#pragma unroll
      for (int q = 0; q < GPC / D4; ++q) ring_round(s0c + q * D4, buf, s0c);
    }
    // Stage chunk c+1 (already in registers) into the other buffer, whose last
    // readers (chunk c-1) passed the previous barrier; then request chunk c+2.
    if (c + 1 < NCH) bstore(buf ^ 1);
    __syncthreads();
    if (c + 2 < NCH) bload(c + 2);
  }
  if (!active) return;

  // ---- epilogue: lane holds features 4g + i of token row mt*16 + r ---------
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int j = mt * 16 + r;
    if (j >= rows) continue;
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
  }
}

template <int MT>
hipError_t launch_mt(const ExpertArgs &a, int task_capacity, hipStream_t s) {
  const int groups = (a.I / 16 + kWaves - 1) / kWaves;
  const long long grid = (long long)task_capacity * groups;
  if (grid <= 0) return hipSuccess;
  hipLaunchKernelGGL(wave_w4_kernel<MT>, dim3((unsigned)grid), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}


// ---------------------------------------------------------------------------
// W4 gate/up with whole-K waves: one 32x32x16 A fragment per wave holds 16
// gate rows (fragment rows 0-15) and the 16 up rows of the same features
// (rows 16-31), so the MFMA output puts gate and up of a (feature, token) in
// the same lane (output rows 8q + 4h + i: q = 0, 1 gate, q = 2, 3 up).
//
// Launched for 64-row tasks (MT = 3) and, with several rows per expert, for
// 16-row tasks (MT = 1).  Unit = (pass, 16 intermediate columns).  A pass is
// one planner task, or two consecutive tasks of an expert with at most 32*MT
// rows together, so
// each weight is decoded once for every row of such an expert.  Per 16-K step
// a wave decodes one packed int4 word per lane (w4_decode8, bit-exact with
// the reference dequantisation) and multiplies it against up to MT 32-token
// B fragments read from LDS.  The lane of a 32x32x16 A fragment holds row
// l%32 and K 16j + 8(l/32) .. +8 of step j: in the tiled layout (lane 16g + r
// of a 16-row block holds K 32j' + 8g) those are words j/2 of block lanes
// 16(l/32) + r (even j) and 16(2 + l/32) + r (odd j): two 16-byte loads per
// lane per 128-K group.
//
// Token rows are staged in LDS in chunks of KC (launched: 128 K, one int4
// group; double buffered), rows padded by 16 bytes: 16 lanes of a
// ds_read_b128 cover all 64 banks, and every B fragment address is one VGPR
// plus an immediate.  Within a group the steps are software pipelined (step
// j + 1's B fragments read and A fragment decoded while step j's MFMAs run).
// The group loop is fully unrolled (NS = H / 128): inside a loop the
// compiler's wait counts at the loop header were conservative and drained the
// weight prefetch.  Launched as 16-wave workgroups at four waves per SIMD
// (at most 128 VGPRs), the configuration that measured fastest against 12-wave
// workgroups at three per SIMD, 8-wave ones at four, 256-K chunks and a
// three-group weight ring.

__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// NW waves per workgroup, MINW waves per SIMD (VGPR budget 512 / MINW),
// NS = H / 128 groups along K, MT 32-token fragments per pass.
// TB: rows of a planner task (token_block).
template <int NW, int MINW, int NS, int MT, int D4, int kPairKC, int TB>
__global__ __launch_bounds__(NW * 64, MINW) void pair_w4_kernel(ExpertArgs a) {
  constexpr int kPairTask = TB;
  constexpr int kPairRowB = kPairKC * 2 + 16;  // padded LDS row
  constexpr int GPC = kPairKC / 128;           // int4 groups per chunk
  constexpr int ROWS = 32 * MT;                  // token rows per pass
  constexpr int CHUNK = ROWS * kPairRowB;        // LDS bytes per chunk
  constexpr int NT = NW * 64;
  constexpr int PIECES = ROWS * (kPairKC / 8);   // 16-byte pieces per chunk
  constexpr int NC = NS / GPC;                   // chunks along K
  constexpr int BPT = (PIECES + NT - 1) / NT;
  __shared__ __attribute__((aligned(16))) uint8_t s_b[2 * CHUNK];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & (kWave - 1);
  const int r32 = lane & 31, h = lane >> 5;
  const int H = a.H, I = a.I;
  const int nunits = I / 16;
  const int groups = (nunits + NW - 1) / NW;
  const int task = blockIdx.x / groups;
  if (task >= *as_const(a.num_tasks)) return;
  const int unit = (blockIdx.x - task * groups) * NW + wave;
  const bool active = unit < nunits;
  const int cb = active ? unit : 0;

  const MOE_CONST int32_t *tk = as_const((const int32_t *)a.tasks) + 4 * task;
  const int expert = tk[0];
  const int row0 = tk[1];
  int rows = tk[2];
  if (ROWS > kPairTask) {
    const int rel = row0 - as_const(a.offsets)[expert];
    const int left = as_const(a.counts)[expert] - rel;  // rows of the expert from this task on
    if ((rel / kPairTask) & 1) {
      if (left + kPairTask <= ROWS) return;             // taken by the previous task's pass
    } else if (left <= ROWS) {
      rows = left;                                       // this task and the next one
    }
  }

  // ---- weight ring (A operand) ----------------------------------------------
  const size_t gblk = (size_t)expert * (2 * I / 16) + cb;  // gate block; up block is I/16 later
  const uint8_t *wb = (const uint8_t *)a.w4_words + gblk * NS * (kWave * 16);
  const uint8_t *sb = (const uint8_t *)a.w4_scales + gblk * NS * 32;
  const uint32_t up_blk = (uint32_t)(r32 >> 4) * (uint32_t)(I / 16) * NS;
  const uint32_t woff = up_blk * (kWave * 16) + (uint32_t)(16 * h + (r32 & 15)) * 16u;
  const uint32_t soff = up_blk * 32u + (uint32_t)(r32 & 15) * 2u;
  u32x4 ring[D4][2];
  uint32_t sring[D4];
  auto load_group = [&](int s, u32x4 (&slot)[2], uint32_t &sslot) __attribute__((always_inline)) {
    slot[0] = load_u128_at(wb, woff + (uint32_t)s * (kWave * 16));
    slot[1] = load_u128_at(wb, woff + (uint32_t)s * (kWave * 16) + 32u * 16u);
    sslot = load_u16_at(sb, soff + (uint32_t)s * 32u);
  };
#pragma unroll
  for (int d = 0; d < D4; ++d) load_group(d, ring[d], sring[d]);

  // ---- token rows (B operand) -------------------------------------------------
  // Piece i of a thread: row idx / (KC / 8), 16-byte chunk idx % (KC / 8) of
  // the chunk; rows past the pass's end load row 0 (finite data in columns the
  // epilogue never stores).
  uint32_t bsrc[BPT], bdst[BPT];
#pragma unroll
  for (int i = 0; i < BPT; ++i) {
    const int idx = min(i * NT + tid, PIECES - 1);  // a short last round repeats the last piece
    const int row = idx / (kPairKC / 8), c = idx % (kPairKC / 8);
    const int rr = row < rows ? row : 0;
    bsrc[i] = ((uint32_t)a.row_token[row0 + rr] * (uint32_t)H + 8u * c) * 2u;
    bdst[i] = (uint32_t)(row * kPairRowB + c * 16);
  }
  u32x4 breg[BPT];
  auto bload = [&](int c) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < BPT; ++i) breg[i] = load_u128_at(a.x, bsrc[i] + (uint32_t)c * (kPairKC * 2));
  };
  auto bstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < BPT; ++i) *(u32x4 *)(s_b + buf * CHUNK + bdst[i]) = breg[i];
  };
  bload(0);
  bstore(0);
  if (NC > 1) bload(1);
  __syncthreads();

  f32x16 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[mt][i] = 0.f;

  const int nmt = __builtin_amdgcn_readfirstlane((rows + 31) >> 5);
  const uint32_t bl = (uint32_t)(r32 * kPairRowB + h * 16);
  auto step = [&](auto s_tag) __attribute__((always_inline)) {
    constexpr int s = decltype(s_tag)::value;
    constexpr int d = s % D4;
    if (active) {
      const uint8_t *bb = s_b + ((s / GPC) & 1) * CHUNK + bl + (s % GPC) * 256;
      const W4Scale ks = w4_scale(bf16_bits_to_f32(sring[d]));
      // Software pipelined: step j + 1's B fragments are read and its A
      // fragment decoded while step j's MFMAs run; the scheduler hints
      // interleave the decode's VALU instructions between the MFMAs.
      u32x4 af = w4_decode8(ring[d][0][0], ks);
      u32x4 bf[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) bf[mt] = *(const u32x4 *)(bb + mt * 32 * kPairRowB);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        u32x4 bn[MT], an;
        if (j < 7) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) bn[mt] = *(const u32x4 *)(bb + mt * 32 * kPairRowB + (j + 1) * 32);
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          if (mt == 0 || mt < nmt) acc[mt] = mfma32(af, bf[mt], acc[mt]);
        }
        if (j < 7) an = w4_decode8(ring[d][(j + 1) & 1][(j + 1) >> 1], ks);
        if (j < 7) {
          af = an;
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) bf[mt] = bn[mt];
        }
      }
    }
    if (s + D4 < NS) load_group(s + D4, ring[d], sring[d]);
    // After a chunk's second group: stage chunk c + 1 (in registers since the
    // start of chunk c) into the other buffer, whose last readers (chunk
    // c - 1) passed the previous barrier; then request chunk c + 2.  The
    // weight loads issued during chunk c stay in flight across the wait.
    constexpr int c = s / GPC;
    if (s % GPC == GPC - 1 && c + 1 < NC) {
      bstore((c + 1) & 1);
      __syncthreads();
      if (c + 2 < NC) bload(c + 2);
    }
  };
  unroll_seq([&](auto st) __attribute__((always_inline)) { step(st); },
             std::make_integer_sequence<int, NS>{});
  if (!active) return;

  // ---- epilogue: lane holds features 8q + 4h + i (q = 0, 1) of token 32mt + r32
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int tok = mt * 32 + r32;
    if (tok >= rows) continue;
    uint16_t *dst = a.act + (size_t)(row0 + tok) * I + cb * 16 + 4 * h;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float gt = bf16_round(acc[mt][4 * q + i]);
        const float up = bf16_round(acc[mt][4 * (q + 2) + i]);
        v[i] = gt / (1.0f + expf(-gt)) * up;
      }
      u32x2 packed;
      packed[0] = pack_bf16x2(v[0], v[1]);
      packed[1] = pack_bf16x2(v[2], v[3]);
      *(u32x2 *)(dst + 8 * q) = packed;
    }
  }
}

}  // namespace

// The 64-row-task kernel: H = 2048 (its unrolled group loop), I a multiple of
// 16, and x small enough for 32-bit buffer offsets.
bool pair_w4_ok(const ExpertArgs &a, int token_block) {
  return (token_block == 64 || token_block == 16) && a.H == 2048 && a.I % 16 == 0 &&
         (long long)a.T * a.H * 2 < (1LL << 31);
}

// K-chunks are 1024 / 512 / 256 wide for 16 / 32 / 64-row tasks (whole ring
// rounds each); H must hold whole chunks.
bool wave_w4_shape_ok(int H, int I, int token_block) {
  if (token_block != 16 && token_block != 32 && token_block != 64) return false;
  const int kc = kChunkBytes / (token_block * 2);
  return I > 0 && I % 16 == 0 && H % kc == 0;
}

hipError_t launch_wave_w4_gate_up(const ExpertArgs &a, int task_capacity, int token_block,
                                  hipStream_t s) {
  if (pair_w4_ok(a, token_block)) {
    constexpr int NW = 16;
    const int groups = (a.I / 16 + NW - 1) / NW;
    const long long grid = (long long)task_capacity * groups;
    if (grid <= 0) return hipSuccess;
    if (token_block == 64)
      hipLaunchKernelGGL((pair_w4_kernel<NW, 4, 16, 3, 2, 128, 64>), dim3((unsigned)grid), dim3(NW * 64), 0, s, a);
    else
      hipLaunchKernelGGL((pair_w4_kernel<NW, 4, 16, 1, 2, 256, 16>), dim3((unsigned)grid), dim3(NW * 64), 0, s, a);
    return hipGetLastError();
  }
  switch (token_block) {
    case 16: return launch_mt<1>(a, task_capacity, s);
    case 32: return launch_mt<2>(a, task_capacity, s);
    case 64: return launch_mt<4>(a, task_capacity, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace moe
