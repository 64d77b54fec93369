// Segmented-KV GQA prefill attention on gfx950 (secondary path).
//
// Semantics (reference: compact_gqa_forward, cuda_gqa_attention_compact.cu:77-209;
// contract docs/MOE_USAGE.md:128-134 and tests/e2e/test_compact_attention.py:49-78):
//   O = softmax(Q K^T * scale + mask) V over the concatenation of up to four
//   K/V segments; every key of the history segments is visible, keys of the
//   last (current) segment are causal (key j visible to query i iff j <= i);
//   query head h reads KV head h / (Hq / Hkv).  Scores and the softmax state
//   are fp32, probabilities are rounded to bf16 for the P.V product (as the
//   reference does), the output is bf16.
//
// Design.  A workgroup of four or eight waves owns 16 * RB query rows of one
// KV head (RB = 1 or 2 16-row blocks, each one query head x 16 tokens).  The
// waves split the workgroup's visible keys into contiguous ranges and each
// wave runs its own online softmax over all of the workgroup's rows, 32 keys
// per step, with no workgroup barrier in the loop:
//   * scores are computed transposed, S^T = K Q^T, with 16x16x32 bf16 MFMAs;
//     Q fragments (B operand) stay in registers for the whole kernel, and the
//     score tile lands in the A-operand layout of the P.V MFMA, so P never
//     goes through LDS;
//   * each step's K and V rows go from HBM straight into a wave-private K
//     stage and V stage in LDS (buffer loads with an LDS destination, whole
//     128-byte lines per load); K is read back as A fragments, V with
//     ds_read_b64_tr_b16, whose 16-lane transpose yields the B operand
//     directly; the next step's loads are issued while the current one
//     computes.
// At the end the waves' (max, sum, O) states are merged in LDS in fixed wave
// order.  When there are too few workgroups to fill the chip the keys are
// also split across workgroups and a second kernel merges the partial states
// in fixed split order (gqa_shape).
#include <climits>
#include <type_traits>
#include "common.h"
#include "gqa_internal.h"

namespace moe {

namespace {

constexpr int kD = 128;      // head_dim
constexpr int kKC = 32;      // keys per wave step
constexpr int kMaxSplits = 16;
constexpr float kLog2e = 1.4426950408889634f;

typedef short i16x4 __attribute__((ext_vector_type(4)));
#define GQA_LDS __attribute__((address_space(3)))

__device__ __forceinline__ int sgpr(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ uint64_t sgpr64(uint64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}

// Loads through the global address space: generic (flat) loads also count in
// the LDS wait counter, so every LDS wait of the compute loop would wait for
// the next tile's prefetch as well.
#define GQA_GLOBAL __attribute__((address_space(1)))
template <class V>
__device__ __forceinline__ V gload_as(const void *p) {
  return *(const GQA_GLOBAL V *)(const GQA_GLOBAL void *)p;
}

// LDS reads of the stages that the buffer loads with an LDS destination
// fill, written as inline assembly: the compiler cannot tell which of those
// loads a read depends on and would wait for all of them, including the
// next step's.  The reads are only issued here; lds_wait() completes them
// and hands the registers on (the "+v" operands keep every use of them
// after it), and the kernel waits for the loads with exact counts itself.
// `off` is a compile-time byte offset.
__device__ __forceinline__ uint32_t lds_addr(const uint8_t *p) {
  return (uint32_t)(uintptr_t)(const GQA_LDS uint8_t *)p;
}
template <int OFF>
__device__ __forceinline__ u32x4 lds_issue_b128(uint32_t addr) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
  return v;
}
// ds_read_b64_tr_b16: within each group of 16 lanes, lane 4a+b receives
// element b of the 8-byte rows addressed by lanes a, a+4, a+8, a+12.
template <int OFF>
__device__ __forceinline__ u32x2 lds_issue_tr16(uint32_t addr) {
  u32x2 v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
  return v;
}
__device__ __forceinline__ void lds_wait(u32x2 (&v)[16]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7]),
                 "+v"(v[8]), "+v"(v[9]), "+v"(v[10]), "+v"(v[11]), "+v"(v[12]), "+v"(v[13]), "+v"(v[14]), "+v"(v[15])
               :
               : "memory");
}
__device__ __forceinline__ void lds_wait(u32x4 (&v)[8]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7])
               :
               : "memory");
}

// 16 bytes per lane from a buffer straight into LDS (lane l's bytes at
// dst + 16 l); lanes whose offset is past the descriptor's size read zero.
// The builtin is compiled in the device pass only: in the host pass a kernel
// that calls it loses its launch stub.
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t rs, uint8_t *dst, uint32_t off) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (GQA_LDS void *)dst, 16, off, 0, 0, 0);
#endif
}

// Reductions over the four 16-lane rows holding one token's keys (lanes
// l, l^16, l^32, l^48) with the gfx950 lane-swap instructions (VALU only):
// swapping halves/rows of two copies leaves each lane with its own value and
// its partner's, combined in the same order on both lanes.
__device__ __forceinline__ float rows_max(float x) {
  const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float y = fmaxf(__uint_as_float(h[0]), __uint_as_float(h[1]));
  const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  return fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
}
__device__ __forceinline__ float rows_sum(float x) {
  const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float y = __uint_as_float(h[0]) + __uint_as_float(h[1]);
  const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// Running maxima lag the true maxima by at most this much (base-2 exponent),
// so probabilities stay <= 2^8 and O is rescaled only when a row's maximum
// grows past it (softmax is invariant to the reference maximum).
constexpr float kRescaleSlack = 8.f;

// One step's keys: up to 32 consecutive keys that all lie in one segment, so
// the row addresses are (segment base) + row * (segment stride) with
// wave-uniform base and stride.
struct Tile {
  int pos;          // global index of the first key
  int n;            // valid rows (1..32; 0 = past the wave's last key)
  int local0;       // index of the first key within its segment
  int send;         // global end of the tile's segment
  bool causal;      // the keys lie in the current (causal) segment
  const uint8_t *kb, *vb;  // row 0 (KV head offset included)
  uint32_t ksb, vsb;       // token strides in bytes (32 * stride < 2^31, checked on the host)
};

// Workgroups are dispatched round-robin over the 8 XCDs, each with its own L2.
// The 1-D grid is remapped so that XCD x runs a contiguous range of logical
// workgroups, ordered KV-head major: the workgroups that read the same K/V
// rows then share one L2.  Returns the logical index of this workgroup.
constexpr int kXcds = 8;
__device__ __forceinline__ int xcd_logical_block(int id, int n) {
  const int x = id % kXcds, slot = id / kXcds, per = n / kXcds, extra = n % kXcds;
  return x * per + min(x, extra) + slot;
}

// RB 16-row blocks per wave; HPW query heads per workgroup (HPW divides RB);
// row block rb is (head rb % HPW, token block rb / HPW); NW waves split the
// workgroup's keys.  With RB = 2 the kernel keeps two waves per SIMD: two
// four-wave workgroups or one eight-wave workgroup per CU.
template <int RB, int HPW, int NW>
__global__ __launch_bounds__(64 * NW, NW == 8 ? 1 : 4 / RB) void gqa_fwd_kernel(GqaArgs a, int head_groups,
                                                                               int nqb, int nsplit) {
  constexpr int kWaves = NW;
  constexpr int kRB = RB;
  constexpr int QT = 16 * (kRB / HPW);                 // tokens per workgroup
  constexpr int kVBlock = 4 * kD * 2 + 32;             // V stage block: four rows + pad
  constexpr int kStage = 8 * kVBlock;                  // V stage per wave (8.25 KiB)
  // LDS: per wave one K stage and one V stage.  The merge after the loop
  // reuses them: O states of row block 0 in the K array, of row block 1 in
  // the V array, (m, l) after the O states in the K array.
  constexpr int kKBlock = 8 * 128 + 64;                // K stage block: 8 keys x 128 bytes + pad
  constexpr int kKStage = 8 * kKBlock;
  constexpr int kOBytes = kWaves * 8 * 64 * 16;        // O states of one row block
  constexpr int kMLBytes = kWaves * kRB * 16 * 2 * 4;  // (m, l) per row
  static_assert(kRB <= 2 && kOBytes <= kWaves * kStage && kOBytes <= kWaves * kKStage,
                "O states fit the stage arrays");
  static_assert(kOBytes + kMLBytes <= kWaves * kKStage, "(m, l) fit after the O states");
  __shared__ __attribute__((aligned(16))) uint8_t kst[kWaves * kKStage];
  __shared__ __attribute__((aligned(16))) uint8_t vst[kWaves * kStage];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = sgpr(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  // Logical workgroup = ((KV head group) * nsplit + split) * nqb + query block.
  const int lb = xcd_logical_block(blockIdx.x, gridDim.x);
  const int qb = lb % nqb, split = (lb / nqb) % nsplit, kvg = lb / (nqb * nsplit);
  const int q0 = qb * QT;
  const int G = a.Hq / a.Hkv;
  const int kvh = kvg / head_groups;
  const int h0 = kvh * G + (kvg % head_groups) * HPW;
  const int T = a.T;
  const int hist = a.history;

  // Segment starts (global key index); absent segments start at INT_MAX and
  // empty ones coincide with the next start, so the count below skips them.
  const int nseg = sgpr(a.num_segments);
  const int l0 = sgpr(a.len[0]), l1 = sgpr(a.len[1]), l2 = sgpr(a.len[2]);
  const int st1 = nseg > 1 ? l0 : INT_MAX;
  const int st2 = nseg > 2 ? l0 + l1 : INT_MAX;
  const int st3 = nseg > 3 ? l0 + l1 + l2 : INT_MAX;

  // Visible keys of the workgroup: all history + current keys < q0 + QT, in
  // 32-key chunks split across workgroups (split) and then across waves.
  const int nvis = hist + min(T, q0 + QT);
  const int nch = (nvis + kKC - 1) / kKC;
  const int c0 = (int)((long long)nch * split / nsplit), c1 = (int)((long long)nch * (split + 1) / nsplit);
  const int cw0 = c0 + (c1 - c0) * wave / kWaves, cw1 = c0 + (c1 - c0) * (wave + 1) / kWaves;
  const int k_beg = cw0 * kKC, k_end = min(cw1 * kKC, nvis);

  auto tile_at = [&](int pos) __attribute__((always_inline)) {
    Tile t;
    const int seg = sgpr((pos >= st1) + (pos >= st2) + (pos >= st3));
    const int sbeg = seg == 0 ? 0 : seg == 1 ? st1 : seg == 2 ? st2 : st3;
    const int send = seg == 0 ? st1 : seg == 1 ? st2 : seg == 2 ? st3 : INT_MAX;
    t.pos = pos;
    t.n = max(0, min(kKC, min(send, k_end) - pos));
    t.local0 = pos - sbeg;
    t.send = send;
    t.causal = seg == nseg - 1;
    // seg is wave-uniform, so these are scalar loads of the kernel arguments.
    const int64_t ks = a.k_stride[seg], vs = a.v_stride[seg];
    t.ksb = (uint32_t)(2 * ks);
    t.vsb = (uint32_t)(2 * vs);
    t.kb = (const uint8_t *)(a.k[seg] + (int64_t)t.local0 * ks + (int64_t)kvh * kD);
    t.vb = (const uint8_t *)(a.v[seg] + (int64_t)t.local0 * vs + (int64_t)kvh * kD);
    return t;
  };

  // Q fragments (B operand of S^T = K Q^T): lane l -> token l%16 of the row
  // block, dims 32*ks + 8*(l/16) .. +8; rows past T repeat row T - 1.
  u32x4 qf[kRB][4];
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) {
    int tok = q0 + 16 * (rb / HPW) + r;
    tok = tok < T ? tok : T - 1;
    const uint16_t *qp = a.q + ((int64_t)tok * a.Hq + h0 + rb % HPW) * kD + 8 * g;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qf[rb][ks] = gload_as<u32x4>(qp + 32 * ks);
  }

  // Online softmax state of the lane's token (l % 16) per row block, fp32,
  // base-2 domain; O[rb][dt] holds tokens 4*(l/16) + i, dims 16*dt + l%16.
  float m_run[kRB], l_run[kRB];
  f32x4 o[kRB][8];
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) {
    m_run[rb] = -INFINITY;
    l_run[rb] = 0.f;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[rb][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const float sl2 = a.scale * kLog2e;

  // K and V of the next step are loaded while this one computes, straight
  // into the wave's LDS stages (buffer loads with an LDS destination: lane l
  // of a load writes 16 bytes at the stage block + 16 l).  Every load goes
  // through a buffer descriptor bounded at the tile's n rows, so rows past a
  // partial tile read as zero (masked out below) and a tile past the wave's
  // last key (n = 0) reads nothing -- but still issues its loads, so the
  // number of loads in flight after any given one is fixed and the waits
  // below are exact counts.
  u32x4 vb[8];
  // (The tile fields are wave-uniform; readfirstlane states it, so the
  // descriptor lives in scalar registers and no load is split per lane.)
  auto rsrc = [&](const uint8_t *base, uint32_t bytes) __attribute__((always_inline)) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)sgpr64((uint64_t)base), (short)0, sgpr((int)bytes), 0x00020000);
  };
  // K stage: load j (block j, kKBlock bytes apart) reads keys 8(j/2) .. +7,
  // bytes 128(j%2) .. +127 of each -- eight lanes per 128-byte line, so
  // every cache line is read whole -- with the eight 16-byte chunks of key k
  // permuted by k%8: lane l takes key 8(j/2) + l/8, chunk (l%8) ^ (l/8).
  auto issue_k = [&](const Tile &t, uint8_t *stage) __attribute__((always_inline)) {
    const auto rs = rsrc(t.kb, (uint32_t)t.n * t.ksb);
    const uint32_t lo = (uint32_t)(lane >> 3) * t.ksb + 16 * ((lane & 7) ^ (lane >> 3));
#pragma unroll
    for (int j = 0; j < 8; ++j)
      buffer_load_lds16(rs, stage + j * kKBlock, lo + (uint32_t)(8 * (j >> 1)) * t.ksb + 128 * (j & 1));
  };
  // A-operand fragment (kt, ks) of S^T -- lane (r, g) needs key 16kt + r,
  // chunk c = 4ks + g -- sits in block 4kt + 2(r/8) + ks/2 at 16-byte slot
  // 8(r%8) + (c%8 ^ r%8); c%8 ^ r%8 = (g ^ r%8) ^ 4(ks%2).  The sixteen
  // lanes of one g then read sixteen different 16-byte bank groups (the
  // blocks of keys r and r + 8 are 2 kKBlock = 128 (mod 256) bytes apart).
  const int kx = r & 7;
  const uint32_t kbase0 = (uint32_t)(2 * kKBlock * (r >> 3) + 128 * kx + 16 * (g ^ kx));
  const uint32_t kbase1 = (uint32_t)(2 * kKBlock * (r >> 3) + 128 * kx + 16 * ((g ^ kx) ^ 4));
  // V stage layout: block b (0..7, kVBlock bytes apart) holds keys b, b + 8,
  // b + 16, b + 24 as four 256-byte rows.  The transposed reads of a 16-lane
  // group then touch four blocks whose 32-byte pad puts their rows in
  // different banks, and every read address is one per-lane base plus an
  // immediate.
  auto issue_v = [&](const Tile &t, uint8_t *stage) __attribute__((always_inline)) {
    const auto rs = rsrc(t.vb, (uint32_t)t.n * t.vsb);
    const uint32_t lo = (uint32_t)(8 * g) * t.vsb + 16 * r;
#pragma unroll
    for (int b = 0; b < 8; ++b)
      buffer_load_lds16(rs, stage + b * kVBlock, lo + b * t.vsb);
  };
  // The tile after t: within a segment only the row pointers advance; the
  // segment's pointers and strides (dynamically indexed kernel arguments, a
  // scalar memory round trip) are read only when crossing into the next one.
  auto next_tile = [&](const Tile &t) __attribute__((always_inline)) {
    const int p = t.pos + t.n;
    Tile u = t;
    if (t.n == 0 || p >= k_end) {
      u.n = 0;
    } else if (p < t.send) {
      u.pos = p;
      u.n = min(kKC, min(t.send, k_end) - p);
      u.local0 = t.local0 + t.n;
      u.kb = t.kb + (size_t)t.n * t.ksb;
      u.vb = t.vb + (size_t)t.n * t.vsb;
    } else {
      u = tile_at(p);
    }
    return u;
  };

  // B operand of P.V from the staged V rows: lane (g, j = (l%16)/4,
  // a = l%4) reads key 4g + j -- block 4(g&1) + j, row g/2 -- at dims
  // 16dt + 4a .. +3, and key 16 + 4g + j two rows further; after the
  // transpose lane l holds dim 16dt + l%16 of keys 4g + 0..3 (+ 16).
  const uint32_t tr_base = (uint32_t)((4 * (g & 1) + (r >> 2)) * kVBlock + (g >> 1) * 256 + 8 * (r & 3));
  uint8_t *const kstage = kst + wave * kKStage;
  uint8_t *const vstage = vst + wave * kStage;

  Tile cur = tile_at(k_beg), nx = next_tile(cur);
  issue_k(cur, kstage);
  issue_v(cur, vstage);
  while (cur.n > 0) {
    // This step's K has landed once at most the 8 loads of its V remain.
    __builtin_amdgcn_s_waitcnt((8 & 15) | ((8 >> 4) << 14) | (7 << 4) | (15 << 8));
    // S^T: lane holds keys 16*kt + 4g + i of token r, per row block.
    f32x4 s[kRB][2];
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) s[rb][kt] = f32x4{0.f, 0.f, 0.f, 0.f};
    // Fragment (kt, ks) -> kf[2 ks + kt].
    u32x4 kf[8];
    {
      const uint32_t ka0 = lds_addr(kstage) + kbase0, ka1 = lds_addr(kstage) + kbase1;
      kf[0] = lds_issue_b128<0 * kKBlock>(ka0);
      kf[1] = lds_issue_b128<4 * kKBlock>(ka0);
      kf[2] = lds_issue_b128<0 * kKBlock>(ka1);
      kf[3] = lds_issue_b128<4 * kKBlock>(ka1);
      kf[4] = lds_issue_b128<1 * kKBlock>(ka0);
      kf[5] = lds_issue_b128<5 * kKBlock>(ka0);
      kf[6] = lds_issue_b128<1 * kKBlock>(ka1);
      kf[7] = lds_issue_b128<5 * kKBlock>(ka1);
      lds_wait(kf);
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) s[rb][kt] = mfma16(kf[2 * ks + kt], qf[rb][ks], s[rb][kt]);
    // The K stage is refilled only after every read of it has returned
    // (lds_wait above: the LDS-destination loads do not queue behind this
    // wave's LDS reads).
    issue_k(nx, kstage);
    // The softmax below runs at raised wave priority: while one wave of a
    // SIMD is in it, the other's MFMAs fill the matrix pipe (measured 1 %
    // faster at T = 96 / 256; raising it for the MFMA blocks instead: 5 %
    // slower).
    __builtin_amdgcn_s_setprio(1);
    const bool full = cur.n == kKC && !cur.causal;
    // Mask (raw scores): rows past the step's end and, in the current
    // segment, keys after the token (key j of the current chunk is token j).
    if (!full) {
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) {
        const int tok = q0 + 16 * (rb / HPW) + r;
        const int lim = cur.causal ? min(cur.n - 1, tok - cur.local0) : cur.n - 1;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) s[rb][kt][i] = 16 * kt + 4 * g + i <= lim ? s[rb][kt][i] : -INFINITY;
      }
    }
    // The row blocks' softmax chains are independent: every stage below runs
    // over all of them before the next, so their dependent instructions
    // interleave.  The scale is positive, so the maximum is taken on raw
    // scores and the scale is folded into the exponent's FMA (base-2 domain).
    float lmax[kRB];
    bool grow = false;
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) {
      lmax[rb] = fmaxf(fmaxf(fmaxf(s[rb][0][0], s[rb][0][1]), fmaxf(s[rb][0][2], s[rb][0][3])),
                       fmaxf(fmaxf(s[rb][1][0], s[rb][1][1]), fmaxf(s[rb][1][2], s[rb][1][3]))) * sl2;
      grow |= lmax[rb] > m_run[rb] + kRescaleSlack;
    }
    // Rescale only when some row's maximum outgrows the slack (one
    // wave-uniform branch for all row blocks).  A row's maximum exceeds
    // m + slack exactly when one of its four lanes' maxima does, so the
    // cross-lane maximum is only taken on this rare path; rows that did not
    // grow get alpha = 1 exactly.  A row with no visible key so far keeps
    // m = -inf.
    if (__builtin_amdgcn_ballot_w64(grow)) {
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) {
        const float m_new = fmaxf(m_run[rb], rows_max(lmax[rb]));
        const float alpha = __builtin_amdgcn_exp2f(m_run[rb] - (m_new == -INFINITY ? 0.f : m_new));
        l_run[rb] *= alpha;
        m_run[rb] = m_new;
        float al[4];  // O rows are tokens 4g + i; their alpha lives in lanes 4g + i
#pragma unroll
        for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * g + i, 64);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
          for (int i = 0; i < 4; ++i) o[rb][dt][i] *= al[i];
      }
    }
    // V is read after the rare rescale branch, so its 32 registers are not
    // live across it; the exponentials below cover the reads' latency.
    // This step's V has landed once at most the 8 loads of the next K remain.
    __builtin_amdgcn_s_waitcnt((8 & 15) | ((8 >> 4) << 14) | (7 << 4) | (15 << 8));
    // vr[2 dt] = dims 16dt.. of keys 4g + 0..3, vr[2 dt + 1] = keys 16 + 4g + 0..3.
    u32x2 vr[16];
    {
      const uint32_t va = lds_addr(vstage) + tr_base;
      vr[0] = lds_issue_tr16<0>(va);
      vr[1] = lds_issue_tr16<512>(va);
      vr[2] = lds_issue_tr16<32>(va);
      vr[3] = lds_issue_tr16<544>(va);
      vr[4] = lds_issue_tr16<64>(va);
      vr[5] = lds_issue_tr16<576>(va);
      vr[6] = lds_issue_tr16<96>(va);
      vr[7] = lds_issue_tr16<608>(va);
      vr[8] = lds_issue_tr16<128>(va);
      vr[9] = lds_issue_tr16<640>(va);
      vr[10] = lds_issue_tr16<160>(va);
      vr[11] = lds_issue_tr16<672>(va);
      vr[12] = lds_issue_tr16<192>(va);
      vr[13] = lds_issue_tr16<704>(va);
      vr[14] = lds_issue_tr16<224>(va);
      vr[15] = lds_issue_tr16<736>(va);
    }
    u32x4 pa[kRB];
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) {
      const float neg_m = m_run[rb] == -INFINITY ? 0.f : -m_run[rb];
      float p[2][4];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) p[kt][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[rb][kt][i], sl2, neg_m));
      // l is kept per lane (the lane's keys only) and summed over the row's
      // four lanes once, after the loop; alpha is the same on all four.
      l_run[rb] += ((p[0][0] + p[0][1]) + (p[0][2] + p[0][3])) + ((p[1][0] + p[1][1]) + (p[1][2] + p[1][3]));
      // A operand of P.V: slots 0..3 = keys 4g + i, slots 4..7 = keys 16 + 4g + i.
      pa[rb] = u32x4{pack_bf16x2(p[0][0], p[0][1]), pack_bf16x2(p[0][2], p[0][3]),
                     pack_bf16x2(p[1][0], p[1][1]), pack_bf16x2(p[1][2], p[1][3])};
    }
    __builtin_amdgcn_s_setprio(0);
    // The reads complete (and the stage may be refilled) once the
    // exponentials above have covered their latency.
    lds_wait(vr);
    issue_v(nx, vstage);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) vb[dt] = u32x4{vr[2 * dt][0], vr[2 * dt][1], vr[2 * dt + 1][0], vr[2 * dt + 1][1]};
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) o[rb][dt] = mfma16(pa[rb], vb[dt], o[rb][dt]);
    cur = nx;
    nx = next_tile(nx);
  }
  // The last issued loads (of empty tiles) may still be in flight; the merge
  // below reuses the stages.
  __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));

#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) l_run[rb] = rows_sum(l_run[rb]);

  // Merge of the waves' states, fixed wave order.  The staging areas
  // are reused, so every wave must be past its loop first.
  // O states of row block rb: [wave][dt][lane] x 4 at ost(rb); (m, l):
  // [wave][rb][row].
  auto ost = [&](int rb) __attribute__((always_inline)) {
    return (float *)(rb ? vst : kst);
  };
  float *ml = (float *)(kst + kOBytes);
  __syncthreads();
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) *(f32x4 *)(ost(rb) + ((wave * 8 + dt) * 64 + lane) * 4) = o[rb][dt];
    if (g == 0) *(f32x2_t *)(ml + ((wave * kRB + rb) * 16 + r) * 2) = f32x2_t{m_run[rb], l_run[rb]};
  }
  __syncthreads();

  // Wave w finalises row block w % RB, dims 16 kDT (w / RB) .. + 16 kDT (64
  // dims per wave with four waves and RB = 2, 32 with eight): lane holds
  // tokens 4g + i, dims 16dt + r.
  static_assert(kWaves % kRB == 0, "row blocks are shared out evenly over the waves");
  constexpr int kDT = 8 * kRB / kWaves;  // 16-dim column tiles per finalising wave
  const int rb = wave % kRB, dt0 = (wave / kRB) * kDT;
  const int head = h0 + rb % HPW;
  const int tb0 = q0 + 16 * (rb / HPW);
  float wgt[kWaves][4], M[4], L[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    M[i] = -INFINITY;
#pragma unroll
    for (int src = 0; src < kWaves; ++src) M[i] = fmaxf(M[i], ml[((src * kRB + rb) * 16 + 4 * g + i) * 2]);
    L[i] = 0.f;
#pragma unroll
    for (int src = 0; src < kWaves; ++src) {
      const f32x2_t st = *(const f32x2_t *)(ml + ((src * kRB + rb) * 16 + 4 * g + i) * 2);
      wgt[src][i] = st[0] == -INFINITY ? 0.f : exp2f(st[0] - M[i]);
      L[i] += wgt[src][i] * st[1];
    }
  }
  f32x4 acc[kDT];
#pragma unroll
  for (int j = 0; j < kDT; ++j) {
    acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int src = 0; src < kWaves; ++src) {
      const f32x4 v = *(const f32x4 *)(ost(rb) + ((src * 8 + dt0 + j) * 64 + lane) * 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[j][i] += wgt[src][i] * v[i];
    }
  }
  if (nsplit == 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tok = tb0 + 4 * g + i;
      if (tok >= T) continue;
      const float inv = L[i] > 0.f ? 1.0f / L[i] : 0.f;
      uint16_t *op = a.out + ((int64_t)tok * a.Hq + head) * kD + 16 * dt0 + r;
#pragma unroll
      for (int j = 0; j < kDT; ++j) op[16 * j] = (uint16_t)(pack_bf16x2(acc[j][i] * inv, 0.f) & 0xffffu);
    }
  } else {
    // Partial state: [split][token][head] {m, l, O[128]} fp32.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tok = tb0 + 4 * g + i;
      if (tok >= T) continue;
      float *pp = a.partial + (((int64_t)split * T + tok) * a.Hq + head) * (kD + 2);
      if (r == 0 && dt0 == 0) {
        pp[0] = M[i];
        pp[1] = L[i];
      }
#pragma unroll
      for (int j = 0; j < kDT; ++j) pp[2 + 16 * (dt0 + j) + r] = acc[j][i];
    }
  }
}

// (token, head) rows per merge workgroup: 1 / 2 / 4 / 8 measured 11.3 / 11.5 /
// 10.9 / 11.6 us per call at T = 32 (config-5 heads, four splits).
constexpr int kMergeRows = 4;

// out[t][h] = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s over the splits,
// combined in fixed split order, four splits per round trip: the loads of a
// group are issued together (a plain loop over a run-time count would issue
// one round trip per split) and the running maximum is rescaled between groups.
__global__ __launch_bounds__(128 * kMergeRows) void gqa_merge_kernel(GqaArgs a, int nsplit) {
  constexpr int kGroup = 4;
  const int th = blockIdx.x * kMergeRows + threadIdx.x / kD;  // token * Hq + head
  const int d = threadIdx.x % kD;
  if (th >= a.T * a.Hq) return;
  const float *base = a.partial + (int64_t)th * (kD + 2);
  const int64_t sstride = (int64_t)a.T * a.Hq * (kD + 2);
  float M = -INFINITY, num = 0.f, den = 0.f;
  for (int s0 = 0; s0 < nsplit; s0 += kGroup) {
    float m[kGroup], l[kGroup], ov[kGroup];
#pragma unroll
    for (int j = 0; j < kGroup; ++j) {
      const float *p = base + min(s0 + j, nsplit - 1) * sstride;
      m[j] = gload_as<float>(p);
      l[j] = gload_as<float>(p + 1);
      ov[j] = gload_as<float>(p + 2 + d);
    }
    float Mn = M;
#pragma unroll
    for (int j = 0; j < kGroup; ++j) Mn = s0 + j < nsplit ? fmaxf(Mn, m[j]) : Mn;
    if (Mn == -INFINITY) continue;  // nothing visible so far
    const float r = M == -INFINITY ? 0.f : exp2f(M - Mn);
    num *= r;
    den *= r;
#pragma unroll
    for (int j = 0; j < kGroup; ++j) {
      const float w = (s0 + j >= nsplit || m[j] == -INFINITY) ? 0.f : exp2f(m[j] - Mn);
      den += w * l[j];
      num += w * ov[j];
    }
    M = Mn;
  }
  const float v = den > 0.f ? num / den : 0.f;
  a.out[(int64_t)th * kD + d] = (uint16_t)(pack_bf16x2(v, 0.f) & 0xffffu);
}

}  // namespace

// Query heads per workgroup: RB row blocks of one head each, as many heads as
// the group has.
int gqa_heads_per_wg(int G, int rb) { return G < rb ? G : rb; }

int gqa_workgroups(int T, int Hkv, int G, int rb) {
  const int hpw = gqa_heads_per_wg(G, rb), qt = 16 * (rb / hpw);
  return ((T + qt - 1) / qt) * Hkv * (G / hpw);
}

// Launch shape.  While workgroups of one 16-row block per wave (RB = 1) fit
// the CUs once, those: the per-step chain of each wave is half as long and
// twice as many CUs work.  Eight-wave workgroups when they fill more than half
// the CUs, else four-wave ones with the keys split across up to four
// workgroups (256 CUs, config-5 heads: T = 16 / 32 / 48 / 64 / 96 / 128 take
// 10.4 / 11.4 / 14.0 / 14.6 / 15.4 / 15.7 us against 13.7 / 14.1 / 16.0 /
// 16.3 / 16.8 / 17.1 us with RB = 2).  Beyond that two row blocks per wave
// (RB = 2, each K/V step shared by 32 rows): with enough workgroups for two
// per CU, four-wave workgroups and no split; otherwise eight-wave
// workgroups, one per CU, and the keys split half as many times as would fill
// the CUs (the merge launch and its partial states cost more than idle CUs).
GqaShape gqa_shape(int T, int Hq, int Hkv, int num_cus) {
  const int G = Hq / Hkv;
  const int w1 = gqa_workgroups(T, Hkv, G, 1);
  if (w1 <= 0) return {1, 4, 2};
  if (w1 <= num_cus) {
    if (2 * w1 > num_cus) return {1, 8, 1};
    const int s = num_cus / w1;
    return {s < 4 ? s : 4, 4, 1};
  }
  const int w2 = gqa_workgroups(T, Hkv, G, 2);
  if (w2 >= 2 * num_cus) return {1, 4, 2};
  int s = num_cus / w2 / 2;
  if (s < 1) s = 1;
  if (s > kMaxSplits) s = kMaxSplits;
  return {s, 8, 2};
}

size_t gqa_partial_bytes(int T, int Hq, int nsplit) {
  return nsplit > 1 ? (size_t)nsplit * T * Hq * (kD + 2) * sizeof(float) : 0;
}

template <int RB, int NW>
hipError_t launch_fwd(const GqaArgs &a, int hpw, dim3 grid, int groups, int nqb, int nsplit,
                      hipStream_t s) {
  const dim3 block(64 * NW);
  if (hpw == 1)
    hipLaunchKernelGGL((gqa_fwd_kernel<RB, 1, NW>), grid, block, 0, s, a, groups, nqb, nsplit);
  else if (RB == 2 && hpw == 2)
    hipLaunchKernelGGL((gqa_fwd_kernel<2, 2, NW>), grid, block, 0, s, a, groups, nqb, nsplit);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_gqa(const GqaArgs &a, GqaShape shape, hipStream_t s) {
  if (a.T == 0) return hipSuccess;
  const int rb = shape.rb, G = a.Hq / a.Hkv, hpw = gqa_heads_per_wg(G, rb);
  const int qt = 16 * (rb / hpw), groups = G / hpw;
  const int nqb = (a.T + qt - 1) / qt;
  const int nsplit = shape.nsplit;
  const dim3 grid(nqb * a.Hkv * groups * nsplit);
  hipError_t e;
  if (rb == 1)
    e = shape.waves == 8 ? launch_fwd<1, 8>(a, hpw, grid, groups, nqb, nsplit, s)
                         : launch_fwd<1, 4>(a, hpw, grid, groups, nqb, nsplit, s);
  else
    e = shape.waves == 8 ? launch_fwd<2, 8>(a, hpw, grid, groups, nqb, nsplit, s)
                         : launch_fwd<2, 4>(a, hpw, grid, groups, nqb, nsplit, s);
  if (e != hipSuccess || nsplit == 1) return e;
  hipLaunchKernelGGL(gqa_merge_kernel, dim3((a.T * a.Hq + kMergeRows - 1) / kMergeRows),
                     dim3(kD * kMergeRows), 0, s, a, nsplit);
  return hipGetLastError();
}

}  // namespace moe
