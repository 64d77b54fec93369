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
// Design.  A workgroup owns one KV head, 16 query tokens and that head's
// G = Hq/Hkv query heads (wave w = query head), so each K/V tile loaded into
// LDS serves 16*G query rows.  Scores are computed transposed, S^T = K Q^T,
// with 16x16x32 bf16 MFMAs: Q fragments stay in registers for the whole
// kernel and the score tile lands in registers already in the A-operand
// layout the P.V MFMA needs (lane l: token l%16, keys {4g..4g+3, 16+4g..})
// so P never goes through LDS.  V is stored transposed in LDS (each lane
// loads 4 keys x 2 dims as fully coalesced 256-byte rows and writes two
// 8-byte columns), XOR-swizzled so the MFMA operand reads are conflict free.
// K tiles use the same 16-byte XOR swizzle as the expert GEMMs.  When there
// are too few (query block, KV head) pairs to fill the chip, the visible keys
// are split across workgroups and a second kernel merges the partial
// (max, sum, O) states in fixed split order.
#include "common.h"
#include "gqa_internal.h"

namespace moe {

namespace {

constexpr int kD = 128;      // head_dim
constexpr int kQB = 16;      // query tokens per workgroup
constexpr int kKT = 64;      // keys per tile
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Global key index -> pointer of key row (segment lookup; clamped keys are
// the caller's business).
__device__ __forceinline__ const uint16_t *key_row(const GqaArgs &a, const uint16_t *const *base,
                                                   const int64_t *stride, int key, int kvh) {
  int s = 0, off = key;
#pragma unroll
  for (int i = 0; i < kGqaMaxSegments - 1; ++i) {
    if (s == i && i < a.num_segments - 1 && off >= a.len[i]) {
      off -= a.len[i];
      s = i + 1;
    }
  }
  return base[s] + (int64_t)off * stride[s] + (int64_t)kvh * kD;
}

// K tile byte offset of 16-byte chunk c of key row r ([64][128] bf16, 256-B rows).
__device__ __forceinline__ int k_off(int r, int c) { return r * 256 + ((c ^ (r & 15)) << 4); }
// V^T tile byte offset of 8-byte chunk c (4 keys) of dim row d ([128][64] bf16).
__device__ __forceinline__ int v_off(int d, int c) { return d * 128 + ((c ^ (d & 15)) << 3); }

template <int G>
__global__ __launch_bounds__(64 * G) void gqa_partial_kernel(GqaArgs a) {
  constexpr int kThreads = 64 * G;
  __shared__ __attribute__((aligned(16))) uint8_t s_k[kKT * kD * 2];
  __shared__ __attribute__((aligned(16))) uint8_t s_v[kKT * kD * 2];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int r = lane & 15, g = lane >> 4;
  const int q0 = blockIdx.x * kQB;
  const int kvh = blockIdx.y;
  const int split = blockIdx.z, nsplit = gridDim.z;
  const int head = kvh * G + wave;
  const int T = a.T;
  const int hist = a.history;

  // Visible keys of this query block: all history + current keys < q0 + 16.
  const int cur_vis = min(T, q0 + kQB);
  const int nvis = hist + cur_vis;
  const int k_beg = (int)((long long)nvis * split / nsplit);
  const int k_end = (int)((long long)nvis * (split + 1) / nsplit);

  // Q fragments (B operand of S^T = K Q^T): lane l -> token q0 + l%16,
  // dims 32*ks + 8*(l/16) .. +8.
  u32x4 qf[4];
  {
    const int tok = q0 + r < T ? q0 + r : T - 1;
    const uint16_t *qp = a.q + ((int64_t)tok * a.Hq + head) * kD + 8 * g;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qf[ks] = *(const u32x4 *)(qp + 32 * ks);
  }

  // Online softmax state for the lane's token (l % 16), fp32, base-2 domain.
  float m_run = -INFINITY, l_run = 0.f;
  f32x4 o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  const float sl2 = a.scale * kLog2e;

  // Register staging of the next tile: K 64 rows x 256 B = 16 KB -> 16 B x
  // (1024 / kThreads * ... ) per thread; V as 4-key x 2-dim dword columns.
  constexpr int K_LOADS = kKT * kD * 2 / 16 / kThreads;  // 16-B loads per thread
  constexpr int V_QUADS = kKT / 4 / G;                    // 4-key groups per wave
  u32x4 kr[K_LOADS];
  uint32_t vr[V_QUADS][4];
  const uint16_t *kbase[kGqaMaxSegments] = {a.k[0], a.k[1], a.k[2], a.k[3]};
  const uint16_t *vbase[kGqaMaxSegments] = {a.v[0], a.v[1], a.v[2], a.v[3]};

  auto gload = [&](int t0) {
#pragma unroll
    for (int i = 0; i < K_LOADS; ++i) {
      const int idx = i * kThreads + tid;  // 16-B chunk index within the tile
      const int row = idx >> 4, c = idx & 15;
      int key = t0 + row;
      key = key < k_end ? key : k_beg;  // clamp: masked below, any valid row will do
      kr[i] = *(const u32x4 *)(key_row(a, kbase, a.k_stride, key, kvh) + 8 * c);
    }
#pragma unroll
    for (int qd = 0; qd < V_QUADS; ++qd) {
      const int kq = (wave * V_QUADS + qd) * 4;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        int key = t0 + kq + j;
        key = key < k_end ? key : k_beg;
        vr[qd][j] = *(const uint32_t *)(key_row(a, vbase, a.v_stride, key, kvh) + 2 * lane);
      }
    }
  };
  auto sts = [&]() {
#pragma unroll
    for (int i = 0; i < K_LOADS; ++i) {
      const int idx = i * kThreads + tid;
      *(u32x4 *)(s_k + k_off(idx >> 4, idx & 15)) = kr[i];
    }
#pragma unroll
    for (int qd = 0; qd < V_QUADS; ++qd) {
      const int c = wave * V_QUADS + qd;  // 4-key chunk index
      u32x2 lo, hi;  // dims 2*lane and 2*lane+1 of keys 4c..4c+3
      lo[0] = (vr[qd][0] & 0xffffu) | (vr[qd][1] << 16);
      lo[1] = (vr[qd][2] & 0xffffu) | (vr[qd][3] << 16);
      hi[0] = (vr[qd][0] >> 16) | (vr[qd][1] & 0xffff0000u);
      hi[1] = (vr[qd][2] >> 16) | (vr[qd][3] & 0xffff0000u);
      *(u32x2 *)(s_v + v_off(2 * lane, c)) = lo;
      *(u32x2 *)(s_v + v_off(2 * lane + 1, c)) = hi;
    }
  };

  if (k_beg < k_end) gload(k_beg);
  for (int t0 = k_beg; t0 < k_end; t0 += kKT) {
    sts();
    lds_barrier();
    if (t0 + kKT < k_end) gload(t0 + kKT);

    // S^T tile: 4 subtiles of 16 keys; lane holds keys 16*kt + 4g + i, token r.
    f32x4 s[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      s[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const u32x4 kf = *(const u32x4 *)(s_k + k_off(16 * kt + r, 4 * ks + g));
        s[kt] = mfma16(kf, qf[ks], s[kt]);
      }
    }
    // Mask, scale, tile max.
    const int tok = q0 + r;
    float tmax = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = t0 + 16 * kt + 4 * g + i;
        const bool ok = key < k_end && tok < T && (key < hist || key - hist <= tok);
        s[kt][i] = ok ? s[kt][i] * sl2 : -INFINITY;
        tmax = fmaxf(tmax, s[kt][i]);
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = m_run == -INFINITY ? 0.f : exp2f(m_run - m_new);
    float psum = 0.f;
    u32x4 pa[2];  // A operand of P.V for key steps kk = 0, 1
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[i] = s[kt][i] == -INFINITY ? 0.f : exp2f(s[kt][i] - m_new);
        psum += p[i];
      }
      pa[kt >> 1][(kt & 1) * 2 + 0] = pack_bf16x2(p[0], p[1]);
      pa[kt >> 1][(kt & 1) * 2 + 1] = pack_bf16x2(p[2], p[3]);
    }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    l_run = l_run * alpha + psum;
    m_run = m_new;

    // Rescale O: lane holds tokens 4g + i; their alpha lives in lanes 4g + i.
    float al[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * g + i, 64);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) o[dt][i] *= al[i];

    // O += P V over the tile's 64 keys (two 32-key steps).
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const int d = 16 * dt + r;
        u32x4 vb;
        const u32x2 v0 = *(const u32x2 *)(s_v + v_off(d, 8 * kk + g));
        const u32x2 v1 = *(const u32x2 *)(s_v + v_off(d, 8 * kk + 4 + g));
        vb[0] = v0[0];
        vb[1] = v0[1];
        vb[2] = v1[0];
        vb[3] = v1[1];
        o[dt] = mfma16(pa[kk], vb, o[dt]);
      }
    }
    lds_barrier();
  }

  // Epilogue.  Lane holds O[tokens 4g + i][dims 16*dt + r]; the row sums and
  // maxima of those tokens live in lanes 4g + i.
  float lt[4], mt[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    lt[i] = __shfl(l_run, 4 * g + i, 64);
    mt[i] = __shfl(m_run, 4 * g + i, 64);
  }
  if (nsplit == 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tok = q0 + 4 * g + i;
      if (tok >= T) continue;
      const float inv = lt[i] > 0.f ? 1.0f / lt[i] : 0.f;
      uint16_t *op = a.out + ((int64_t)tok * a.Hq + head) * kD + r;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) op[16 * dt] = (uint16_t)(pack_bf16x2(o[dt][i] * inv, 0.f) & 0xffffu);
    }
  } else {
    // Partial state: [split][token][head] {m, l, O[128]} fp32.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tok = q0 + 4 * g + i;
      if (tok >= T) continue;
      float *pp = a.partial + (((int64_t)split * T + tok) * a.Hq + head) * (kD + 2);
      if (r == 0) {
        pp[0] = mt[i];
        pp[1] = lt[i];
      }
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) pp[2 + 16 * dt + r] = o[dt][i];
    }
  }
}

// out[t][h] = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s, splits in order.
__global__ __launch_bounds__(128) void gqa_merge_kernel(GqaArgs a, int nsplit) {
  const int th = blockIdx.x;  // token * Hq + head
  const int d = threadIdx.x;  // 0..127
  const float *base = a.partial + (int64_t)th * (kD + 2);
  const int64_t sstride = (int64_t)a.T * a.Hq * (kD + 2);
  float M = -INFINITY;
  for (int s = 0; s < nsplit; ++s) M = fmaxf(M, base[s * sstride]);
  float num = 0.f, den = 0.f;
  for (int s = 0; s < nsplit; ++s) {
    const float *p = base + s * sstride;
    const float w = p[0] == -INFINITY ? 0.f : exp2f(p[0] - M);
    den += w * p[1];
    num += w * p[2 + d];
  }
  const float v = den > 0.f ? num / den : 0.f;
  a.out[(int64_t)th * kD + d] = (uint16_t)(pack_bf16x2(v, 0.f) & 0xffffu);
}

}  // namespace

int gqa_num_splits(int T, int Hkv, int num_cus) {
  const int blocks = ((T + kQB - 1) / kQB) * Hkv;
  if (blocks <= 0) return 1;
  int s = (2 * num_cus + blocks - 1) / blocks;  // aim for ~2 workgroups per CU
  if (s < 1) s = 1;
  if (s > 16) s = 16;
  return s;
}

size_t gqa_partial_bytes(int T, int Hq, int nsplit) {
  return nsplit > 1 ? (size_t)nsplit * T * Hq * (kD + 2) * sizeof(float) : 0;
}

hipError_t launch_gqa(const GqaArgs &a, int nsplit, hipStream_t s) {
  if (a.T == 0) return hipSuccess;
  const int G = a.Hq / a.Hkv;
  const dim3 grid((a.T + kQB - 1) / kQB, a.Hkv, nsplit);
  switch (G) {
    case 1: hipLaunchKernelGGL(gqa_partial_kernel<1>, grid, dim3(64), 0, s, a); break;
    case 2: hipLaunchKernelGGL(gqa_partial_kernel<2>, grid, dim3(128), 0, s, a); break;
    case 4: hipLaunchKernelGGL(gqa_partial_kernel<4>, grid, dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL(gqa_partial_kernel<8>, grid, dim3(512), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || nsplit == 1) return e;
  hipLaunchKernelGGL(gqa_merge_kernel, dim3(a.T * a.Hq), dim3(kD), 0, s, a, nsplit);
  return hipGetLastError();
}

}  // namespace moe
