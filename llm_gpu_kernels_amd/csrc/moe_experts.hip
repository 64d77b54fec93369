// Expert stage helpers of the MoE forward on gfx950 (CDNA4): the weighted
// combine, generic (any-shape) expert kernels and the W4 expansion kernel.
// The MFMA streaming GEMMs live in moe_stream.hip.
//
// gate/up + SwiGLU (reference: _dynamic_grouped_gate_up_swiglu,
// moe_fused.py:18-73; cuda_gate_up_bf16, cuda_gate_up.cu:53-131; W4:
// cuda_gate_up_w4_sync, cuda_w4_gate_up.cu:46-100), down projection
// (_dynamic_grouped, moe.py:69-95) and the slot-ordered weighted combine
// (_combine, moe.py:109-121).
//
// Rounding follows the reference's M4 contract: gate and up accumulate in
// fp32 and are rounded to bf16, SwiGLU runs in fp32 and is stored as bf16;
// the down projection is rounded to bf16; the combine sums w * value in
// fp32 in slot order with unfused multiply/add and rounds once to bf16.
#include "common.h"
#include "moe_internal.h"

namespace moe {

namespace {

// out[t] = bf16(sum_s fp32(routed[t*K+s]) * w[t,s]), slot order, no FMA.
// Slots are taken eight at a time with every load of a chunk issued before
// the first add, so a token costs one memory round trip per eight slots.
// The combine is the last launch of every forward: it also zeroes the work
// counters of the streaming GEMMs (their own last workgroups already do), so
// a workspace whose counters were left nonzero -- an aborted forward, a reused
// arena -- is clean again from the next forward on.
__device__ __forceinline__ void clear_counters(const ExpertArgs &a) {
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x < 4) a.counters[threadIdx.x] = 0;
}

__global__ __launch_bounds__(256) void combine_kernel(ExpertArgs a) {
  clear_counters(a);
  const int t = blockIdx.x;
  const int h = (blockIdx.y * 256 + threadIdx.x) * 8;
  if (h >= a.H) return;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;
  for (int s0 = 0; s0 < a.K; s0 += 8) {
    int mp[8];
    float wt[8];
    u32x4 v[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int q = t * a.K + s0 + s;
      const bool in = s0 + s < a.K;
      mp[s] = in ? a.map[q] : -1;
      wt[s] = in ? a.weights[q] : 0.f;
      // Every route's row is read (in bounds); a dropped route's row is
      // never added, whatever it holds.
      v[s] = *(const u32x4 *)(a.routed + (size_t)(in ? q : t * a.K) * a.H + h);
    }
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      if (mp[s] < 0) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float lo = bf16_bits_to_f32(v[s][i] & 0xffffu);
        const float hi = bf16_bits_to_f32(v[s][i] >> 16);
        acc[2 * i] = __fadd_rn(acc[2 * i], __fmul_rn(lo, wt[s]));
        acc[2 * i + 1] = __fadd_rn(acc[2 * i + 1], __fmul_rn(hi, wt[s]));
      }
    }
  }
  u32x4 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = pack_bf16x2(acc[2 * i], acc[2 * i + 1]);
  *(u32x4 *)(a.out + (size_t)t * a.H + h) = o;
}

// ---- generic kernels for shapes the MFMA path does not take ---------------
__device__ __forceinline__ float ld_bf16(const uint16_t *p) { return bf16_bits_to_f32(*p); }

__global__ __launch_bounds__(256) void gate_up_generic_kernel(ExpertArgs a, int token_block) {
  const int task = blockIdx.x;
  if (task >= *a.num_tasks) return;
  const int4 tk = a.tasks[task];
  const int idx = blockIdx.y * 256 + threadIdx.x;
  const int j = idx / a.I, n = idx - j * a.I;
  if (j >= tk.z || j >= token_block) return;
  const int p = tk.y + j;
  const int t = a.row_route[p] / a.K;
  const uint16_t *xr = a.x + (size_t)t * a.H;
  const uint16_t *wg = a.gate_up + ((size_t)tk.x * 2 * a.I + n) * a.H;
  const uint16_t *wu = wg + (size_t)a.I * a.H;
  float sg = 0.f, su = 0.f;
  for (int k = 0; k < a.H; ++k) {
    const float xv = ld_bf16(xr + k);
    sg = __builtin_fmaf(xv, ld_bf16(wg + k), sg);
    su = __builtin_fmaf(xv, ld_bf16(wu + k), su);
  }
  const float gt = bf16_round(sg), up = bf16_round(su);
  a.act[(size_t)p * a.I + n] = (uint16_t)f32_to_bf16_bits(gt / (1.0f + expf(-gt)) * up);
}

__global__ __launch_bounds__(256) void down_generic_kernel(ExpertArgs a, int token_block) {
  const int task = blockIdx.x;
  if (task >= *a.num_tasks) return;
  const int4 tk = a.tasks[task];
  const int idx = blockIdx.y * 256 + threadIdx.x;
  const int j = idx / a.H, n = idx - j * a.H;
  if (j >= tk.z || j >= token_block) return;
  const int p = tk.y + j;
  const uint16_t *ar = a.act + (size_t)p * a.I;
  const uint16_t *wd = a.down + ((size_t)tk.x * a.H + n) * a.I;
  float s = 0.f;
  for (int k = 0; k < a.I; ++k) s = __builtin_fmaf(ld_bf16(ar + k), ld_bf16(wd + k), s);
  a.routed[(size_t)a.row_route[p] * a.H + n] = (uint16_t)f32_to_bf16_bits(s);
}

__global__ __launch_bounds__(256) void combine_generic_kernel(ExpertArgs a) {
  clear_counters(a);
  const int t = blockIdx.x;
  const int h = blockIdx.y * 256 + threadIdx.x;
  if (h >= a.H) return;
  float acc = 0.f;
  for (int s = 0; s < a.K; ++s) {
    const int q = t * a.K + s;
    if (a.map[q] < 0) continue;
    acc = __fadd_rn(acc, __fmul_rn(ld_bf16(a.routed + (size_t)q * a.H + h), a.weights[q]));
  }
  a.out[(size_t)t * a.H + h] = (uint16_t)f32_to_bf16_bits(acc);
}

// Tiled W4 -> dense bf16 [E, N, K] with the GEMM's decode (w4_decode8).
__global__ __launch_bounds__(256) void w4_dequant_kernel(const uint32_t *__restrict__ words_t,
                                                         const uint16_t *__restrict__ scales_t,
                                                         int E, int N, int K,
                                                         uint16_t *__restrict__ out) {
  // One thread per (row block, group, lane) 16-byte chunk of words.
  const int G = K >> 7;
  const size_t total = (size_t)E * (N / 16) * G * kWave;
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int lane = (int)(i % kWave);
  const size_t ug = i / kWave;  // (e * N/16 + rb) * G + grp
  const int grp = (int)(ug % G);
  const size_t erb = ug / G;
  const int e = (int)(erb / (N / 16));
  const int rb = (int)(erb % (N / 16));
  const int r = lane & 15, g = lane >> 4;
  const u32x4 w = ((const u32x4 *)words_t)[i];
  const W4Scale ks = w4_scale(bf16_bits_to_f32(scales_t[ug * 16 + r]));
  uint16_t *row = out + ((size_t)e * N + rb * 16 + r) * K + grp * 128 + g * 8;
#pragma unroll
  for (int j = 0; j < 4; ++j) *(u32x4 *)(row + 32 * j) = w4_decode8(w[j], ks);
}

// bf16 streaming GEMMs through LDS (moe_dma.hip) rather than straight into
// registers (moe_stream.hip), where the shape allows.
constexpr bool kDmaStreaming = true;
constexpr bool kDmaDown = true;

}  // namespace

hipError_t launch_gate_up(const ExpertArgs &a, int task_capacity, int token_block, bool w4,
                          int path, int num_cus, hipStream_t s) {
  // W4 with several rows per expert, and every 64-row task: decode each weight
  // fragment once for up to 64 token rows (one unit per wave).  With about one
  // row per expert the split-K streaming kernel overlaps the decode better, and
  // with the folded decode it is faster for 16-row tasks too (T = 193: gate/up
  // 49 vs 61 us).
  const bool wave_ok = w4 && wave_w4_shape_ok(a.H, a.I, token_block);
  if (wave_ok && path != kGeneric && (token_block == 64 || ((long long)a.R >= 4LL * a.E && !a.w4_fold)))
    return launch_wave_w4_gate_up(a, task_capacity, token_block, s);
  if (path == kTile) return w4 ? hipErrorInvalidValue : launch_tile_gate_up(a, task_capacity, num_cus, s);
  if (path == kStream) {
    if (!w4 && kDmaStreaming && dma_shape_ok(a.H, a.I, token_block))
      return launch_dma_gate_up(a, token_block, num_cus, s);
    return launch_stream_gate_up(a, task_capacity, token_block, w4, num_cus, s);
  }
  // Shapes the tuned kernels do not take: the W4 wave kernel where its K-chunks
  // fit, else the run-time-K MFMA kernel, else (bf16, H or I not a multiple of
  // 32) the scalar one.
  if (wave_ok) return launch_wave_w4_gate_up(a, task_capacity, token_block, s);
  if (path == kGeneric && flex_shape_ok(a.H, a.I, w4))
    return launch_flex_gate_up(a, task_capacity, token_block, w4, s);
  if (w4) return hipErrorInvalidValue;
  const dim3 grid(task_capacity, (token_block * a.I + 255) / 256);
  hipLaunchKernelGGL(gate_up_generic_kernel, grid, dim3(256), 0, s, a, token_block);
  return hipGetLastError();
}

hipError_t launch_down(const ExpertArgs &a, int task_capacity, int token_block, int path,
                       int num_cus, hipStream_t s) {
  if (path == kTile) return launch_tile_down(a, task_capacity, num_cus, s);
  if (path == kStream) {
    if (kDmaStreaming && kDmaDown && dma_shape_ok(a.H, a.I, token_block)) return launch_dma_down(a, token_block, num_cus, s);
    return launch_stream_down(a, task_capacity, token_block, num_cus, s);
  }
  if (path == kGeneric && flex_shape_ok(a.H, a.I, false))
    return launch_flex_down(a, task_capacity, token_block, s);
  const dim3 grid(task_capacity, (token_block * a.H + 255) / 256);
  hipLaunchKernelGGL(down_generic_kernel, grid, dim3(256), 0, s, a, token_block);
  return hipGetLastError();
}

hipError_t launch_combine(const ExpertArgs &a, hipStream_t s) {
  if (a.H % 8 == 0 && ((uintptr_t)a.out % 16) == 0) {
    const dim3 grid(a.T, (a.H / 8 + 255) / 256);
    hipLaunchKernelGGL(combine_kernel, grid, dim3(256), 0, s, a);
  } else {
    const dim3 grid(a.T, (a.H + 255) / 256);
    hipLaunchKernelGGL(combine_generic_kernel, grid, dim3(256), 0, s, a);
  }
  return hipGetLastError();
}

namespace {
__global__ void reset_counters_kernel(int32_t *c, uint32_t *status, int32_t *partials, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < 4) c[i] = 0;
  if (status && i >= 4 && i < 6) status[i - 4] = 0;
  if (i < n) partials[i] = 0;
}
}  // namespace

hipError_t launch_reset_counters(int32_t *counters, uint32_t *status, int32_t *partials,
                                 int n_partials, hipStream_t s) {
  const int blocks = n_partials > 64 ? (n_partials + 255) / 256 : 1;
  hipLaunchKernelGGL(reset_counters_kernel, dim3(blocks), dim3(256), 0, s, counters, status,
                     partials, n_partials);
  return hipGetLastError();
}

hipError_t launch_w4_dequantize(const uint32_t *words_t, const uint16_t *scales_t, int E, int N,
                                int K, uint16_t *out, hipStream_t s) {
  const size_t total = (size_t)E * (N / 16) * (K / 128) * kWave;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(w4_dequant_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                     words_t, scales_t, E, N, K, out);
  return hipGetLastError();
}

}  // namespace moe
