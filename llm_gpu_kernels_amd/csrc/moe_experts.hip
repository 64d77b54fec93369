// Expert stage of the MoE forward on gfx950 (CDNA4).
//
// gate/up + SwiGLU (reference: _dynamic_grouped_gate_up_swiglu,
// moe_fused.py:18-73; cuda_gate_up_bf16, cuda_gate_up.cu:53-131; W4:
// cuda_gate_up_w4_sync, cuda_w4_gate_up.cu:46-100), down projection
// (_dynamic_grouped, moe.py:69-95) and the slot-ordered weighted combine
// (_combine, moe.py:109-121).
//
// Design (weight streaming).  A task is one expert and up to 16*MT of its
// grouped rows.  The workgroup gathers those token rows of x straight from
// the route list into LDS, already in the MFMA B-operand order, so no
// permuted copy of x is materialised.  Each of its 8 waves then streams its
// own 16-row blocks of the expert's weights from HBM directly into MFMA
// A-operand registers (one 128-bit load per lane per 16x16x32 MFMA) and
// multiplies them against every 16-token group held in LDS.  Weights are the
// only large operand and each weight byte is read once per task, which is the
// HBM-bound regime of every BASELINE configuration.
//
// Rounding follows the reference's M4 contract: gate and up accumulate in
// fp32 and are rounded to bf16, SwiGLU runs in fp32 and is stored as bf16;
// the down projection is rounded to bf16; the combine sums w * value in
// fp32 in slot order with unfused multiply/add and rounds once to bf16.
#include "common.h"
#include "moe_internal.h"

namespace moe {

namespace {

constexpr int kThreads = 512;           // 8 waves per workgroup
constexpr int kWaves = kThreads / kWave;
constexpr int kGateUpCols = kWaves * 16;  // intermediate columns per workgroup
constexpr int kDownCols = kWaves * 32;    // hidden columns per workgroup
constexpr int kUnroll = 4;                // k-steps per pipeline stage

// Gather `rows` token rows (row j -> token row_route[row0+j] / K, or grouped
// row row0+j itself when `direct`) of a bf16 [*, width] matrix into LDS in
// B-operand order: [mt][k-step][lane] 16-byte chunks, lane = 16*(k%32/8) + j%16.
template <int MT>
__device__ __forceinline__ void gather_rows(u32x4 *__restrict__ lds, const uint16_t *__restrict__ src,
                                            int width, int row0, int rows,
                                            const int32_t *__restrict__ row_route, int K,
                                            bool direct) {
  const int cpr = width >> 3;      // 16-byte chunks per row
  const int steps = width >> 5;    // k-steps
  for (int i = threadIdx.x; i < 16 * MT * cpr; i += kThreads) {
    const int j = i / cpr;
    const int c = i - j * cpr;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (j < rows) {
      const int srow = direct ? row0 + j : row_route[row0 + j] / K;
      v = *(const u32x4 *)(src + (size_t)srow * width + c * 8);
    }
    lds[((j >> 4) * steps + (c >> 2)) * kWave + (c & 3) * 16 + (j & 15)] = v;
  }
}

template <int MT, bool W4>
__global__ __launch_bounds__(kThreads) void gate_up_kernel(ExpertArgs a) {
  extern __shared__ u32x4 s_act[];
  const int task = blockIdx.x;
  if (task >= *a.num_tasks) return;
  const int4 tk = a.tasks[task];
  const int e = tk.x, row0 = tk.y, rows = tk.z;
  const int H = a.H, I = a.I;
  const int S = H >> 5;

  gather_rows<MT>(s_act, a.x, H, row0, rows, a.row_route, a.K, false);
  __syncthreads();

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & (kWave - 1);
  const int n0 = blockIdx.y * kGateUpCols + wave * 16;
  if (n0 >= I) return;
  const int r = lane & 15, g = lane >> 4;

  f32x4 accg[MT], accu[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) accg[m] = accu[m] = f32x4{0.f, 0.f, 0.f, 0.f};

  if constexpr (!W4) {
    const uint16_t *pg = a.gate_up + ((size_t)e * 2 * I + n0 + r) * H + g * 8;
    const uint16_t *pu = pg + (size_t)I * H;
    u32x4 bg[kUnroll], bu[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      bg[u] = *(const u32x4 *)(pg + u * 32);
      bu[u] = *(const u32x4 *)(pu + u * 32);
    }
    for (int s0 = 0; s0 < S; s0 += kUnroll) {
      // Prefetch the next stage; the last stage re-reads itself (in cache).
      const int sn = (s0 + kUnroll < S) ? s0 + kUnroll : s0;
      u32x4 ng[kUnroll], nu[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        ng[u] = *(const u32x4 *)(pg + (sn + u) * 32);
        nu[u] = *(const u32x4 *)(pu + (sn + u) * 32);
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          const u32x4 b = s_act[(m * S + s0 + u) * kWave + lane];
          accg[m] = mfma16(bg[u], b, accg[m]);
          accu[m] = mfma16(bu[u], b, accu[m]);
        }
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        bg[u] = ng[u];
        bu[u] = nu[u];
      }
    }
  } else {
    // Tiled W4: [E][2I/16][H/128][64][4] words, [E][2I/16][H/128][16] scales.
    const int G = H >> 7;
    const size_t rb_g = (size_t)e * (2 * I / 16) + n0 / 16;
    const size_t rb_u = rb_g + I / 16;
    const u32x4 *wg = (const u32x4 *)a.w4_words + rb_g * G * kWave + lane;
    const u32x4 *wu = (const u32x4 *)a.w4_words + rb_u * G * kWave + lane;
    const uint16_t *sg = a.w4_scales + rb_g * G * 16 + r;
    const uint16_t *su = a.w4_scales + rb_u * G * 16 + r;
    u32x4 cg = wg[0], cu = wu[0];
    uint32_t csg = sg[0], csu = su[0];
    for (int grp = 0; grp < G; ++grp) {
      const int gn = grp + 1 < G ? grp + 1 : grp;
      const u32x4 ng = wg[(size_t)gn * kWave], nu = wu[(size_t)gn * kWave];
      const uint32_t nsg = sg[gn * 16], nsu = su[gn * 16];
      const float fsg = bf16_bits_to_f32(csg), fsu = bf16_bits_to_f32(csu);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u32x4 ag = w4_decode8(cg[j], fsg, -24.f * fsg);
        const u32x4 au = w4_decode8(cu[j], fsu, -24.f * fsu);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          const u32x4 b = s_act[(m * S + grp * 4 + j) * kWave + lane];
          accg[m] = mfma16(ag, b, accg[m]);
          accu[m] = mfma16(au, b, accu[m]);
        }
      }
      cg = ng;
      cu = nu;
      csg = nsg;
      csu = nsu;
    }
  }

  // Epilogue: lane holds rows n0 + 4g + i of token (grouped row) m*16 + r.
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const int j = m * 16 + r;
    if (j < rows) {
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float gt = bf16_round(accg[m][i]);
        const float up = bf16_round(accu[m][i]);
        v[i] = gt / (1.0f + expf(-gt)) * up;
      }
      u32x2 packed;
      packed[0] = pack_bf16x2(v[0], v[1]);
      packed[1] = pack_bf16x2(v[2], v[3]);
      *(u32x2 *)(a.act + (size_t)(row0 + j) * I + n0 + 4 * g) = packed;
    }
  }
}

template <int MT>
__global__ __launch_bounds__(kThreads) void down_kernel(ExpertArgs a) {
  extern __shared__ u32x4 s_act[];
  const int task = blockIdx.x;
  if (task >= *a.num_tasks) return;
  const int4 tk = a.tasks[task];
  const int e = tk.x, row0 = tk.y, rows = tk.z;
  const int H = a.H, I = a.I;
  const int S = I >> 5;

  gather_rows<MT>(s_act, a.act, I, row0, rows, nullptr, 1, true);
  __syncthreads();

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & (kWave - 1);
  const int n0 = blockIdx.y * kDownCols + wave * 32;
  if (n0 >= H) return;
  const int r = lane & 15, g = lane >> 4;

  f32x4 acc0[MT], acc1[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc0[m] = acc1[m] = f32x4{0.f, 0.f, 0.f, 0.f};

  const uint16_t *p0 = a.down + ((size_t)e * H + n0 + r) * I + g * 8;
  const uint16_t *p1 = p0 + (size_t)16 * I;
  u32x4 b0[kUnroll], b1[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    b0[u] = *(const u32x4 *)(p0 + u * 32);
    b1[u] = *(const u32x4 *)(p1 + u * 32);
  }
  for (int s0 = 0; s0 < S; s0 += kUnroll) {
    const int sn = (s0 + kUnroll < S) ? s0 + kUnroll : s0;
    u32x4 n0v[kUnroll], n1v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      n0v[u] = *(const u32x4 *)(p0 + (sn + u) * 32);
      n1v[u] = *(const u32x4 *)(p1 + (sn + u) * 32);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const u32x4 b = s_act[(m * S + s0 + u) * kWave + lane];
        acc0[m] = mfma16(b0[u], b, acc0[m]);
        acc1[m] = mfma16(b1[u], b, acc1[m]);
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      b0[u] = n0v[u];
      b1[u] = n1v[u];
    }
  }

#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const int j = m * 16 + r;
    if (j < rows) {
      const int q = a.row_route[row0 + j];
      uint16_t *dst = a.routed + (size_t)q * H + n0 + 4 * g;
      u32x2 v0, v1;
      v0[0] = pack_bf16x2(acc0[m][0], acc0[m][1]);
      v0[1] = pack_bf16x2(acc0[m][2], acc0[m][3]);
      v1[0] = pack_bf16x2(acc1[m][0], acc1[m][1]);
      v1[1] = pack_bf16x2(acc1[m][2], acc1[m][3]);
      *(u32x2 *)dst = v0;
      *(u32x2 *)(dst + 16) = v1;
    }
  }
}

// out[t] = bf16(sum_s fp32(routed[t*K+s]) * w[t,s]), slot order, no FMA.
__global__ __launch_bounds__(256) void combine_kernel(ExpertArgs a) {
  const int t = blockIdx.x;
  const int h = (blockIdx.y * 256 + threadIdx.x) * 8;
  if (h >= a.H) return;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;
  for (int s = 0; s < a.K; ++s) {
    const int q = t * a.K + s;
    if (a.map[q] < 0) continue;
    const float w = a.weights[q];
    const u32x4 v = *(const u32x4 *)(a.routed + (size_t)q * a.H + h);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = bf16_bits_to_f32(v[i] & 0xffffu);
      const float hi = bf16_bits_to_f32(v[i] >> 16);
      acc[2 * i] = __fadd_rn(acc[2 * i], __fmul_rn(lo, w));
      acc[2 * i + 1] = __fadd_rn(acc[2 * i + 1], __fmul_rn(hi, w));
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
  const float s = bf16_bits_to_f32(scales_t[ug * 16 + r]);
  uint16_t *row = out + ((size_t)e * N + rb * 16 + r) * K + grp * 128 + g * 8;
#pragma unroll
  for (int j = 0; j < 4; ++j) *(u32x4 *)(row + 32 * j) = w4_decode8(w[j], s, -24.f * s);
}

// Opt every MFMA kernel into the full 160 KiB of LDS once per process (the
// attribute belongs to the function, not to a launch).
template <typename Kern>
hipError_t set_lds(Kern k, size_t) {
  static hipError_t once = hipFuncSetAttribute(
      (const void *)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxLds);
  return once;
}

}  // namespace

size_t gate_up_lds_bytes(int H, int token_block) { return (size_t)token_block * H * 2; }
size_t down_lds_bytes(int I, int token_block) { return (size_t)token_block * I * 2; }

hipError_t launch_gate_up(const ExpertArgs &a, int task_capacity, int token_block, bool w4,
                          bool fast, hipStream_t s) {
  if (!fast) {
    const dim3 grid(task_capacity, (token_block * a.I + 255) / 256);
    hipLaunchKernelGGL(gate_up_generic_kernel, grid, dim3(256), 0, s, a, token_block);
    return hipGetLastError();
  }
  const dim3 grid(task_capacity, (a.I + kGateUpCols - 1) / kGateUpCols);
  const size_t lds = gate_up_lds_bytes(a.H, token_block);
  hipError_t err;
#define MOE_LAUNCH_GU(MT, W)                                                        \
  do {                                                                              \
    if ((err = set_lds(gate_up_kernel<MT, W>, lds)) != hipSuccess) return err;      \
    hipLaunchKernelGGL((gate_up_kernel<MT, W>), grid, dim3(kThreads), lds, s, a);   \
  } while (0)
  if (token_block == 16) {
    if (w4) MOE_LAUNCH_GU(1, true); else MOE_LAUNCH_GU(1, false);
  } else {
    if (w4) MOE_LAUNCH_GU(2, true); else MOE_LAUNCH_GU(2, false);
  }
#undef MOE_LAUNCH_GU
  return hipGetLastError();
}

hipError_t launch_down(const ExpertArgs &a, int task_capacity, int token_block, bool fast,
                       hipStream_t s) {
  if (!fast) {
    const dim3 grid(task_capacity, (token_block * a.H + 255) / 256);
    hipLaunchKernelGGL(down_generic_kernel, grid, dim3(256), 0, s, a, token_block);
    return hipGetLastError();
  }
  const dim3 grid(task_capacity, (a.H + kDownCols - 1) / kDownCols);
  const size_t lds = down_lds_bytes(a.I, token_block);
  hipError_t err;
  if (token_block == 16) {
    if ((err = set_lds(down_kernel<1>, lds)) != hipSuccess) return err;
    hipLaunchKernelGGL(down_kernel<1>, grid, dim3(kThreads), lds, s, a);
  } else {
    if ((err = set_lds(down_kernel<2>, lds)) != hipSuccess) return err;
    hipLaunchKernelGGL(down_kernel<2>, grid, dim3(kThreads), lds, s, a);
  }
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

hipError_t launch_w4_dequantize(const uint32_t *words_t, const uint16_t *scales_t, int E, int N,
                                int K, uint16_t *out, hipStream_t s) {
  const size_t total = (size_t)E * (N / 16) * (K / 128) * kWave;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(w4_dequant_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                     words_t, scales_t, E, N, K, out);
  return hipGetLastError();
}

}  // namespace moe
