// Shared device helpers for the gfx950 MoE / attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

// IEEE round-to-nearest-even float -> bf16 bits; every NaN becomes the
// canonical 0x7fc0 (the bits torch's conversion gives).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

__device__ __forceinline__ float bf16_round(float f) {
  return bf16_bits_to_f32(f32_to_bf16_bits(f));
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) {
  return __builtin_bit_cast(bf16x8, v);
}

// MFMA 16x16x32 bf16 -> fp32 (CDNA4).  Lane l supplies A[l%16][8*(l/16)..+8]
// and B[8*(l/16)..+8][l%16]; it receives C[4*(l/16)+r][l%16], r = 0..3.
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ uint64_t lanemask_lt() {
  const int lane = threadIdx.x & (kWave - 1);
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// Decode one packed word of eight int4 values (nibble = q + 8, earliest K in
// the low nibble) into eight bf16 values bf16_rn(q * scale), packed in pairs.
// 16 + n is built exactly as a float (n in mantissa bits 22..19), and
// fma(16 + n, s, -24 s) = (n - 8) s is exact (<= 13 significant bits), so the
// only rounding is the final bf16 conversion -- identical to rounding the
// exact product float(q) * float(scale).
__device__ __forceinline__ u32x4 w4_decode8(uint32_t w, float s, float neg24s) {
  float f[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t nib = (w >> (4 * i)) & 0xfu;
    f[i] = __builtin_fmaf(__uint_as_float(0x41800000u | (nib << 19)), s, neg24s);
  }
  u32x4 r;
  r[0] = pack_bf16x2(f[0], f[1]);
  r[1] = pack_bf16x2(f[2], f[3]);
  r[2] = pack_bf16x2(f[4], f[5]);
  r[3] = pack_bf16x2(f[6], f[7]);
  return r;
}

}  // namespace moe
