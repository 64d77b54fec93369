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

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two floats -> packed bf16 with gfx950's v_cvt_pk_bf16_f32 (IEEE
// round-to-nearest-even, identical to f32_to_bf16_bits for every non-NaN).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ float bf16_round(float f) {
  return bf16_bits_to_f32(pack_bf16x2(f, 0.f) & 0xffffu);
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) {
  return __builtin_bit_cast(bf16x8, v);
}

// MFMA 16x16x32 bf16 -> fp32 (CDNA4).  Lane l supplies A[l%16][8*(l/16)..+8]
// and B[8*(l/16)..+8][l%16]; it receives C[4*(l/16)+r][l%16], r = 0..3.
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
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

// Loads from a wave-uniform base plus a 32-bit per-lane byte offset, as
// buffer loads: the base goes into a scalar resource and no lane computes a
// 64-bit address.  `base` must be the same in every lane of the wave.
__device__ __forceinline__ u32x4 load_u128_at(const void *base, uint32_t off) {
  const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, 0x7fffffff, 0x00020000);
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
}
__device__ __forceinline__ uint32_t load_u16_at(const void *base, uint32_t off) {
  const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, 0x7fffffff, 0x00020000);
  return __builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0);
}

// W4G128 decode: packed word of eight int4 (nibble = q + 8, earliest K in the
// low nibble) -> eight bf16 values bf16_rn(q * scale), packed in pairs.
//
// One bit insert places two nibbles, one per 16-bit half, into the mantissa
// of an fp16 number: nibbles at bits 0..3 of a half under the exponent of
// 1024 (0x6400, ulp 1) read as 1024 + n, nibbles at bits 4..7 under the
// exponent of 64 (0x5400, ulp 1/16) as 64 + n.  gfx950's v_fma_mix_f32 takes
// either half as an fp16 operand of a single-rounding fp32 FMA, so with
// per-group constants (exact: an 8-bit-significand scale times
// 1032 = 2^10 + 2^3 or 72 = 2^6 + 2^3)
//   fma(1024 + n, s, -1032 s) = fma(64 + n, s, -72 s) = (n - 8) s
// exactly (<= 12 significant bits), and the only rounding is the final bf16
// conversion -- the same as rounding float(q) * float(scale).  Per eight
// weights: one shift, four bit inserts, eight FMAs, four bf16 packs.  (q = 0
// decodes as +0 whatever the scale's sign; the quantizer's scales are >= 0.)
struct W4Scale {
  float s, c0, c1;
};

__device__ __forceinline__ W4Scale w4_scale(float s) {
  return W4Scale{s, -1032.0f * s, -72.0f * s};
}

// (mask & src) | (~mask & other), as gfx950's three-input bit operation
// (truth table 0xca), which issues faster than v_bfi_b32 on MI355X (measured
// ~3.4 vs ~4.5 cycles per wave64 instruction).
__device__ __forceinline__ uint32_t bfi_b32(uint32_t mask, uint32_t src, uint32_t other) {
  uint32_t d;
  asm("v_bitop3_b32 %0, %1, %2, %3 bitop3:0xca" : "=v"(d) : "v"(mask), "v"(src), "v"(other));
  return d;
}

// fma(float(fp16 half HI of h2), s, c): one v_fma_mix_f32 (the compiler
// folds the half select and the fp16 -> fp32 conversion into the FMA).
template <int HI>
__device__ __forceinline__ float fma_mix(uint32_t h2, float s, float c) {
  const _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)(HI ? h2 >> 16 : h2 & 0xffffu));
  return __builtin_fmaf((float)h, s, c);
}

__device__ __forceinline__ u32x4 w4_decode8(uint32_t w, const W4Scale &k) {
  const uint32_t m0 = 0x64006400u, m1 = 0x54005400u;  // fp16 1024 / 64 in both halves
  const uint32_t w8 = w >> 8;
  const uint32_t a = bfi_b32(0x000f000fu, w, m0);   // 1024 + n0 | 1024 + n4
  const uint32_t b = bfi_b32(0x00f000f0u, w, m1);   //   64 + n1 |   64 + n5
  const uint32_t c = bfi_b32(0x000f000fu, w8, m0);  // n2 | n6
  const uint32_t d = bfi_b32(0x00f000f0u, w8, m1);  // n3 | n7
  u32x4 r;
  r[0] = pack_bf16x2(fma_mix<0>(a, k.s, k.c0), fma_mix<0>(b, k.s, k.c1));
  r[1] = pack_bf16x2(fma_mix<0>(c, k.s, k.c0), fma_mix<0>(d, k.s, k.c1));
  r[2] = pack_bf16x2(fma_mix<1>(a, k.s, k.c0), fma_mix<1>(b, k.s, k.c1));
  r[3] = pack_bf16x2(fma_mix<1>(c, k.s, k.c0), fma_mix<1>(d, k.s, k.c1));
  return r;
}

// W4 "folded" decode for MFMA operands: one AND-OR per register places the
// nibbles of a word's two 16-bit halves (k and k + 4 of the eight K values)
// under the bf16 exponent of 128, i.e. the exact values 128 + n = 136 + q.
// Register j holds (k_j, k_{j+4}), so the B operand must carry its K values
// in the same order (w4_fold_b); the group scale and the -136 offset are
// applied to the fp32 sum of the group's MFMAs.  Seven VALU instructions per
// eight weights.
__device__ __forceinline__ u32x4 w4_fold8(uint32_t w) {
  const uint32_t m = 0x000f000fu, e = 0x43004300u;
  u32x4 r;
  r[0] = (w & m) | e;
  r[1] = ((w >> 4) & m) | e;
  r[2] = ((w >> 8) & m) | e;
  r[3] = ((w >> 12) & m) | e;
  return r;
}
// Natural-order bf16 x (x0 x1 | x2 x3 | x4 x5 | x6 x7) -> (x0 x4 | x1 x5 | x2 x6 | x3 x7).
__device__ __forceinline__ u32x4 w4_fold_b(u32x4 x) {
  u32x4 r;
  r[0] = __builtin_amdgcn_perm(x[2], x[0], 0x05040100u);
  r[1] = __builtin_amdgcn_perm(x[2], x[0], 0x07060302u);
  r[2] = __builtin_amdgcn_perm(x[3], x[1], 0x05040100u);
  r[3] = __builtin_amdgcn_perm(x[3], x[1], 0x07060302u);
  return r;
}
__device__ __forceinline__ float bf16x8_sum(u32x4 x) {
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) t += bf16_bits_to_f32(x[i] & 0xffffu) + bf16_bits_to_f32(x[i] >> 16);
  return t;
}

}  // namespace moe
