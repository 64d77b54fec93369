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

// W4G128 decode: packed word of eight int4 (nibble = q + 8, earliest K in the
// low nibble) -> eight bf16 values bf16_rn(q * scale), packed in pairs.
//
// Nibble n sitting at bits 4p..4p+3 (p = 2, 3, 4: inside the 23-bit mantissa)
// of a word whose other bits are replaced by those of 2^23 (one v_bfi_b32)
// reads as the float 2^23 + n * 16^p.  With per-group constants
// sp = s * 16^-p and cp = -(2^(23-4p) + 8) * s (both exact: power-of-two
// scaling, and an 8-bit-significand scale times an integer of at most 13
// significant bits),
//   fma(2^23 + n * 16^p, sp, cp) = (2^(23-4p) + n) s - (2^(23-4p) + 8) s
//                                = (n - 8) s  exactly (<= 12 significant bits),
// so the only rounding is the final bf16 conversion -- the same as rounding
// float(q) * float(scale).  Nibbles 2..4 decode in place, nibbles 0..1 from
// w << 8 and nibbles 5..7 from w >> 12.
struct W4Scale {
  float sp[3], cp[3];  // p = 2, 3, 4
};

__device__ __forceinline__ W4Scale w4_scale(float s) {
  W4Scale k;
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const int p = i + 2;
    k.sp[i] = s * __uint_as_float((uint32_t)(127 - 4 * p) << 23);  // s * 2^-4p
    k.cp[i] = -s * (float)((1 << (23 - 4 * p)) + 8);
  }
  return k;
}

// (mask & src) | (~mask & other), as gfx950's three-input bit operation
// (truth table 0xca), which issues faster than v_bfi_b32 on MI355X (measured
// ~3.4 vs ~4.5 cycles per wave64 instruction).
__device__ __forceinline__ uint32_t bfi_b32(uint32_t mask, uint32_t src, uint32_t other) {
  uint32_t d;
  asm("v_bitop3_b32 %0, %1, %2, %3 bitop3:0xca" : "=v"(d) : "v"(mask), "v"(src), "v"(other));
  return d;
}

__device__ __forceinline__ u32x4 w4_decode8(uint32_t w, const W4Scale &k) {
  const uint32_t magic = 0x4b000000u;  // 2^23: exponent bits only, empty mantissa
  const uint32_t lo = w << 8, hi = w >> 12;
  auto dq = [&](uint32_t src, int p) {
    return __builtin_fmaf(__uint_as_float(bfi_b32(0xfu << (4 * p), src, magic)), k.sp[p - 2],
                          k.cp[p - 2]);
  };
  u32x4 r;
  r[0] = pack_bf16x2(dq(lo, 2), dq(lo, 3));  // nibbles 0, 1
  r[1] = pack_bf16x2(dq(w, 2), dq(w, 3));    // nibbles 2, 3
  r[2] = pack_bf16x2(dq(w, 4), dq(hi, 2));   // nibbles 4, 5
  r[3] = pack_bf16x2(dq(hi, 3), dq(hi, 4));  // nibbles 6, 7
  return r;
}

}  // namespace moe
