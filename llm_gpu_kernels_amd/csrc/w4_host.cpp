// Host-side W4G128 weight preparation (offline; never inside a forward).
//
// moe_w4_quantize follows quantize_gate_up (src/llm_gpu_kernels/
// moe_weight_quant.py:55-105) for any [E, N, K] with K % 128 == 0:
//   scale = bf16_rn(max|w| / 7) per 128-K group (1 when the group is all
//   zero); q = clamp(round_half_even(w / scale), -7, 7) in fp32; nibble q + 8,
//   word j holds K = 8j..8j+7 with the earliest K in the low nibble.
// moe_w4_tile rearranges that v1 format into the layout the gfx950 kernels
// stream: one 1 KiB block per (16 rows, 128 K) with lane l = 16*g + r holding
// row r and K chunks 32*j + 8*g (j = 0..3), i.e. v1 words 16*grp + 4*j + g.
#include <math.h>
#include <string.h>

#include <cfenv>

#include "../../include/moe_mi355x.h"

namespace {

float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

}  // namespace

extern "C" {

int moe_w4_quantize(const uint16_t *weight, int32_t E, int32_t N, int32_t K, uint32_t *words,
                    uint16_t *scales) {
  if (!weight || !words || !scales || E < 1 || N < 1 || K < 128 || K % 128) return MOE_EINVAL;
  const int G = K / 128;
  std::fesetround(FE_TONEAREST);
  for (long long row = 0; row < (long long)E * N; ++row) {
    const uint16_t *w = weight + row * K;
    for (int grp = 0; grp < G; ++grp) {
      float mx = 0.f;
      for (int k = 0; k < 128; ++k) {
        const float v = bf16_to_f32(w[grp * 128 + k]);
        if (!isfinite(v)) return MOE_EINVAL;
        mx = fmaxf(mx, fabsf(v));
      }
      const uint16_t sb = f32_to_bf16(mx == 0.f ? 1.f : mx / 7.f);
      const float s = bf16_to_f32(sb);
      if (!(s > 0.f) || !isfinite(s)) return MOE_EINVAL;
      scales[row * G + grp] = sb;
      for (int j = 0; j < 16; ++j) {
        uint32_t word = 0;
        for (int i = 0; i < 8; ++i) {
          float q = nearbyintf(bf16_to_f32(w[grp * 128 + j * 8 + i]) / s);
          q = fminf(7.f, fmaxf(-7.f, q));
          word |= (uint32_t)((int)q + 8) << (4 * i);
        }
        words[row * (K / 8) + grp * 16 + j] = word;
      }
    }
  }
  return MOE_OK;
}

size_t moe_w4_tiled_words_bytes(int32_t E, int32_t N, int32_t K) {
  return (size_t)E * N * (K / 8) * 4;
}

size_t moe_w4_tiled_scales_bytes(int32_t E, int32_t N, int32_t K) {
  return (size_t)E * N * (K / 128) * 2;
}

int moe_w4_tile(const uint32_t *words, const uint16_t *scales, int32_t E, int32_t N, int32_t K,
                uint32_t *words_t, uint16_t *scales_t) {
  if (!words || !scales || !words_t || !scales_t || E < 1 || N < 16 || N % 16 || K < 128 ||
      K % 128)
    return MOE_EINVAL;
  const int G = K / 128, KW = K / 8;
  const int RB = N / 16;
  for (int e = 0; e < E; ++e)
    for (int rb = 0; rb < RB; ++rb)
      for (int grp = 0; grp < G; ++grp) {
        const size_t unit = ((size_t)e * RB + rb) * G + grp;
        for (int lane = 0; lane < 64; ++lane) {
          const int r = lane & 15, g = lane >> 4;
          const size_t src_row = ((size_t)e * N + rb * 16 + r) * KW;
          for (int j = 0; j < 4; ++j)
            words_t[(unit * 64 + lane) * 4 + j] = words[src_row + grp * 16 + 4 * j + g];
        }
        for (int r = 0; r < 16; ++r)
          scales_t[unit * 16 + r] = scales[((size_t)e * N + rb * 16 + r) * G + grp];
      }
  return MOE_OK;
}

}  // extern "C"
