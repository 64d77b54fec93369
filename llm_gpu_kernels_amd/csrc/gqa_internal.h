// Internal launch interface of the segmented-KV GQA attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

constexpr int kGqaMaxSegments = 4;

struct GqaArgs {
  const uint16_t *q;                     // [T, Hq, 128] bf16
  uint16_t *out;                         // [T, Hq, 128] bf16
  const uint16_t *k[kGqaMaxSegments];    // [len, Hkv, 128] bf16, token stride k_stride
  const uint16_t *v[kGqaMaxSegments];
  int64_t k_stride[kGqaMaxSegments];     // elements between consecutive tokens
  int64_t v_stride[kGqaMaxSegments];
  int len[kGqaMaxSegments];
  int num_segments;                      // the last one is the current (causal) chunk
  int T, Hq, Hkv, history;
  float scale;
  float *partial;                        // split-K partial states (nsplit > 1)
};

// Launch shape: key splits across workgroups (merged by a second kernel when
// > 1), waves per workgroup (4 or 8) and 16-row blocks per wave (1 or 2).
struct GqaShape {
  int nsplit;
  int waves;
  int rb;
};
GqaShape gqa_shape(int T, int Hq, int Hkv, int num_cus);
size_t gqa_partial_bytes(int T, int Hq, int nsplit);
hipError_t launch_gqa(const GqaArgs &a, GqaShape shape, hipStream_t s);

}  // namespace moe
