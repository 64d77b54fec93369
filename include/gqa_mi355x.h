/*
 * gqa_mi355x.h -- C ABI of the MI355X (gfx950) segmented-KV GQA prefill
 * attention (secondary path of the MoE build).
 *
 * Replaces CompactCudaGqaPlan(q, ks, vs, out, stages) + run()
 * (src/llm_gpu_kernels/cuda_gqa_attention_compact.cu:211-280) behind
 * prepare_cuda_gqa_compact (attention_cuda_compact.py:135-186).  Same
 * conventions as moe_mi355x.h: device pointers owned by the caller, 0 or a
 * negative MOE_E* code, message in moe_last_error().
 *
 * q [T, Hq, 128] bf16 contiguous; 1..4 KV segments, each k/v [L, Hkv, 128]
 * bf16 with inner strides (128, 1) and a token stride (elements) >= Hkv*128
 * and <= 2^25,
 * multiple of 8; the last segment is the current chunk (L == T, causal), the
 * others are fully visible history.  out [T, Hq, 128] bf16 contiguous.
 * Hq % Hkv == 0 and Hq / Hkv in {1, 2, 4, 8}; head_dim must be 128.
 */
#ifndef GQA_MI355X_H
#define GQA_MI355X_H

#include <stddef.h>
#include <stdint.h>

#include "moe_mi355x.h"

#ifdef __cplusplus
extern "C" {
#endif

#define GQA_MAX_SEGMENTS 4

typedef struct gqa_seg_desc {
  int32_t T, Hq, Hkv, D, num_segments;
  int32_t len[GQA_MAX_SEGMENTS];
  const void *q;
  void *out;
  const void *k[GQA_MAX_SEGMENTS];
  const void *v[GQA_MAX_SEGMENTS];
  int64_t k_stride[GQA_MAX_SEGMENTS]; /* token stride in elements */
  int64_t v_stride[GQA_MAX_SEGMENTS];
  float scale;                        /* <= 0 or non-finite: 1/sqrt(D) */
  void *workspace;                    /* split-K partials; >= gqa_seg_workspace_bytes() */
  size_t workspace_bytes;
} gqa_seg_desc;

typedef struct gqa_seg_plan gqa_seg_plan;

/* Workspace bytes the plan needs on the current device (0 when unsplit). */
int gqa_seg_workspace_bytes(const gqa_seg_desc *d, size_t *bytes);
int gqa_seg_plan_create(gqa_seg_plan **out, const gqa_seg_desc *d);
/* Enqueue on `stream` (hipStream_t); no sync, no allocation; T == 0 launches nothing. */
int gqa_seg_plan_run(gqa_seg_plan *p, void *stream);
void gqa_seg_plan_destroy(gqa_seg_plan *p);

#ifdef __cplusplus
}
#endif
#endif /* GQA_MI355X_H */
