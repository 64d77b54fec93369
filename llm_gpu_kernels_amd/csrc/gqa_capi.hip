// C ABI of the segmented-KV GQA attention (include/gqa_mi355x.h).
//
// Validation mirrors _validate_attention_input / _validate_output of the
// reference (attention_cuda_compact.py:97-121): bf16, [L, heads, 128] with
// inner strides (128, 1), token stride >= heads*128 and a multiple of 8,
// 16-byte aligned bases; the current segment's length equals T.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include <new>

#include "../../include/gqa_mi355x.h"
#include "gqa_internal.h"

namespace moe {
int capi_fail(int code, const char *fmt, ...);  // moe_capi.hip (thread-local message)
}

struct gqa_seg_plan {
  moe::GqaArgs a;
  moe::GqaShape shape;
  int device;
};

namespace {

constexpr int64_t kMaxTokenStride = 1LL << 25;

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

int validate(const gqa_seg_desc *d, int num_cus, moe::GqaShape *shape) {
  using moe::capi_fail;
  if (!d) return capi_fail(MOE_EINVAL, "null descriptor");
  if (d->D != 128) return capi_fail(MOE_EINVAL, "head_dim must be 128 (got %d)", d->D);
  if (d->T < 0) return capi_fail(MOE_EINVAL, "T must be >= 0");
  if (d->Hkv < 1 || d->Hq < 1 || d->Hq % d->Hkv)
    return capi_fail(MOE_EINVAL, "Hq must be a positive multiple of Hkv");
  const int G = d->Hq / d->Hkv;
  if (G != 1 && G != 2 && G != 4 && G != 8)
    return capi_fail(MOE_EINVAL, "Hq / Hkv must be 1, 2, 4 or 8 (got %d)", G);
  if (d->num_segments < 1 || d->num_segments > GQA_MAX_SEGMENTS)
    return capi_fail(MOE_EINVAL, "1..4 KV segments required");
  if (d->len[d->num_segments - 1] != d->T)
    return capi_fail(MOE_EINVAL, "the current segment must have T = %d tokens", d->T);
  for (int s = 0; s < d->num_segments; ++s) {
    if (d->len[s] < 0) return capi_fail(MOE_EINVAL, "segment %d has negative length", s);
    if (d->len[s] == 0) continue;
    if (!d->k[s] || !d->v[s] || !aligned16(d->k[s]) || !aligned16(d->v[s]))
      return capi_fail(MOE_EINVAL, "segment %d k/v must be non-null and 16-byte aligned", s);
    const int64_t minst = (int64_t)d->Hkv * 128;
    if (d->k_stride[s] < minst || d->v_stride[s] < minst || d->k_stride[s] % 8 ||
        d->v_stride[s] % 8)
      return capi_fail(MOE_EINVAL, "segment %d token stride must be >= %lld and a multiple of 8",
                       s, (long long)minst);
    // The kernel addresses 32 consecutive rows with 32-bit byte offsets.
    if (d->k_stride[s] > kMaxTokenStride || d->v_stride[s] > kMaxTokenStride)
      return capi_fail(MOE_EINVAL, "segment %d token stride must be <= %lld elements", s,
                       (long long)kMaxTokenStride);
  }
  if (d->T > 0 && (!d->q || !d->out || !aligned16(d->q) || !aligned16(d->out)))
    return capi_fail(MOE_EINVAL, "q/out must be non-null and 16-byte aligned");
  if ((long long)d->T * d->Hq * 128 >= (1LL << 31))
    return capi_fail(MOE_EINVAL, "T * Hq * 128 must be < 2^31");
  *shape = moe::gqa_shape(d->T, d->Hq, d->Hkv, num_cus);
  return MOE_OK;
}

int device_cus(int *device, int *cus) {
  hipError_t e = hipGetDevice(device);
  if (e == hipSuccess) e = hipDeviceGetAttribute(cus, hipDeviceAttributeMultiprocessorCount, *device);
  if (e != hipSuccess) return moe::capi_fail(MOE_EDEVICE, "device query: %s", hipGetErrorString(e));
  return MOE_OK;
}

}  // namespace

extern "C" {

int gqa_seg_workspace_bytes(const gqa_seg_desc *d, size_t *bytes) {
  int dev = 0, cus = 0;
  moe::GqaShape shape{1, 4, 2};
  int rc = device_cus(&dev, &cus);
  if (rc) return rc;
  if ((rc = validate(d, cus, &shape))) return rc;
  if (!bytes) return moe::capi_fail(MOE_EINVAL, "null bytes");
  *bytes = moe::gqa_partial_bytes(d->T, d->Hq, shape.nsplit);
  return MOE_OK;
}

int gqa_seg_plan_create(gqa_seg_plan **out, const gqa_seg_desc *d) {
  if (!out) return moe::capi_fail(MOE_EINVAL, "null plan pointer");
  *out = nullptr;
  int dev = 0, cus = 0;
  moe::GqaShape shape{1, 4, 2};
  int rc = device_cus(&dev, &cus);
  if (rc) return rc;
  if ((rc = validate(d, cus, &shape))) return rc;
  const size_t need = moe::gqa_partial_bytes(d->T, d->Hq, shape.nsplit);
  if (need && (d->workspace_bytes < need || !d->workspace || !aligned16(d->workspace)))
    return moe::capi_fail(MOE_ESPACE, "workspace has %zu bytes, needs %zu", d->workspace_bytes,
                          need);
  gqa_seg_plan *p = new (std::nothrow) gqa_seg_plan;
  if (!p) return moe::capi_fail(MOE_EINVAL, "out of host memory");
  moe::GqaArgs &a = p->a;
  a.q = (const uint16_t *)d->q;
  a.out = (uint16_t *)d->out;
  a.num_segments = d->num_segments;
  a.history = 0;
  for (int s = 0; s < moe::kGqaMaxSegments; ++s) {
    const bool live = s < d->num_segments;
    a.k[s] = live ? (const uint16_t *)d->k[s] : nullptr;
    a.v[s] = live ? (const uint16_t *)d->v[s] : nullptr;
    a.k_stride[s] = live ? d->k_stride[s] : 0;
    a.v_stride[s] = live ? d->v_stride[s] : 0;
    a.len[s] = live ? d->len[s] : 0;
    if (live && s < d->num_segments - 1) a.history += d->len[s];
  }
  a.T = d->T;
  a.Hq = d->Hq;
  a.Hkv = d->Hkv;
  a.scale = (d->scale > 0.f && d->scale < INFINITY) ? d->scale : 1.0f / sqrtf((float)d->D);
  a.partial = (float *)d->workspace;
  p->shape = shape;
  p->device = dev;
  *out = p;
  return MOE_OK;
}

int gqa_seg_plan_run(gqa_seg_plan *p, void *stream) {
  if (!p) return moe::capi_fail(MOE_EINVAL, "null plan");
  if (p->a.T == 0) return MOE_OK;
  int prev = -1;
  hipError_t e = hipGetDevice(&prev);
  if (e == hipSuccess && prev != p->device) e = hipSetDevice(p->device);
  if (e == hipSuccess) e = moe::launch_gqa(p->a, p->shape, (hipStream_t)stream);
  if (prev >= 0 && prev != p->device) (void)hipSetDevice(prev);
  if (e != hipSuccess) return moe::capi_fail(MOE_EDEVICE, "gqa launch: %s", hipGetErrorString(e));
  return MOE_OK;
}

void gqa_seg_plan_destroy(gqa_seg_plan *p) { delete p; }

}  // extern "C"
