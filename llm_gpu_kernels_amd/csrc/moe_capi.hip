// C ABI for the MI355X MoE forward (include/moe_mi355x.h).
//
// Validation mirrors prepare_moe (src/llm_gpu_kernels/moe.py:220-235) and the
// contract of docs/MOE_USAGE.md:13-34: 1 <= E <= 256, H > 0, I > 0,
// 1 <= K <= 32, R = T*K < 2^31, R * max(H, 2I) < 2^31.  A plan stores
// pointers only; the caller owns every buffer.  moe_plan_run enqueues on the
// given stream with no synchronisation and no allocation.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <new>

#include "../../include/moe_mi355x.h"
#include "moe_internal.h"
#include <stdlib.h>

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char *what) {
  return fail(MOE_EDEVICE, "%s: %s", what, hipGetErrorString(e));
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Router fused into the planner's single workgroup while one round of its 16
// waves routes every token: one token per wave up to 16 tokens, two per wave
// (32 lanes each, E <= 128) up to 32.  Beyond that the standalone
// one-wave-per-token launch routes all tokens in parallel across CUs, which
// is faster than further serial rounds.
int fuse_router_mode(const moe_desc *d) {
  if (d->route_mode != MOE_ROUTE_LOGITS) return 0;
  if (d->T <= 16) return 1;
  if (d->T <= 32 && d->E <= 128) return 2;
  return 0;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

bool is_w4(int fmt) { return fmt == MOE_WEIGHTS_W4G128 || fmt == MOE_WEIGHTS_W4G128_FOLD; }

// Shape-only kernel policy (never route contents, so a captured graph stays
// valid when IDs change): mean rows per expert R/E below 32 -> weight
// streaming with 16- or 32-row tasks; otherwise LDS-tiled GEMMs with 64-row
// tasks.  An explicit token_block (16/32 stream, 64 tile) overrides it.
int choose_token_block(const moe_desc *d) {
  if (d->token_block == 16 || d->token_block == 32 || d->token_block == 64)
    return d->token_block;
  const long long r = (long long)d->T * d->K;
  if (r <= 16LL * d->E) return 16;
  if (r < 32LL * d->E) return 32;
  return 64;
}

int choose_path(const moe_desc *d, int tb) {
  const bool w4 = is_w4(d->weight_format);
  if (tb == 64) {
    if (moe::tile_shape_ok(d->H, d->I, w4)) return moe::kTile;
    return moe::stream_shape_ok(d->H, d->I, w4) ? moe::kStream : moe::kGeneric;
  }
  return moe::stream_shape_ok(d->H, d->I, w4) ? moe::kStream : moe::kGeneric;
}

int validate(const moe_desc *d) {
  if (!d) return fail(MOE_EINVAL, "null descriptor");
  if (d->E < 1 || d->E > 256) return fail(MOE_EINVAL, "E must be in [1, 256] (got %d)", d->E);
  if (d->H <= 0 || d->I <= 0) return fail(MOE_EINVAL, "H and I must be positive");
  if (d->K < 1 || d->K > 32) return fail(MOE_EINVAL, "top-k must be in [1, 32] (got %d)", d->K);
  if (d->T < 0) return fail(MOE_EINVAL, "T must be >= 0");
  const long long r = (long long)d->T * d->K;
  const long long wide = d->H > 2LL * d->I ? d->H : 2LL * d->I;
  if (r >= (1LL << 31) || r * wide >= (1LL << 31))
    return fail(MOE_EINVAL, "R=T*K and R*max(H,2I) must be < 2^31");
  if (d->weight_format != MOE_WEIGHTS_BF16 && !is_w4(d->weight_format))
    return fail(MOE_EINVAL, "unknown weight format %d", d->weight_format);
  if (d->id_dtype != MOE_IDS_INT32 && d->id_dtype != MOE_IDS_INT64)
    return fail(MOE_EINVAL, "unknown id dtype %d", d->id_dtype);
  if (d->route_mode != MOE_ROUTE_FIXED && d->route_mode != MOE_ROUTE_LOGITS)
    return fail(MOE_EINVAL, "unknown route mode %d", d->route_mode);
  if (d->route_mode == MOE_ROUTE_LOGITS) {
    if (d->id_dtype != MOE_IDS_INT32) return fail(MOE_EINVAL, "router mode writes int32 ids");
    if (d->K > d->E) return fail(MOE_EINVAL, "top-k %d exceeds E %d", d->K, d->E);
  }
  if (d->token_block != 0 && d->token_block != 16 && d->token_block != 32 &&
      d->token_block != 64)
    return fail(MOE_EINVAL, "token_block must be 0, 16, 32 or 64");
  if (is_w4(d->weight_format)) {
    if (!moe::flex_shape_ok(d->H, d->I, true))
      return fail(MOE_EINVAL, "W4G128 needs H %% 128 == 0 and I %% 32 == 0");
  }
  return MOE_OK;
}

// Router-fused shapes with 16-row tasks whose gate/up is a streaming kernel
// (bf16 through LDS, W4 straight into registers) plan in the gate/up prologue
// instead of a planner launch.  W4 shapes that take the decode-once wave
// kernel (R >= 4E, exact decode) keep the planner launch.
bool planned_gate_up(const moe_desc *d, int path, int tb) {
  if (path != moe::kStream || tb != 16) return false;
  const int fr = fuse_router_mode(d);
  if (!is_w4(d->weight_format)) return moe::dma_plan_ok(d->H, d->I, d->T, d->K, d->E, fr);
  const bool fold = d->weight_format == MOE_WEIGHTS_W4G128_FOLD;
  const bool wave = moe::wave_w4_shape_ok(d->H, d->I, tb) && (long long)d->T * d->K >= 4LL * d->E && !fold;
  return !wave && moe::stream_plan_ok(d->H, d->I, d->T, d->K, d->E, fr);
}

// Shapes the single-workgroup planner does not route itself (T > 32 with
// logits, every fixed-route shape) route and plan in one launch of several
// workgroups, all resident at once (at most one per CU).
constexpr int kAssumedCUs = 256;  // MI355X; plans use the device's own count
bool multi_planner(const moe_desc *d, int path, int tb, int num_cus) {
  if (planned_gate_up(d, path, tb) || fuse_router_mode(d) != 0) return false;
  return moe::multi_plan_ok(d->T, d->K, d->E, d->route_mode == MOE_ROUTE_LOGITS, num_cus);
}

int launch_count(const moe_desc *d, int path, int tb, int num_cus) {
  if (d->T == 0) return 0;
  if (planned_gate_up(d, path, tb)) return 3;  // gate/up (planning), down, combine
  if (multi_planner(d, path, tb, num_cus)) return 4;  // route+plan, gate/up, down, combine
  return 4 + (d->route_mode == MOE_ROUTE_LOGITS && fuse_router_mode(d) == 0 ? 1 : 0);
}

moe_layout compute_layout(const moe_desc *d) {
  moe_layout L;
  memset(&L, 0, sizeof(L));
  const size_t R = (size_t)d->T * d->K;
  const int tb = choose_token_block(d);
  const size_t cap = (R + tb - 1) / tb + (R < (size_t)d->E ? R : (size_t)d->E);
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o = align_up(o + bytes, 256);
    return at;
  };
  // status and counters first: at fixed offsets for every shape, so memory
  // reused across shapes (the static workspace) keeps them where the last
  // forward left them zero.
  L.status = take(4 * sizeof(uint32_t));
  L.counters = take(4 * 4);
  L.counts = take((size_t)d->E * 4);
  L.offsets = take((size_t)d->E * 4);
  L.ranks = take(R * 4);
  L.map = take(R * 4);
  L.row_route = take(R * 4 + 64 * 4);  // slack: scalar reads of up to 64 rows past R
  L.row_token = take(R * 4 + 64 * 4);
  L.tasks = take(cap * 16);
  L.num_tasks = take(4);
  {
    const int tpw = moe::multi_plan_tokens(d->K, d->E, d->route_mode == MOE_ROUTE_LOGITS);
    const size_t W = tpw > 0 ? ((size_t)d->T + tpw - 1) / tpw : 0;
    L.partials = take(W * ((size_t)d->E + 1) * 4 + 4);  // + the planner's arrival counter
  }
  L.act = take(R * (size_t)d->I * 2);
  L.routed = take(R * (size_t)d->H * 2);
  L.total = o;
  L.task_capacity = (int32_t)cap;
  L.token_block = tb;
  L.fast_path = choose_path(d, tb);
  L.launches = launch_count(d, L.fast_path, tb, kAssumedCUs);
  return L;
}

}  // namespace

namespace moe {
int capi_fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}
}  // namespace moe

struct moe_plan {
  moe_desc d;
  moe_layout L;
  int device;
  int num_cus;
  int fuse_router;  // 0: router launch, 1: one token per planner wave, 2: two
  bool planned;     // gate/up routes and plans in its prologue (no planner launch)
  bool multi;       // multi-workgroup router + planner launch
  bool test_planner_hold;  // MOE_TEST_PLANNER_HOLD=1 at create: see run_stages
  int path;
};

namespace {

// Validate `d` and fill `p` (no allocation, no device work).  The workspace
// pointer and size are checked against the layout the descriptor needs.
int bind_plan(moe_plan *p, const moe_desc *d) {
  int rc = validate(d);
  if (rc) return rc;
  const moe_layout L = compute_layout(d);
  if (d->T > 0) {
    if (!d->x || !d->ids || !d->weights || !d->down || !d->out || !d->workspace)
      return fail(MOE_EINVAL, "null tensor pointer");
    if (d->route_mode == MOE_ROUTE_LOGITS && !d->logits)
      return fail(MOE_EINVAL, "router mode needs logits");
    if (d->weight_format == MOE_WEIGHTS_BF16 && !d->gate_up)
      return fail(MOE_EINVAL, "null gate_up");
    if (is_w4(d->weight_format) && (!d->w4_words || !d->w4_scales))
      return fail(MOE_EINVAL, "null W4 words/scales");
    if (((uintptr_t)d->workspace & 255u) != 0)
      return fail(MOE_EINVAL, "workspace must be 256-byte aligned");
    if (d->workspace_bytes < L.total)
      return fail(MOE_ESPACE, "workspace has %zu bytes, needs %zu", d->workspace_bytes, L.total);
  }
  int path = L.fast_path;
  // A stream-sized task block on a shape only the tiled kernels take (or the
  // reverse) cannot happen: choose_path already matched them.  Every MFMA
  // kernel (tuned or run-time-K) reads 16-byte fragments: with an unaligned
  // buffer a bf16 forward takes the scalar kernels.
  const bool aligned = aligned16(d->x) && aligned16(d->down) && aligned16(d->out) &&
                       (is_w4(d->weight_format) ? aligned16(d->w4_words)
                                                               : aligned16(d->gate_up));
  if (!aligned && is_w4(d->weight_format))
    return fail(MOE_EINVAL, "W4G128 buffers must be 16-byte aligned");
  if (!aligned) path = moe::kScalar;
  p->d = *d;
  p->L = L;
  p->L.fast_path = path == moe::kScalar ? moe::kGeneric : path;
  p->path = path;
  p->fuse_router = fuse_router_mode(d);
  p->planned = planned_gate_up(d, path, L.token_block);
  hipError_t e = hipGetDevice(&p->device);
  if (e == hipSuccess)
    e = hipDeviceGetAttribute(&p->num_cus, hipDeviceAttributeMultiprocessorCount, p->device);
  if (e != hipSuccess) return hip_fail(e, "device query");
  p->multi = multi_planner(d, path, L.token_block, p->num_cus);
  {
    const char *h = getenv("MOE_TEST_PLANNER_HOLD");
    p->test_planner_hold = h && h[0] == '1';
  }
  p->L.launches = launch_count(d, path, L.token_block, p->num_cus);
  return MOE_OK;
}

// ---- workspace for callers that cannot allocate ---------------------------
// One array per GPU the library runs on, held until the process ends.  Host
// code never uses the array's name as an address: the device address comes
// from hipGetSymbolAddress, once per device, with that device current.
constexpr size_t kStaticWorkspaceBytes = MOE_STATIC_WORKSPACE_BYTES;
static __device__ __align__(256) uint8_t scratch[kStaticWorkspaceBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on `device` (current), looked up on first use.
int static_workspace(int device, void **ptr) {
  if (device < 0 || device >= kMaxDevices) return fail(MOE_EINVAL, "device %d out of range", device);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!p) return fail(MOE_EDEVICE, "null static workspace address");
    g_scratch_ptr[device] = p;
  }
  *ptr = g_scratch_ptr[device];
  return MOE_OK;
}

}  // namespace

extern "C" {

int moe_abi_version(void) { return MOE_ABI_VERSION; }

const char *moe_last_error(void) { return g_err; }

int moe_workspace_layout(const moe_desc *d, moe_layout *out) {
  int rc = validate(d);
  if (rc) return rc;
  if (!out) return fail(MOE_EINVAL, "null layout");
  *out = compute_layout(d);
  return MOE_OK;
}

int moe_plan_create(moe_plan **out, const moe_desc *d) {
  if (!out) return fail(MOE_EINVAL, "null plan pointer");
  *out = nullptr;
  moe_plan tmp;
  int rc = bind_plan(&tmp, d);
  if (rc) return rc;
  moe_plan *p = new (std::nothrow) moe_plan(tmp);
  if (!p) return fail(MOE_EINVAL, "out of host memory");
  *out = p;
  return MOE_OK;
}

int moe_plan_layout(const moe_plan *p, moe_layout *out) {
  if (!p || !out) return fail(MOE_EINVAL, "null argument");
  *out = p->L;
  return MOE_OK;
}

// Launch stages [first, last) of one forward.  Stage order:
// [router] route_plan gate_up down combine, or gate_up (planning) down combine.
static int run_stages(moe_plan *p, int first, int last, void *stream) {
  const moe_desc &d = p->d;
  if (d.T == 0) return MOE_OK;
  int prev = -1;
  hipError_t e = hipGetDevice(&prev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (prev != p->device && (e = hipSetDevice(p->device)) != hipSuccess)
    return hip_fail(e, "hipSetDevice");
  hipStream_t s = (hipStream_t)stream;
  char *ws = (char *)d.workspace;
  const moe_layout &L = p->L;

  moe::RouteArgs ra;
  ra.logits = (const float *)d.logits;
  ra.ids = d.ids;
  ra.weights = (float *)d.weights;
  ra.status = (uint32_t *)(ws + L.status);
  ra.counts = (int32_t *)(ws + L.counts);
  ra.offsets = (int32_t *)(ws + L.offsets);
  ra.ranks = (int32_t *)(ws + L.ranks);
  ra.map = (int32_t *)(ws + L.map);
  ra.row_route = (int32_t *)(ws + L.row_route);
  ra.row_token = (int32_t *)(ws + L.row_token);
  ra.tasks = (int4 *)(ws + L.tasks);
  ra.num_tasks = (int32_t *)(ws + L.num_tasks);
  ra.counters = (int32_t *)(ws + L.counters);
  ra.T = d.T;
  ra.K = d.K;
  ra.E = d.E;
  ra.R = d.T * d.K;
  ra.route_logits = d.route_mode == MOE_ROUTE_LOGITS;
  ra.renormalize = d.renormalize;
  ra.id64 = d.id_dtype == MOE_IDS_INT64;
  ra.fuse_router = p->fuse_router;
  ra.token_block = L.token_block;
  ra.partials = (int32_t *)(ws + L.partials);
  ra.plan_tpw = moe::multi_plan_tokens(d.K, d.E, ra.route_logits);
  ra.plan_spin_cap = moe::kMultiSpinCap;
  ra.plan_hold_wg = -1;
  // Test hook (failure-handling tests only): the last planner workgroup
  // withholds its counts and every wait gives up after a few rounds, so the
  // stalled-plan path runs with every kernel exiting normally.
  if (p->test_planner_hold) {
    ra.plan_spin_cap = 64;
    ra.plan_hold_wg = (d.T + ra.plan_tpw - 1) / ra.plan_tpw - 1;
  }

  moe::ExpertArgs xa;
  xa.x = (const uint16_t *)d.x;
  xa.gate_up = (const uint16_t *)d.gate_up;
  xa.w4_words = (const uint32_t *)d.w4_words;
  xa.w4_scales = (const uint16_t *)d.w4_scales;
  xa.down = (const uint16_t *)d.down;
  xa.weights = (const float *)d.weights;
  xa.map = ra.map;
  xa.row_route = ra.row_route;
  xa.row_token = ra.row_token;
  xa.num_tasks = ra.num_tasks;
  xa.counts = ra.counts;
  xa.offsets = ra.offsets;
  xa.tasks = ra.tasks;
  xa.counters = ra.counters;
  xa.status = ra.status;
  xa.act = (uint16_t *)(ws + L.act);
  xa.routed = (uint16_t *)(ws + L.routed);
  xa.out = (uint16_t *)d.out;
  xa.T = d.T;
  xa.H = d.H;
  xa.I = d.I;
  xa.E = d.E;
  xa.K = d.K;
  xa.R = ra.R;
  xa.w4_fold = d.weight_format == MOE_WEIGHTS_W4G128_FOLD ? 1 : 0;

  const bool w4 = is_w4(d.weight_format);
  const bool router = ra.route_logits && !ra.fuse_router;
  int rc = MOE_OK;
  for (int st = first; st < last && rc == MOE_OK; ++st) {
    // 0 router, 1 plan, 2 gate/up, 3 down, 4 combine, 5 gate/up with the plan,
    // 6 multi-workgroup router + plan
    const int kind = p->planned ? (st == 0 ? 5 : st + 2)
                     : p->multi ? (st == 0 ? 6 : st + 1)
                     : router   ? st
                                : st + 1;
    switch (kind) {
      case 0: e = moe::launch_router(ra, s); break;
      case 1: e = moe::launch_route_plan(ra, s); break;
      case 2:
        e = moe::launch_gate_up(xa, L.task_capacity, L.token_block, w4, p->path, p->num_cus, s);
        break;
      case 3:
        e = moe::launch_down(xa, L.task_capacity, L.token_block, p->path, p->num_cus, s);
        break;
      case 4: e = moe::launch_combine(xa, s); break;
      case 5:
        e = w4 ? moe::launch_stream_gate_up_planned(xa, ra, L.task_capacity, p->num_cus, s)
               : moe::launch_dma_gate_up_planned(xa, ra, p->num_cus, s);
        break;
      default: e = moe::launch_route_plan_multi(ra, s); break;
    }
    if (e != hipSuccess) {
      static const char *names[] = {"router", "route plan", "gate/up", "down", "combine", "gate/up",
                                    "route plan"};
      rc = hip_fail(e, names[kind]);
    }
  }
  if (prev != p->device) (void)hipSetDevice(prev);
  return rc;
}

int moe_plan_run(moe_plan *p, void *stream) {
  if (!p) return fail(MOE_EINVAL, "null plan");
  return run_stages(p, 0, p->L.launches, stream);
}

int moe_plan_run_stage(moe_plan *p, int32_t stage, void *stream) {
  if (!p) return fail(MOE_EINVAL, "null plan");
  if (stage < 0 || stage >= p->L.launches)
    return fail(MOE_EINVAL, "stage %d outside [0, %d)", stage, p->L.launches);
  return run_stages(p, stage, stage + 1, stream);
}

int moe_plan_read_status(moe_plan *p, void *stream, uint32_t *flags) {
  if (!p || !flags) return fail(MOE_EINVAL, "null argument");
  *flags = 0;
  if (p->d.T == 0) return MOE_OK;
  hipError_t e = hipStreamSynchronize((hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
  const char *ws = (const char *)p->d.workspace;
  e = hipMemcpy(flags, ws + p->L.status, sizeof(uint32_t), hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(e, "status readback");
  // Every completed launch leaves the work counters at zero; anything else
  // means a launch did not run to completion on this workspace.
  int32_t cnt[4];
  e = hipMemcpy(cnt, ws + p->L.counters, sizeof(cnt), hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(e, "counter readback");
  if (cnt[0] | cnt[1] | cnt[2] | cnt[3]) *flags |= MOE_STATUS_DIRTY_COUNTERS;
  return MOE_OK;
}

int moe_forward_static(const moe_desc *d, void *stream) {
  if (!d) return fail(MOE_EINVAL, "null descriptor");
  int rc = validate(d);
  if (rc) return rc;
  if (d->T == 0) return MOE_OK;
  const moe_layout L = compute_layout(d);
  if (L.total > kStaticWorkspaceBytes)
    return fail(MOE_ESPACE,
                "moe_forward_static: this shape needs %zu workspace bytes; the static "
                "workspace holds %zu (use moe_plan_create with a caller workspace)",
                L.total, kStaticWorkspaceBytes);
  int device = -1;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  void *ws = nullptr;
  if ((rc = static_workspace(device, &ws))) return rc;
  moe_desc sd = *d;
  sd.workspace = ws;
  sd.workspace_bytes = kStaticWorkspaceBytes;
  moe_plan p;
  if ((rc = bind_plan(&p, &sd))) return rc;
  // The array keeps the previous call's contents: the work counters and the
  // status words must start at zero.
  e = moe::launch_reset_counters((int32_t *)((char *)ws + L.counters),
                                 (uint32_t *)((char *)ws + L.status),
                                 (int32_t *)((char *)ws + L.partials),
                                 (int)((L.act - L.partials) / 4), (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "static workspace reset");
  return run_stages(&p, 0, p.L.launches, stream);
}

int moe_plan_reset_counters(moe_plan *p, void *stream) {
  if (!p) return fail(MOE_EINVAL, "null plan");
  if (p->d.T == 0) return MOE_OK;
  int prev = -1;
  hipError_t e = hipGetDevice(&prev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (prev != p->device && (e = hipSetDevice(p->device)) != hipSuccess)
    return hip_fail(e, "hipSetDevice");
  char *ws = (char *)p->d.workspace;
  e = moe::launch_reset_counters((int32_t *)(ws + p->L.counters), nullptr,
                                 (int32_t *)(ws + p->L.partials),
                                 (int)((p->L.act - p->L.partials) / 4), (hipStream_t)stream);
  if (prev != p->device) (void)hipSetDevice(prev);
  if (e != hipSuccess) return hip_fail(e, "counter reset");
  return MOE_OK;
}

void moe_plan_destroy(moe_plan *p) { delete p; }

int moe_w4_dequantize(const void *words_t, const void *scales_t, int32_t E, int32_t N, int32_t K,
                      void *out_bf16, void *stream) {
  if (E < 1 || N < 16 || N % 16 || K < 128 || K % 128)
    return fail(MOE_EINVAL, "W4 dequantize needs N %% 16 == 0, K %% 128 == 0");
  if (!words_t || !scales_t || !out_bf16 || !aligned16(words_t) || !aligned16(out_bf16))
    return fail(MOE_EINVAL, "null or misaligned W4 buffer");
  hipError_t e = moe::launch_w4_dequantize((const uint32_t *)words_t, (const uint16_t *)scales_t,
                                           E, N, K, (uint16_t *)out_bf16, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "W4 dequantize launch");
  return MOE_OK;
}

}  // extern "C"
