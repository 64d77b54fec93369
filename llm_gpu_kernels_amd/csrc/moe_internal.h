// Internal launch interface between the C ABI layer and the kernel files.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

// Routing stage: router (optional), status, canonical ranks, scan, map, tasks.
struct RouteArgs {
  const float *logits;     // [T, E] (logits mode)
  void *ids;               // [T, K] int32 / int64 (int32 output in logits mode)
  float *weights;          // [T, K]
  uint32_t *status;        // [2]: status bits, router flag word (self-clearing)
  int32_t *counts, *offsets, *ranks, *map, *row_route;
  int32_t *row_token;      // [R] token of grouped row p (row_route[p] / K)
  int4 *tasks;             // {expert, first grouped row, rows, 0}
  int32_t *num_tasks;
  int32_t *counters;       // [4] work counters of the streaming GEMMs
  int32_t *partials;       // multi-workgroup planner: [W][E + 1] tagged counts and flags
  int T, K, E, R;
  int route_logits, renormalize, id64, fuse_router;
  int token_block;
  int plan_tpw;            // multi-workgroup planner: tokens per workgroup
  int plan_spin_cap;       // multi-workgroup planner: re-reads of a batch before it gives up
  int plan_hold_wg;        // test hook: this workgroup never publishes (-1: none)
};

// Multi-workgroup planner wait bound (re-read rounds of about 1 us).
constexpr int kMultiSpinCap = 1 << 20;

// Status bit set when a bounded cross-workgroup wait ran out (never expected).
constexpr uint32_t kStatusStalled = 16u;
constexpr uint32_t kStatusDirtyCounters = 8u;

// Expert stage: gate/up + SwiGLU, down projection, weighted combine.
struct ExpertArgs {
  const uint16_t *x;           // [T, H] bf16
  const uint16_t *gate_up;     // [E, 2I, H] bf16
  const uint32_t *w4_words;    // tiled int4 words
  const uint16_t *w4_scales;   // tiled bf16 scales
  const uint16_t *down;        // [E, H, I] bf16
  const float *weights;        // [T, K]
  const int32_t *map, *row_route, *row_token, *num_tasks;
  const int32_t *counts, *offsets;  // [E] rows per expert and their first grouped row
  const int4 *tasks;
  int32_t *counters;           // [4] {units taken, workgroups done} of gate/up, down
  uint32_t *status;            // [4] status words (status[0]: MOE_STATUS_* bits)
  uint16_t *act;               // [R, I] bf16, grouped-row order
  uint16_t *routed;            // [R, H] bf16, route order
  uint16_t *out;               // [T, H] bf16
  int T, H, I, E, K, R;
  int w4_fold;                 // W4: folded decode where the kernel implements it (MOE_WEIGHTS_W4G128_FOLD)
};

// Router kernel for large T (one wave per token); folds its flags into status[1].
hipError_t launch_router(const RouteArgs &a, hipStream_t s);
// Single-workgroup planner (fuses the router when a.fuse_router).
hipError_t launch_route_plan(const RouteArgs &a, hipStream_t s);
// Multi-workgroup router + planner (a.plan_tpw tokens per workgroup).
int multi_plan_tokens(int K, int E, bool router);
bool multi_plan_ok(int T, int K, int E, bool router, int num_cus);
hipError_t launch_route_plan_multi(const RouteArgs &a, hipStream_t s);

// token_block: 16 or 32 grouped rows per task.  fast: MFMA kernels (shape
// constraints checked by the caller), otherwise the generic kernels.
hipError_t launch_gate_up(const ExpertArgs &a, int task_capacity, int token_block, bool w4,
                          int path, int num_cus, hipStream_t s);
hipError_t launch_down(const ExpertArgs &a, int task_capacity, int token_block, int path,
                       int num_cus, hipStream_t s);
hipError_t launch_stream_gate_up(const ExpertArgs &a, int task_capacity, int token_block, bool w4,
                                 int num_cus, hipStream_t s);
hipError_t launch_stream_down(const ExpertArgs &a, int task_capacity, int token_block,
                              int num_cus, hipStream_t s);
bool stream_shape_ok(int H, int I, bool w4);
// W4 gate/up that routes and plans in its prologue (no planner launch).
bool stream_plan_ok(int H, int I, int T, int K, int E, int fuse_router);
hipError_t launch_stream_gate_up_planned(const ExpertArgs &a, const RouteArgs &ra, int task_capacity,
                                         int num_cus, hipStream_t s);
// bf16 streaming GEMMs through LDS (16/32-row tasks), moe_dma.hip.
bool dma_shape_ok(int H, int I, int token_block);
hipError_t launch_dma_gate_up(const ExpertArgs &a, int token_block, int num_cus, hipStream_t s);
hipError_t launch_dma_down(const ExpertArgs &a, int token_block, int num_cus, hipStream_t s);
// The same gate/up kernel routing and planning in its prologue (replaces the
// planner launch for router-fused shapes; writes every global plan array).
bool dma_plan_ok(int H, int I, int T, int K, int E, int fuse_router);
hipError_t launch_dma_gate_up_planned(const ExpertArgs &a, const RouteArgs &ra, int num_cus,
                                      hipStream_t s);
// W4 gate/up + SwiGLU, one unit per wave with K-chunked token rows in LDS, for
// tasks with several rows per expert (token_block 16, 32 or 64).
bool wave_w4_shape_ok(int H, int I, int token_block);
hipError_t launch_wave_w4_gate_up(const ExpertArgs &a, int task_capacity, int token_block,
                                  hipStream_t s);
hipError_t launch_tile_gate_up(const ExpertArgs &a, int task_capacity, int num_cus,
                               hipStream_t s);
hipError_t launch_tile_down(const ExpertArgs &a, int task_capacity, int num_cus, hipStream_t s);
bool tile_shape_ok(int H, int I, bool w4);

// Expert-stage kernel families (moe_layout.fast_path).
// kGeneric: the run-time-K MFMA kernels (or scalar kernels where H or I is not
// a multiple of 32); kScalar: the scalar kernels (unaligned bf16 buffers).
enum Path { kGeneric = 0, kStream = 1, kTile = 2, kScalar = 3 };
// MFMA kernels for any H, I that are multiples of 32 (W4: H of 128) -- the
// shapes the tuned kernels above do not take (kGeneric path).
bool flex_shape_ok(int H, int I, bool w4);
hipError_t launch_flex_gate_up(const ExpertArgs &a, int task_capacity, int token_block, bool w4,
                               hipStream_t s);
hipError_t launch_flex_down(const ExpertArgs &a, int task_capacity, int token_block, hipStream_t s);
hipError_t launch_combine(const ExpertArgs &a, hipStream_t s);
// Zero the four work counters, the planner's `n_partials` published words
// and, when `status` is not null, the two status words, with a kernel:
// capturable, no memset node.
hipError_t launch_reset_counters(int32_t *counters, uint32_t *status, int32_t *partials,
                                 int n_partials, hipStream_t s);
hipError_t launch_w4_dequantize(const uint32_t *words_t, const uint16_t *scales_t, int E, int N,
                                int K, uint16_t *out, hipStream_t s);

constexpr size_t kMaxLds = 160 * 1024;

}  // namespace moe
