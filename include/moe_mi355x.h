/*
 * moe_mi355x.h -- C ABI of the MI355X (gfx950) MoE forward.
 *
 * Plain C: pointers, sizes and status codes only.  Every device pointer is
 * owned by the caller (PyTorch in the Python layer); a plan stores pointers
 * and never frees them.  All functions return 0 on success or a negative
 * MOE_E* code; moe_last_error() then holds a thread-local message.
 *
 * Reference interfaces replaced (paths relative to the reference root):
 *   moe_plan_create / moe_plan_run   <- prepare_moe + PreparedMoE.run
 *       (src/llm_gpu_kernels/moe.py:124-245), the ranked launcher
 *       (moe_ranked.py:68-169), prepare_configured_moe (moe_configured.py:17)
 *       and the native GateUpPlan / W4GateUpPlan / W4LayoutGateUpPlan
 *       constructors + run() (cuda_gate_up.cu:133-183,
 *       cuda_w4_gate_up.cu:102-144, cuda_w4_layout_gate_up.cu:112-160).
 *   moe_plan_read_status             <- PreparedMoE.check_inputs (moe.py:157-160)
 *   moe_w4_quantize                  <- quantize_gate_up (moe_weight_quant.py:55-105)
 *   moe_w4_tile                      <- repack_gate_up (moe_weight_layout.py:81-127)
 *   moe_w4_dequantize                <- dequantize_gate_up_reference
 *                                       (moe_weight_quant.py:35-52)
 */
#ifndef MOE_MI355X_H
#define MOE_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOE_ABI_VERSION 2

/* Return codes. */
#define MOE_OK 0
#define MOE_EINVAL (-1)   /* bad shape / dtype / pointer (ValueError in Python)   */
#define MOE_EDEVICE (-2)  /* HIP runtime error (RuntimeError in Python)            */
#define MOE_ESPACE (-3)   /* workspace smaller than moe_workspace_bytes()          */

/* Status bits written by the forward on the device (moe_ranked.py:26-31). */
#define MOE_STATUS_BAD_ID 1u      /* an expert ID outside [0, E)              */
#define MOE_STATUS_BAD_WEIGHT 2u  /* a non-finite routing weight              */
#define MOE_STATUS_BAD_LOGIT 4u   /* a non-finite router logit (router mode)  */
#define MOE_STATUS_STALLED 16u    /* the multi-workgroup planner's view was
                                     incomplete: a bounded cross-workgroup wait ran
                                     out (its workgroups did not all become resident
                                     together, e.g. another stream's kernel held CUs)
                                     or a published count failed its bounds (a
                                     workspace that was not zeroed).  The forward
                                     then ran no GEMM tasks: the output is invalid */
#define MOE_STATUS_DIRTY_COUNTERS 8u /* the work counters were not zero when a
                                        counter-scheduled GEMM launched (the launch
                                        counts the units it ran and latches this bit
                                        when the count is off: the output is invalid),
                                        or read_status found them nonzero after the
                                        stream drained.  moe_plan_reset_counters or
                                        any later complete forward clears them     */

/* moe_desc.weight_format */
#define MOE_WEIGHTS_BF16 0        /* gate_up bf16 [E, 2I, H]                  */
#define MOE_WEIGHTS_W4G128 1      /* gate_up int4 in the tiled layout below;  *
                                   * needs H % 128 == 0 and I % 32 == 0        */
/* The same W4G128 weights, opt-in folded decode: where a kernel implements it
 * (the split-K streaming gate/up, used in this mode for 16- and 32-row tasks), the
 * MFMAs run on the exact values 136 + q and each 128-K group's fp32 sum is
 * scaled after subtracting 136 x the group's token sums, i.e. the effective
 * weights are q * scale exactly instead of bf16_rn(q * scale) (no counterpart
 * in the reference, whose kernels dequantise to bf16; within the layer
 * tolerance, 7 instead of 17 decode instructions per 8 weights).  Other
 * kernels keep the bit-exact bf16 decode. */
#define MOE_WEIGHTS_W4G128_FOLD 2

/* moe_desc.id_dtype */
#define MOE_IDS_INT32 0
#define MOE_IDS_INT64 1

/* moe_desc.route_mode */
#define MOE_ROUTE_FIXED 0         /* ids + weights given (reference semantics) */
#define MOE_ROUTE_LOGITS 1        /* softmax -> top-k -> renorm on the GPU;
                                     ids (int32) and weights are outputs      */

typedef struct moe_desc {
  int32_t T, H, I, E, K;          /* tokens, hidden, intermediate, experts, top-k */
  int32_t weight_format;          /* MOE_WEIGHTS_*                                 */
  int32_t id_dtype;               /* MOE_IDS_*   (MOE_IDS_INT32 in logits mode)    */
  int32_t route_mode;             /* MOE_ROUTE_*                                   */
  int32_t renormalize;            /* logits mode: divide top-k weights by their sum */
  int32_t token_block;            /* 0 = choose from shape; 16/32 (stream) or 64 (tile) */
  const void *x;                  /* [T, H] bf16                                   */
  const void *logits;             /* [T, E] fp32 (logits mode) or NULL             */
  void *ids;                      /* [T, K] int32/int64                            */
  void *weights;                  /* [T, K] fp32                                   */
  const void *gate_up;            /* [E, 2I, H] bf16 (MOE_WEIGHTS_BF16)            */
  const void *w4_words;           /* moe_w4_tile() words  (MOE_WEIGHTS_W4G128)     */
  const void *w4_scales;          /* moe_w4_tile() scales (MOE_WEIGHTS_W4G128)     */
  const void *down;               /* [E, H, I] bf16                                */
  void *out;                      /* [T, H] bf16                                   */
  void *workspace;                /* device, >= moe_workspace_bytes(), 256-B aligned */
  size_t workspace_bytes;
} moe_desc;

/* Byte offsets of the inspectable workspace arrays (int32 unless noted). */
typedef struct moe_layout {
  size_t status;      /* [4]  uint32: status bits, router bits, planner epoch, 0  */
  size_t counts;      /* [E]  routes per expert                                  */
  size_t offsets;     /* [E]  exclusive scan of counts                           */
  size_t ranks;       /* [R]  expert-local rank of route q = t*K + s (-1: bad id) */
  size_t map;         /* [R]  grouped row of route q (-1: bad id)                */
  size_t row_route;   /* [R]  route of grouped row p (inverse of map)            */
  size_t row_token;   /* [R]  token of grouped row p (row_route[p] / K)          */
  size_t tasks;       /* [task_capacity][4] {expert, first row, rows, 0}         */
  size_t num_tasks;   /* [1]                                                     */
  size_t counters;    /* [4]  work counters of the streaming GEMMs (0 between launches) */
  size_t partials;    /* [W][E+1] uint32 per-workgroup counts of the multi-workgroup
                         planner, tagged with the planner epoch                    */
  size_t act;         /* [R, I] bf16 SwiGLU activations in grouped-row order     */
  size_t routed;      /* [R, H] bf16 down projections in route order             */
  size_t total;       /* workspace bytes                                          */
  int32_t task_capacity;
  int32_t token_block;
  int32_t launches;   /* kernel launches per forward: 4 route+plan, gate/up,     *
                       * down, combine (one planner launch routes too); 3 when   *
                       * the bf16 gate/up launch routes and plans itself         *
                       * (T <= 32); 5 (separate router launch) only for shapes   *
                       * with more tokens than the planner's workgroups hold     *
                       * (T > 16 x CU count); 0 when T == 0                      */
  int32_t fast_path;  /* 0 run-time-K MFMA kernels (other shapes; scalar where   
                         H or I is not a multiple of 32), 1 MFMA weight         
                         streaming, 2 MFMA LDS-tiled (many rows per expert)     */
} moe_layout;

typedef struct moe_plan moe_plan;

int moe_abi_version(void);
const char *moe_last_error(void);

/* Workspace size and layout for a descriptor (pointers may be NULL). */
int moe_workspace_layout(const moe_desc *d, moe_layout *out);

/* Validate the descriptor and bind its pointers.  No allocation, no launch,
 * no device work (so it may run during stream capture).  The workspace must
 * be zeroed before its first forward (or cleaned with moe_plan_reset_counters):
 * the streaming GEMMs hand out work from four counters that must read zero
 * when they start, and the multi-workgroup planner takes only words tagged
 * with the current launch's epoch from its exchange area, which a zeroed area
 * never holds.  Every complete forward leaves both clean.  A forward that
 * finds them dirty reports MOE_STATUS_DIRTY_COUNTERS or MOE_STATUS_STALLED
 * and the next forward is clean again.  The multi-workgroup planner (fixed
 * routes, or T > 32 with logits) assumes its workgroups (at most one per CU)
 * become resident together: a kernel of another stream that holds CUs for
 * its whole duration makes it report MOE_STATUS_STALLED instead of hanging. */
int moe_plan_create(moe_plan **out, const moe_desc *d);
/* Enqueue one forward on `stream` (hipStream_t; NULL = default stream).
 * No host sync and no allocation; T == 0 launches nothing. */
int moe_plan_run(moe_plan *p, void *stream);
/* Synchronise `stream` and read the device status bits (MOE_STATUS_*). */
int moe_plan_read_status(moe_plan *p, void *stream, uint32_t *flags);
/* Enqueue a kernel that zeroes the work counters and the planner's published
 * per-workgroup counts (capturable: a kernel node, not a memset).  No counterpart in the reference, whose Triton
 * GEMMs use a static grid; for C-ABI callers that reuse workspace memory. */
int moe_plan_reset_counters(moe_plan *p, void *stream);
/* Enqueue launch `stage` (0 <= stage < layout.launches) of one forward alone:
 * per-kernel timing, as the reference's per-stage graphs
 * (moe_benchmark.py:258-282).  Stages read what earlier stages wrote. */
int moe_plan_run_stage(moe_plan *p, int32_t stage, void *stream);
int moe_plan_layout(const moe_plan *p, moe_layout *out);

/* One forward that allocates nothing.  No counterpart in the reference: for
 * callers that cannot call hipMalloc (code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation).  `d` is as for
 * moe_plan_create except that d->workspace and d->workspace_bytes are
 * ignored: the workspace is a static device array of
 * MOE_STATIC_WORKSPACE_BYTES per GPU, held until the process ends.  Shapes
 * whose moe_workspace_layout().total exceeds it fail with MOE_ESPACE (Qwen3
 * E128/H2048/I768/K8: T <= 370).  Enqueues a counter-reset kernel and the
 * forward's launches on `stream`; no plan object, no host sync.  All calls on
 * one GPU share the array: calls that overlap on one GPU (different streams,
 * or host threads, without ordering) race, and the workspace arrays read
 * back after a call hold that call's values only until the next one. */
#define MOE_STATIC_WORKSPACE_BYTES (16u << 20)
int moe_forward_static(const moe_desc *d, void *stream);
void moe_plan_destroy(moe_plan *p);

/* ---- W4G128 weights (host functions, no GPU needed) ------------------------
 * Reference v1 format (moe_weight_quant.py:1-7): words [E, N, K/8] uint32,
 * word j = nibbles (q + 8) of K = 8j..8j+7, low nibble first; scales
 * [E, N, K/128] bf16.  K % 128 == 0, N % 16 == 0 for tiling. */
int moe_w4_quantize(const uint16_t *weight_bf16, int32_t E, int32_t N, int32_t K,
                    uint32_t *words, uint16_t *scales);
/* v1 -> tiled layout read by the GPU kernels:
 *   words_t [E][N/16][K/128][64 lanes][4] uint32: lane l holds row l%16 and
 *     the four 8-K chunks (l/16)*8 + 32*j (j = 0..3) of the 128-K group;
 *   scales_t [E][N/16][K/128][16] bf16. */
size_t moe_w4_tiled_words_bytes(int32_t E, int32_t N, int32_t K);
size_t moe_w4_tiled_scales_bytes(int32_t E, int32_t N, int32_t K);
int moe_w4_tile(const uint32_t *words, const uint16_t *scales, int32_t E, int32_t N, int32_t K,
                uint32_t *words_t, uint16_t *scales_t);
/* GPU: expand tiled W4 into bf16 [E, N, K] with the GEMM's own decode. */
int moe_w4_dequantize(const void *words_t, const void *scales_t, int32_t E, int32_t N,
                      int32_t K, void *out_bf16, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* MOE_MI355X_H */
