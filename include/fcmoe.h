/*
 * fcmoe.h -- C ABI of the MI355X (gfx950) fused-MoE library libfcmoe.so.
 *
 * The reference (hearth-stone/fused_cpp) exposes its fused MoE only through
 * pybind modules (`fused_cpp._moe_C`, `fused_cpp._C`); it states that it has
 * no standalone C ABI (docs/public_contracts.md:16-19). These entry points are
 * the seam a binding would use instead of those pybind functions; each one
 * names the reference function it replaces. All pointers are DEVICE pointers
 * unless stated otherwise; all work is enqueued on `stream` (no host
 * synchronisation); every function returns 0 on success or a negative
 * FCMOE_E* code, with a message available from fcmoe_last_error().
 *
 * Element formats: bf16 values travel as uint16_t bit patterns; topk ids are
 * int32 or int64 (ids_is_i64); routing weights are fp32.
 */
#ifndef FCMOE_H_
#define FCMOE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* hipStream_t;

#define FCMOE_OK 0
#define FCMOE_EINVAL -1   /* bad shape, dtype or argument */
#define FCMOE_ESPACE -2   /* workspace too small */
#define FCMOE_EDEVICE -3  /* HIP runtime error */

/* Activation codes (src/fused_cpp/moe/bf16_tiled.py:227-260). */
#define FCMOE_ACT_SILU 0
#define FCMOE_ACT_GELU 1
#define FCMOE_ACT_SWIGLUOAI 2
#define FCMOE_ACT_SILU_CLAMP10 3

/* Thread-local message of the last failed call ("" if none). */
const char* fcmoe_last_error(void);
/* ABI version (bumped on incompatible change). */
int fcmoe_abi_version(void);

/* ---- weight preparation ------------------------------------------------ */

/* Per-output-channel symmetric int8 quantisation of bf16 weights [rows, cols]:
 * scale = max|w|/127 (1 if 0), q = rint(w/scale) clamped to +-127.
 * Replaces the quantize lambda of fused_moe_w8a8_tiled_prepare_weights
 * (csrc/moe/arm/i8mm_w8a8/kernels.cpp:446-461). */
int fcmoe_quantize_weight_rows(const uint16_t* w, int64_t rows, int64_t cols, int8_t* q, float* scales,
                               hipStream_t stream);

/* Bytes of one packed expert for a [n, k] weight of elem_bytes (1: int8,
 * 2: bf16) split into n_groups equal channel groups (2 for gate/up W13, 1 for
 * W2); each group is padded to 16 channels, k to 64 bytes. */
int64_t fcmoe_packed_expert_bytes(int elem_bytes, int64_t n, int64_t k, int n_groups);

/* Pack [experts, n, k] weights into the MFMA operand layout (16-channel x
 * 64-byte tiles, lane order). Replaces pack_expert_weights
 * (csrc/moe/arm/i8mm_w8a8/kernels.cpp:70-98) and the BF16 packers
 * (csrc/moe/arm/common/fused_moe_bf16_tiled.cpp:6125-6209). dst holds
 * experts * fcmoe_packed_expert_bytes(...) bytes. */
int fcmoe_pack_experts(const void* src, int elem_bytes, int64_t experts, int64_t n, int64_t k, int n_groups,
                       void* dst, hipStream_t stream);

/* ---- routing ------------------------------------------------------------ */

/* Per-expert route lists in ascending flat-route order (route r = t*kt + s,
 * kt = top_k + (shared_id >= 0)); slot top_k is the appended shared expert.
 * Replaces the route build of csrc/moe/arm/i8mm_w8a8/kernels.cpp:583-592 and
 * csrc/moe/arm/common/fused_moe_bf16_tiled.cpp:6454-6483. Outputs (device):
 * counts [experts], offsets [experts+1], sorted_routes [tokens*kt] (first
 * offsets[experts] valid), invalid_count [1] (the number of ids outside
 * [0, experts); written, so it needs no zeroing beforehand).
 * workspace: fcmoe_route_workspace_bytes(). */
size_t fcmoe_route_workspace_bytes(int64_t tokens, int64_t top_k, int64_t experts, int64_t shared_id);
int fcmoe_route_build(const void* topk_ids, int ids_is_i64, int64_t tokens, int64_t top_k, int64_t experts,
                      int64_t shared_id, int32_t* counts, int32_t* offsets, int32_t* sorted_routes,
                      int32_t* invalid_count, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Per-row dynamic int8 activation quantisation of bf16 rows [rows, cols] into
 * q [rows, ldq] (columns cols..ldq-1 zeroed) and scales [rows].
 * rounding 0: quantize_bf16_row (x*(1/s), half away from zero;
 * csrc/moe/arm/i8mm_w8a8/kernels.cpp:211-228); rounding 1: i8gemm
 * (x/s, ties to even, clamp [-128,127]; csrc/i8gemm.cpp:368-392).
 * x_is_f32 selects fp32 input rows (rounding 1 only). */
int fcmoe_quantize_rows(const void* x, int x_is_f32, int64_t rows, int64_t cols, int rounding, int8_t* q,
                        int64_t ldq, float* scales, hipStream_t stream);

/* Top-k softmax router (the caller step before the MoE op; the reference
 * receives ids/weights from vLLM: src/fused_cpp/moe/bf16_tiled.py:676-681,
 * docs/vllm_bf16_tiled_moe_integration.md:75-87). logits [tokens, experts]
 * fp32 -> topk_ids [tokens, top_k] (int64 if ids_is_i64 else int32, in
 * descending logit order, lower id first on ties) and topk_weights
 * [tokens, top_k] fp32 = softmax prob (/ sum of the selected probs if
 * renormalize) * scale. experts <= 1024, top_k <= min(experts, 64). */
int fcmoe_router_topk(const float* logits, int64_t tokens, int64_t experts, int64_t top_k, int renormalize,
                      float scale, void* topk_ids, int ids_is_i64, float* topk_weights, hipStream_t stream);

/* ---- fused MoE forward -------------------------------------------------- */

typedef struct fcmoe_moe_args {
  /* activations */
  const uint16_t* x;          /* [tokens, hidden] bf16 */
  int64_t tokens;
  int64_t hidden;             /* H */
  int64_t inter;              /* F (per-expert intermediate) */
  /* routing */
  const void* topk_ids;       /* [tokens, top_k] int32/int64; may be NULL if top_k == 0 */
  int ids_is_i64;
  const float* topk_weights;  /* [tokens, top_k] fp32 */
  int64_t top_k;
  int64_t experts;            /* prepared experts (incl. an appended shared expert) */
  int64_t valid_experts;      /* ids must be < this (global_num_experts, or experts) */
  int64_t shared_expert_id;   /* -1: none; else appended slot with weight 1.0 */
  float routed_scaling;       /* multiplies topk_weights when a shared expert is appended */
  /* weights: packed by fcmoe_pack_experts (W13 with n_groups = 2) */
  const void* w13;
  const void* w2;
  const float* w13_scale;     /* W8A8: [experts, 2F] */
  const float* w2_scale;      /* W8A8: [experts, H] */
  const float* w13_bias;      /* BF16: optional [experts, 2F] */
  const float* w2_bias;       /* BF16: optional [experts, H] */
  int activation;             /* BF16: FCMOE_ACT_*; W8A8: must be FCMOE_ACT_SILU_CLAMP10 */
  int skip_weighted;          /* BF16 only, requires top_k == 1 and no shared expert */
  /* output */
  uint16_t* out;              /* [tokens, hidden] bf16 */
  int32_t* invalid_count;     /* optional device int32 [1]: set to the number of invalid ids */
  void* workspace;
  size_t workspace_bytes;
} fcmoe_moe_args;

/* W8A8 dynamic-per-token INT8 fused MoE with clamped SwiGLU (limit 10).
 * Replaces fused_moe_w8a8_tiled_async_plan_v2
 * (csrc/moe/arm/i8mm_w8a8/kernels.cpp:463-694) behind
 * fused_moe_w8a8_tiled{,_async_plan,_with_shared}
 * (src/fused_cpp/moe/bf16_tiled.py:964-1043, 1450-1573). */
size_t fcmoe_w8a8_workspace_bytes(const fcmoe_moe_args* args);
int fcmoe_w8a8_forward(const fcmoe_moe_args* args, hipStream_t stream);

/* W8A8 forward that allocates nothing. No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * arguments and results as fcmoe_w8a8_forward; args->workspace and
 * args->workspace_bytes are ignored. Its workspace is a fixed per-GPU device
 * array of FCMOE_NOALLOC_SCRATCH_BYTES bytes (held until the process ends),
 * so calls with fcmoe_w8a8_workspace_bytes(args) above that size fail with
 * FCMOE_ESPACE (at H = 7168, F = 2048, top-8 + shared: up to ~200 tokens).
 * Every call on one GPU shares that array: calls that overlap on one GPU
 * (different streams, or host threads) race and must be serialised by the
 * caller. Tile classes of a GEMM stage run in order on `stream`; no side
 * streams or events are created. */
#define FCMOE_NOALLOC_SCRATCH_BYTES (64ll << 20)
int fcmoe_w8a8_forward_noalloc(const fcmoe_moe_args* args, hipStream_t stream);

/* BF16 fused MoE (bf16 MFMA, fp32 accumulation, bf16 intermediate, fp32 route
 * rows, top-k merge). Replaces fused_moe_bf16_tiled
 * (csrc/moe/arm/common/fused_moe_bf16_tiled.cpp:6376-7218) behind
 * fused_moe_bf16_tiled{,_with_shared} and, with top_k = 0 and a shared expert
 * id of 0, shared_mlp_bf16_tiled (fused_moe_bf16_tiled.cpp:10307-10455;
 * bf16_tiled.py:676-878, 1805-1873). */
size_t fcmoe_bf16_workspace_bytes(const fcmoe_moe_args* args);
int fcmoe_bf16_forward(const fcmoe_moe_args* args, hipStream_t stream);

/* W8A16 fused MoE (src/fused_cpp/moe/bf16_tiled.py:1309-1447; native W8A16
 * executor csrc/moe/arm/common/fused_moe_bf16_tiled.cpp:6211-6288): bf16
 * activations, int8 weights packed by fcmoe_pack_experts (elem_bytes 1,
 * the W8A8 layout) with fp32 per-output-channel scales w13_scale [E, 2F] and
 * w2_scale [E, H]. Products accumulate in fp32 on bf16 MFMA (int8 weights are
 * exact in bf16); the channel scale multiplies the accumulator. Activation
 * SILU, GELU or SILU_CLAMP10; no biases. Routing, intermediate (bf16) and
 * combine as fcmoe_bf16_forward. Weight streaming runs 16/32-row tiles. */
size_t fcmoe_w8a16_workspace_bytes(const fcmoe_moe_args* args);
int fcmoe_w8a16_forward(const fcmoe_moe_args* args, hipStream_t stream);

/* ---- i8gemm ------------------------------------------------------------- */

/* Dynamic per-row W8A8 linear: quantise x [m, k] (bf16 or fp32) per row
 * (ties to even), int32 GEMM with w packed by fcmoe_pack_experts (1 expert,
 * n_groups 1), out = (float)acc * x_scale * w_scale[n] (+ bias[n]) stored as
 * bf16 (out_is_bf16) or fp32 [m, n]. Replaces i8gemm_dynamic_scaled_mm
 * (csrc/i8gemm.cpp:318-452) behind i8gemm.dynamic_scaled_mm
 * (src/fused_cpp/i8gemm.py:88-137). Workspace: fcmoe_i8gemm_workspace_bytes(m,
 * k, n): it includes the K splits' int32 partial sums (splits x m x n; none
 * when one split covers K), so it depends on n; above 256 rows the split
 * count also depends on the current device's CU count, so query it with the
 * device current that the call will run on (a smaller workspace is refused
 * with FCMOE_ESPACE). */
size_t fcmoe_i8gemm_workspace_bytes(int64_t m, int64_t k, int64_t n);
int fcmoe_i8gemm(const void* x, int x_is_f32, int64_t m, int64_t k, const void* w_packed, const float* w_scale,
                 int64_t n, const float* bias, void* out, int out_is_bf16, void* workspace, size_t workspace_bytes,
                 hipStream_t stream);

/* Two bf16-output GEMMs of one bf16 input [m, k] sharing a single per-row
 * activation quantisation (ties to even; scale = max|x|/127): out1 [m, n1]
 * and out2 [m, n2], no bias. Replaces i8gemm_dynamic_scaled_mm_pair
 * (csrc/i8gemm.cpp:453-570) behind i8gemm.dynamic_scaled_mm_pair
 * (src/fused_cpp/i8gemm.py:151-189). Workspace: fcmoe_i8gemm_pair_workspace_bytes
 * (room for the larger of the two GEMMs' partial sums; they run one after
 * the other on `stream`). */
size_t fcmoe_i8gemm_pair_workspace_bytes(int64_t m, int64_t k, int64_t n1, int64_t n2);
int fcmoe_i8gemm_pair(const uint16_t* x, int64_t m, int64_t k, const void* w1_packed, const float* w1_scale,
                      int64_t n1, const void* w2_packed, const float* w2_scale, int64_t n2, uint16_t* out1,
                      uint16_t* out2, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ---- diagnostics (stage-level parity checks) ---------------------------- */

/* Grouped int8 GEMM returning raw int32 accumulators: for each expert e and
 * each j < counts[e], acc[offsets[e] + j, :] = a[row_map ? row_map[pos] : pos]
 * . w[e]^T with w packed (n_groups = 1, [n, k] int8), a int8 with row stride
 * lda (a multiple of 64, zero padded). acc has n columns. With a row_map, the
 * rows it addresses must lie within the first 2 GiB of a. Used to show the
 * int32 accumulators equal an exact integer GEMM bit for bit. */
int fcmoe_grouped_gemm_i8_acc(const int8_t* a, int64_t lda, const int32_t* row_map, const int32_t* counts,
                              const int32_t* offsets, int64_t experts, int64_t total_rows, const void* w_packed,
                              int64_t n, int64_t k, int32_t* acc, void* workspace, size_t workspace_bytes,
                              hipStream_t stream);
size_t fcmoe_grouped_gemm_workspace_bytes(int64_t experts, int64_t total_rows);

/* Copies of the W8A8 stage buffers from the last fcmoe_w8a8_forward that used
 * `workspace` (device pointers into it, valid until the workspace is reused):
 * sorted routes [R], y [R, ldy] bf16, q2 [R, ldq] int8, s2row [R],
 * route_out [R, hidden] fp32 (indexed by flat route). NULL args are skipped. */
int fcmoe_w8a8_stage_views(const fcmoe_moe_args* args, const int32_t** sorted_routes, const uint16_t** y,
                           int64_t* ldy, const int8_t** q2, int64_t* ldq, const float** s2row,
                           const float** route_out);

/* The same for the last fcmoe_bf16_forward (w8a16 = 0) or fcmoe_w8a16_forward
 * (w8a16 = 1) that used `workspace`: route_pos [R] (flat route -> sorted
 * position, -1 for a dropped route), route_weight [R] (the combined weight
 * each route row is merged with: routed weight x routed_scaling, 1.0 for the
 * shared slot) and route_out [R, hidden] fp32 (the W2 rows the top-k merge of
 * csrc/moe/arm/sve_bf16/route_merge.cpp:47-126 reads). A dense shared MLP
 * (top_k 0, one expert, shared id 0) of at most 256 tokens runs no route
 * build: its route_pos and route_weight views are then not written. */
int fcmoe_bf16_stage_views(const fcmoe_moe_args* args, int w8a16, const int32_t** route_pos,
                           const float** route_weight, const float** route_out);

/* W8A8 prefill launch plan for the route scan's tile counts per class
 * (class_tiles[0..3]: tiles of 16 / 128 / 192 / 256 rows), as the device
 * chooses it inside fcmoe_w8a8_forward (same environment overrides): returns
 * 0 = classic (one launch per class), 1 = mixed (persistent MFMA launch
 * beside the 16-row streaming launch), 2 = partitioned classic (the 256-row
 * class on *part_wgs_out CUs); a negative FCMOE_E* code on bad arguments.
 * No reference counterpart (the reference's CPU planner makes no such
 * choice); for benchmarks and tests that attribute stage times. */
int fcmoe_w8a8_prefill_plan(const int32_t* class_tiles, int* part_wgs_out);

/* ---- stage timing ------------------------------------------------------ */

/* Stage ids for fcmoe_stage_timing_read. W13 / W2 class stages are per tile
 * class c (BM = 16, 32, 64, 128, 192, 256 for c = 0..5). W8A8 prefill
 * records the launches of both launch plans (the classic per-class launches
 * and the mixed plan's persistent MFMA and 16-row streaming launches); the
 * plan not chosen on the device exits at once and records a few
 * microseconds. */
#define FCMOE_STAGE_ROUTE 0
#define FCMOE_STAGE_QUANT 1
#define FCMOE_STAGE_REQUANT 2
#define FCMOE_STAGE_ACT 3
#define FCMOE_STAGE_COMBINE 4
#define FCMOE_STAGE_W13_CLASS0 8
#define FCMOE_STAGE_W13_MIXED_MFMA 14
#define FCMOE_STAGE_W13_MIXED_STREAM 15
#define FCMOE_STAGE_W2_CLASS0 16
#define FCMOE_STAGE_W2_MIXED_MFMA 22
#define FCMOE_STAGE_W2_MIXED_STREAM 23
#define FCMOE_STAGE_COUNT 24

/* Per-stage GPU timing with hipEvents recorded on the launch stream around
 * each stage of fcmoe_w8a8_forward / fcmoe_bf16_forward / fcmoe_w8a16_forward
 * (fcmoe_i8gemm and _pair record their row quantisation as
 * FCMOE_STAGE_QUANT and each GEMM launch under the W13 class of its tile
 * rows): the device-side
 * counterpart of the reference's FUSED_CPP_MOE_STAGE_TIMING stderr timers
 * (csrc/moe/arm/common/fused_moe_bf16_tiled.cpp:6446, 7122-7131).
 * enable != 0 starts recording (the environment variable
 * FUSED_CPP_MOE_STAGE_TIMING=1 enables it at load). _read synchronises on the
 * recorded events, writes total milliseconds and launch counts per stage id
 * (arrays of FCMOE_STAGE_COUNT) and clears the records. */
int fcmoe_stage_timing_enable(int enable);
int fcmoe_stage_timing_read(double* total_ms, int64_t* launches);

#ifdef __cplusplus
}
#endif

#endif /* FCMOE_H_ */
