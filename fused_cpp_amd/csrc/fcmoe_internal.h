// fcmoe_internal.h -- host-side declarations shared by the libfcmoe sources.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/fcmoe.h"

namespace fcmoe {

// Thread-local error message plumbing for fcmoe_last_error().
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);

// Bump allocator over a caller-provided workspace; 256-byte aligned slices.
struct Arena {
  char* base = nullptr;
  size_t cap = 0;
  size_t used = 0;
  template <typename T>
  T* take(int64_t count) {
    size_t bytes = (size_t)(count > 0 ? count : 1) * sizeof(T);
    size_t off = (used + 255) & ~(size_t)255;
    used = off + bytes;
    return base ? reinterpret_cast<T*>(base + off) : nullptr;
  }
  bool ok() const { return base == nullptr || used <= cap; }
};

// ---- routing (fcmoe_route.hip) ----
// Tile classes: experts are assigned to the smallest class whose BM covers
// their row count (the last class takes the rest, in several M tiles).
constexpr int kMaxClasses = 6;
struct TileClasses {
  int n = 0;
  int bm[kMaxClasses] = {0};
  int64_t bound[kMaxClasses] = {0};  // max tiles a class can receive
};
TileClasses make_tile_classes(const int* bms, int n, int64_t routes, int64_t experts);

struct RouteBuffers {
  int32_t* chunk_hist = nullptr;     // [chunks, experts]
  int32_t* chunk_invalid = nullptr;  // [chunks] invalid ids per chunk (multi-kernel path)
  int32_t* counts = nullptr;         // [experts]
  int32_t* offsets = nullptr;        // [experts + 1]
  int32_t* sorted_routes = nullptr;  // [routes]  sorted position -> flat route
  int32_t* row_token = nullptr;      // [routes]  sorted position -> token
  int32_t* route_pos = nullptr;      // [routes]  flat route -> sorted position (-1 invalid)
  float* route_weight = nullptr;     // [routes]  combined routing weight
  int32_t* tiles = nullptr;          // [classes][bound][2] (expert, m_begin)
  int32_t* tile_count = nullptr;     // [classes]
  int32_t* invalid = nullptr;        // [1]
  int32_t* queues = nullptr;         // [kRouteQueues] work-queue counters, zeroed by the route launch
};
// Work-queue counters the route launch zeroes for the GEMM launches after it
// (the mixed prefill plan's persistent launch: one per XCD and stage).
constexpr int kRouteQueues = 32;
// Routes per workgroup of the count / scatter kernels. (1024-route chunks
// shortened the column scan but left too few workgroups: C3's route stage
// went from 30 to 39 us.)
constexpr int kRouteChunk = 256;
void route_take(Arena& a, RouteBuffers& rb, int64_t routes, int64_t experts, const TileClasses& tc);
// bf16 token rows to quantise (quantize_bf16_row semantics by `rounding`,
// as quant_rows_launch): at small batch the route kernel takes this job into
// its own launch.
struct QuantRows {
  const uint16_t* x;
  int64_t rows, cols;
  int rounding;
  int8_t* q;
  int64_t ldq;
  float* scales;
};
// quant / quant_done: optional. When the rows qualify (cols % 8 == 0,
// ldq % 8 == 0, cols <= 16384), they are quantised by extra workgroups of a
// route launch (the single-workgroup small-batch routing, or the count launch
// of a larger one) and *quant_done is set; otherwise *quant_done is false and
// the caller runs quant_rows_launch.
int route_launch(const void* ids, int ids_is_i64, const float* topk_w, int64_t tokens, int64_t top_k,
                 int64_t experts, int64_t valid_experts, int64_t shared_id, float routed_scale, bool scale_routed,
                 const RouteBuffers& rb, const TileClasses& tc, int32_t* invalid_out, hipStream_t stream,
                 const QuantRows* quant = nullptr, bool* quant_done = nullptr);

int tiles_from_counts_launch(const int32_t* counts, int64_t experts, const TileClasses& tc, int32_t* tiles,
                             int32_t* tile_count, hipStream_t stream);

// ---- quantisation / packing (fcmoe_quant.hip) ----
int fill_u32_launch(uint32_t* p, int64_t n, uint32_t v, hipStream_t stream);
int quant_rows_launch(const void* x, int x_is_f32, int64_t rows, int64_t cols, int rounding, int8_t* q, int64_t ldq,
                      float* scales, hipStream_t stream);
// rowpart: [rows, parts] per-(row, 16-channel gate tile) maxima of |y| written
// by the W13 epilogue; the row scale uses their maximum.
int requant_launch(const uint16_t* y, int64_t ldy, int64_t rows, int64_t cols, const float* rowpart, int64_t parts,
                   int8_t* q, int64_t ldq, float* scales, hipStream_t stream);
int act_bf16_launch(const float* gate_up, int64_t ldg, int64_t rows, int64_t f, int64_t fp16, int mode, uint16_t* y,
                    int64_t ldy, hipStream_t stream);

// ---- grouped GEMM (fcmoe_gemm.hip) ----
enum Epilogue : int {
  kEpiRawI32 = 0,     // int8: store raw int32 accumulators
  kEpiW13SwigluI8,    // int8: clamped SwiGLU (FEXPA exp) -> bf16 y + row max
  kEpiW2RouteI8,      // int8: acc * (s_row * s_w) -> fp32 route rows
  kEpiI8Gemm,         // int8: acc * xs * ws (+bias) -> bf16 / fp32 output
  kEpiW13ActBf16,     // bf16: acc (+bias) -> activation -> bf16 y
  kEpiRawF32Bias,     // bf16: acc (+bias) -> fp32 gate_up (natural channel order)
  kEpiW2RouteBf16,    // bf16: acc (+bias) -> fp32 route rows
  kEpiW13ActW8,       // W8A16 (bf16 A, int8 B): acc * s_w -> activation -> bf16 y
  kEpiW2RouteW8,      // W8A16: acc * s_w -> fp32 route rows
};

struct GemmParams {
  const void* a;             // int8 or bf16 rows
  int64_t lda;               // row stride in elements (a multiple of 64 bytes)
  int64_t a_rows;            // rows of A the row indices may address (0: unknown, taken as < 2 GiB)
  const int32_t* row_map;    // sorted position -> A row (NULL: identity)
  const int32_t* offsets;    // [experts+1] first sorted position of each expert
  const int32_t* counts;     // [experts]
  const int32_t* tiles;      // (expert, m_begin) pairs for this class
  const int32_t* tile_count; // number of valid tiles
  const void* w;             // packed weights
  int64_t w_expert_bytes;    // bytes per expert
  int64_t n;                 // logical output channels (W13: 2F)
  int64_t n_half;            // W13: F (channels per gate/up group); else n
  int64_t n_tiles;           // 16-channel tiles per group (padded)
  int64_t k_chunks;          // 64-byte K chunks
  int n_groups;              // 2 for gate/up W13, else 1
  // epilogue
  void* out;                 // destination
  int64_t ldo;               // row stride of out (elements)
  const float* scale_row;    // per sorted row (or per A row) scale
  const float* scale_col;    // per expert per channel scale [experts, n]
  const float* bias;         // [experts, n] (bf16 path / i8gemm)
  float* rowpart;            // W13 int8: [sorted rows, n_tiles] max |y| per 16-channel gate tile
  const int32_t* sorted_routes;  // W2: sorted position -> flat route
  int activation;            // bf16 W13
  int out_bf16;              // i8gemm output dtype
  // Persistent launch: > 0 = this many workgroups (a multiple of the XCD
  // count) loop over the items; 0 = one workgroup per item slot.
  int persist;
  // Streaming role of the 16-row class beside a persistent LDS-kernel launch
  // (4 waves per workgroup, few enough VGPRs to share each SIMD with it).
  int stream_role;
  // Launch-plan gate (W8A8 prefill; see the forward): when plan_tiles is set
  // the launch does its work only if (*plan_tiles >= plan_min and, when
  // plan_tiles2 is set, *plan_tiles2 >= plan_min2) == plan_mixed, and
  // otherwise every workgroup exits at once.
  const int32_t* plan_tiles;
  int plan_min;
  const int32_t* plan_tiles2;  // optional second count that must also reach plan_min2
  int plan_min2;
  int plan_mixed;
  // Several classes' tile lists as one item space (the persistent LDS launch
  // of the mixed plan): u_n > 0 replaces tiles / tile_count by lists
  // u_tiles[0..u_n) (largest tile class first), each run last-first.
  int u_n;
  const int32_t* u_tiles[3];
  const int32_t* u_count[3];
  // Persistent LDS launches: per-XCD item counters (8, zero at launch); a
  // workgroup takes its XCD's next item from them instead of striding.
  int32_t* queue;
  // Partitioned classic plan (W8A8 prefill). part_counts: the four class
  // tile counts of the route scan (NULL: not partitioned). When the classic
  // plan is chosen and part_wgs(part_counts) > 0, the persistent launch's
  // first part_wgs workgroups run the 256-row class (part_tiles, items from
  // part_queue) on their own CUs while the classic launches of the other
  // classes run on the rest; the classic 256-row launch (part_exit set)
  // then exits.
  const int32_t* part_counts;
  const int32_t* part_tiles;
  int32_t* part_queue;
  int part_exit;
  // i8gemm: the device's CUs (0: unknown); the 256-row launch picks its
  // workgroup width (384 or 256 channels) from the rounds of items it needs.
  int cus;
  // i8gemm split K (LDS kernel): k_total > 0 splits the k_total chunks into
  // ranges of k_chunks (grid.y = split); split s writes its raw int32 sums to
  // split_out + s * m * n ([m, n] row-major, m = split_rows), and a reduce
  // launch adds the splits and applies the epilogue.
  int64_t k_total;
  int32_t* split_out;
  int64_t split_rows;
};

// Whether a launch's plan gate lets it run (device side).
// Workgroups the partitioned classic plan gives the 256-row class (a
// multiple of the 8 XCDs; 0: not partitioned), from the class tile counts
// c[0..3] (16 / 128 / 192 / 256 rows). Each 256-row tile holds MFMA-bound
// work; each 128/192-row tile streams one expert's weights (a 16-row tile an
// eighth of that). The 256-row class gets CUs in proportion to its weighted
// share, 2.5 : 1, within [32, 128]; when it would need more than 128 (or has
// no tiles) the classic launches share every CU instead.
__host__ __device__ __forceinline__ int part_wgs(const int32_t* c) {
  const int64_t t3 = 20 * (int64_t)c[3], ts = 8 * ((int64_t)c[1] + c[2]) + c[0];
  if (t3 == 0) return 0;
  const int64_t w = 256 * t3 / (t3 + ts) / 8 * 8;
  return w > 128 ? 0 : (w < 32 ? 32 : (int)w);
}

__device__ __forceinline__ bool plan_open(const GemmParams& p) {
  if (!p.plan_tiles) return true;
  const bool mixed = *p.plan_tiles >= p.plan_min && (!p.plan_tiles2 || *p.plan_tiles2 >= p.plan_min2);
  if (mixed != (p.plan_mixed != 0)) return false;
  return !(p.part_exit && part_wgs(p.part_counts) > 0);
}

int gemm_launch(int epi, int bm, const GemmParams& p, int64_t max_tiles, hipStream_t stream);

// i8gemm at few rows (fcmoe_gemm_smallm.hip): m <= kSmallMRows, all rows per
// wave, weights read once, K split over about one workgroup per CU.
// smallm_splits: the K splits for a shape (0 outside the domain);
// smallm_workspace_bytes: the splits' int32 partial sums (0 with one split).
constexpr int64_t kSmallMRows = 256;
int64_t smallm_splits(int64_t m, int64_t k, int64_t n);
// Adds splits x [m, n] int32 partial sums in split order and applies the
// i8gemm epilogue (write_scaled_output) into out [m, n].
int i8gemm_reduce_launch(const int32_t* partial, int64_t splits, int64_t m, int64_t n, const float* scale_row,
                         const float* scale_col, const float* bias, void* out, int out_bf16, hipStream_t stream);
size_t smallm_workspace_bytes(int64_t m, int64_t k, int64_t n);
int smallm_i8gemm_launch(const int8_t* a, int64_t lda, int64_t m, int64_t k, const void* w_packed,
                         const float* scale_row, const float* scale_col, int64_t n, const float* bias, void* out,
                         int out_bf16, int32_t* partial, size_t partial_bytes, hipStream_t stream);
// The i8gemm pair at few rows: both GEMMs of the same quantised rows in one
// launch (bf16 outputs, no bias), then a reduce per GEMM with more than one
// split; the partial sums of the two sit back to back in `partial`.
// (one split count for both: about one workgroup per CU over the two)
int64_t smallm_pair_splits(int64_t m, int64_t k, int64_t n1, int64_t n2);
size_t smallm_pair_workspace_bytes(int64_t m, int64_t k, int64_t n1, int64_t n2);
int smallm_i8gemm_pair_launch(const int8_t* a, int64_t lda, int64_t m, int64_t k, const float* scale_row,
                              const void* w1, const float* sc1, int64_t n1, uint16_t* out1, const void* w2,
                              const float* sc2, int64_t n2, uint16_t* out2, int32_t* partial, size_t partial_bytes,
                              hipStream_t stream);
// The BF16 dense MLP at few rows on the same kernel: W13 (out_row null: the
// activation store into y, bf16 [m, ldo]) or W2 (the fp32 route store into
// out at row out_row[r]). k_chunks: 64-byte K chunks; weights packed bf16
// with n_groups groups of n_half channels.
struct SmallMBf16 {
  const void* a;           // bf16 rows
  int64_t lda_bytes;
  int64_t a_rows;          // rows A may address
  const int32_t* row_map;  // product row r reads A row row_map[r] (null: r)
  int64_t m, k_chunks;
  const void* w;
  int64_t n_groups, n_half;
  const float* bias;
  void* out;
  int64_t ldo;
  const int32_t* out_row;
  int activation;
  float* partial;
  size_t partial_bytes;
  const int32_t* m_dev;    // rows actually routed (device), at most m; null: m
  // W2 with one route per token (merge_out set): the reduce launch also does
  // the merge of that one route, out[t] = bf16(fma(row, weight, 0)) (or the
  // row itself with skip_weighted; 0 for a dropped route), so no combine
  // launch follows. Product row route_pos[t] is token t's route row (null:
  // row t, weight 1: the dense shared MLP, which runs no route build and
  // whose merge launch also zeroes invalid_count when that is set).
  uint16_t* merge_out;
  const int32_t* route_pos;
  const float* route_weight;
  int64_t tokens;
  int skip_weighted;
  int32_t* invalid_count;
};
int64_t smallm_bf16_splits(int64_t m, int64_t k_chunks, int64_t tiles);
int smallm_bf16_launch(const SmallMBf16& q, hipStream_t stream);
// LDS-staged kernel for bm in {128, 192, 256} (fcmoe_gemm_lds.hip); gemm_launch
// dispatches to it unless FCMOE_GEMM_LDS=0.
int gemm_lds_launch(int epi, int bm, const GemmParams& p, int64_t max_tiles, hipStream_t stream);
// A bytes the LDS-staged kernel can address (32-bit buffer offsets).
constexpr int64_t kLdsMaxABytes = 0x7ffffff0;

// ---- combine (fcmoe_combine.hip) ----
int combine_launch(const float* route_out, const float* route_weight, const int32_t* route_pos, int64_t tokens,
                   int64_t kt, int64_t hidden, int tree, int skip_weighted, uint16_t* out, hipStream_t stream);

// ---- W8A8 decode tail (fcmoe_decode_tail.hip) ----
// requant + W2 + ordered merge in one launch for batches of a token or two;
// writes out and the q2 / s2row / route_out views as the unfused path does.
constexpr int kDecodeTailSlots = 16;  // slots per token (top_k + shared) it supports
struct DecodeTailArgs {
  int64_t tokens;
  int kt, top_k, shared_id, ids_is_i64;
  const void* ids;             // [tokens, top_k]
  const int32_t* route_pos;    // [tokens * kt] flat route -> sorted position (-1 dropped)
  const float* route_weight;   // [tokens * kt]
  const uint16_t* y;           // [positions, ldy] bf16 intermediate
  int64_t ldy;
  const float* rowpart;        // [positions, parts] W13 tile maxima of |y|
  int64_t parts;               // ceil(inter / 16), at most 128
  int64_t inter;               // I
  const void* w;               // packed W2 [E][ceil(H/16) tiles][k_chunks][1 KB]
  int64_t w_expert_bytes;
  int64_t k_chunks;            // ldq / 64
  const float* scale_col;      // [E, hidden]
  int64_t hidden;
  int8_t* q2;                  // [positions, ldq] (view)
  int64_t ldq;
  float* s2row;                // [positions] (view)
  float* route_out;            // [tokens * kt, hidden] (view)
  uint16_t* out;               // [tokens, hidden] bf16
};
int decode_tail_launch(const DecodeTailArgs& a, hipStream_t stream);
// One-token head: route + token-row quantisation + W13 in one launch; writes
// y, rowpart and the route metadata (route_pos, route_weight, sorted_routes,
// row_token, the invalid count) as the route and W13 launches do.
constexpr int64_t kDecodeHeadMaxK = 8192;  // padded hidden size it takes (the row lives in LDS)
struct DecodeHeadArgs {
  int kt, top_k, shared_id, ids_is_i64, valid_experts, scale_routed;
  float scale;
  const void* ids;           // [top_k] the token's ids
  const float* topk_w;       // [top_k] or null (weights 1)
  const uint16_t* x;         // [hidden] bf16 token row
  int64_t hidden;
  const void* w;             // packed W13 [E][2 groups][n_tiles][k_chunks][1 KB]
  int64_t w_expert_bytes;
  int64_t k_chunks;          // hp / 64
  int64_t n_tiles;           // ceil(inter / 16)
  int64_t inter;
  const float* scale_col;    // [E, 2 inter]
  uint16_t* y;               // [positions, ldy]
  int64_t ldy;
  float* rowpart;            // [positions, n_tiles]
  float* xs;                 // [1] the token row's scale
  int32_t* route_pos;        // [kt]
  float* route_weight;       // [kt]
  int32_t* sorted_routes;    // [kt]
  int32_t* row_token;        // [kt]
  int32_t* invalid;          // [1]
};
int decode_head_launch(const DecodeHeadArgs& a, hipStream_t stream);

}  // namespace fcmoe
