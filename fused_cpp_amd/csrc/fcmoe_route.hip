// fcmoe_route.hip -- top-k route build on the GPU.
//
// Semantics (bit-exact target): for every expert, the list of flat routes
// r = t*kt + s routed to it, in ascending r. This is the order in which the
// reference builds its per-expert route vectors
// (csrc/moe/arm/i8mm_w8a8/kernels.cpp:583-592,
//  csrc/moe/arm/common/fused_moe_bf16_tiled.cpp:6454-6483). Slot s == top_k is
// the appended shared expert with weight 1.0 and the routed weights are scaled
// by routed_scaling_factor (src/fused_cpp/moe/bf16_tiled.py:1007-1013).
//
// Three launches, all O(routes):
//   1. count:   per 256-route chunk, an LDS histogram over experts (the
//               W8A8 token rows are quantised by extra workgroups of this
//               launch).
//   2. scan:    one block: per-expert exclusive scan over chunks, exclusive
//               scan over experts (offsets), and the per-tile-class work lists
//               for the grouped GEMMs (the tokens-per-expert tile selector).
//   3. scatter: per chunk, the in-chunk rank of each route among earlier
//               routes of the same expert gives its stable sorted position.
#include <utility>

#include "fcmoe_device.h"
#include "fcmoe_internal.h"
#include "fcmoe_quant_row.h"

namespace fcmoe {

namespace {

constexpr int kScanThreads = 1024;
constexpr int kMaxExperts = 1024;
static_assert(kMaxExperts == kScanThreads, "the single-workgroup route kernel gives each expert a thread");

struct RouteArgs {
  const void* ids;
  int ids_is_i64;
  const float* topk_w;
  int64_t tokens;
  int top_k;
  int kt;
  int experts;        // total prepared experts (histogram width)
  int valid_experts;  // routed ids must be < this
  int shared_id;      // -1 none
  float scale;
  int scale_routed;
};

// Block 0 of a route launch zeroes the work-queue counters the GEMM launches
// after it use.
__device__ __forceinline__ void zero_queues(int32_t* queues) {
  if (queues && blockIdx.x == 0 && threadIdx.x < kRouteQueues) queues[threadIdx.x] = 0;
}

__device__ __forceinline__ int route_expert(const RouteArgs& a, int64_t r, bool* valid) {
  const int64_t t = r / a.kt;
  const int s = (int)(r - t * a.kt);
  if (s >= a.top_k) {
    *valid = true;
    return a.shared_id;
  }
  const int64_t idx = t * a.top_k + s;
  int64_t e = a.ids_is_i64 ? ((const int64_t*)a.ids)[idx] : (int64_t)((const int32_t*)a.ids)[idx];
  *valid = e >= 0 && e < a.valid_experts;
  return *valid ? (int)e : -1;
}

// Combined weight of flat route r: the routed slots carry topk_w (times the
// routed scale when asked), the appended shared slot carries 1.
__device__ __forceinline__ float route_weight_of(const RouteArgs& a, int64_t r) {
  const int64_t t = r / a.kt;
  const int s = (int)(r - t * a.kt);
  float w = 1.0f;
  if (s < a.top_k) {
    w = a.topk_w ? a.topk_w[t * a.top_k + s] : 1.0f;
    if (a.scale_routed) w = w * a.scale;
  }
  return w;
}

// Invalid ids are counted per chunk (chunk_invalid, plain stores) and summed
// by the scan kernel, which writes the total: the caller's counter needs no
// zeroing launch beforehand.
__device__ __forceinline__ void route_count_body(const RouteArgs& a, int64_t routes, int32_t* chunk_hist,
                                                 float* route_weight, int32_t* chunk_invalid) {
  extern __shared__ int32_t hist[];
  __shared__ int32_t n_invalid;
  const int tid = threadIdx.x;
  for (int e = tid; e < a.experts; e += kRouteChunk) hist[e] = 0;
  if (tid == 0) n_invalid = 0;
  __syncthreads();
  const int64_t r = (int64_t)blockIdx.x * kRouteChunk + tid;
  if (r < routes) {
    bool valid;
    const int e = route_expert(a, r, &valid);
    route_weight[r] = route_weight_of(a, r);
    if (valid)
      atomicAdd(&hist[e], 1);
    else
      atomicAdd(&n_invalid, 1);
  }
  __syncthreads();
  if (tid == 0) chunk_invalid[blockIdx.x] = n_invalid;
  int32_t* dst = chunk_hist + (int64_t)blockIdx.x * a.experts;
  for (int e = tid; e < a.experts; e += kRouteChunk) dst[e] = hist[e];
}

__global__ __launch_bounds__(kRouteChunk) void route_count_kernel(RouteArgs a, int64_t routes, int32_t* chunk_hist,
                                                                   float* route_weight, int32_t* chunk_invalid) {
  route_count_body(a, routes, chunk_hist, route_weight, chunk_invalid);
}

struct ClassArgs {
  int n;
  int bm[kMaxClasses];
  int64_t bound[kMaxClasses];
};

// Block-wide exclusive scan over 1024 threads; returns the total in *total.
__device__ int block_exclusive_scan(int v, int* total) {
  __shared__ int wave_tot[kScanThreads / kWave];
  const int lane = threadIdx.x % kWave;
  const int wid = threadIdx.x / kWave;
  int incl = v;
  for (int o = 1; o < kWave; o <<= 1) {
    int n = __shfl_up(incl, o);
    if (lane >= o) incl += n;
  }
  if (lane == kWave - 1) wave_tot[wid] = incl;
  __syncthreads();
  int base = 0, all = 0;
  for (int w = 0; w < kScanThreads / kWave; ++w) {
    int x = wave_tot[w];
    if (w < wid) base += x;
    all += x;
  }
  __syncthreads();
  *total = all;
  return base + incl - v;
}

// Appends this expert's (expert, m_begin) tiles to the list of the smallest
// class whose BM covers its row count (the last class splits larger experts).
// Called by all 1024 threads of the block (contains block scans).
__device__ void emit_tiles(int count, int e, const ClassArgs& cls, int32_t* tiles, int32_t* tile_count) {
  int my_class = -1;
  if (count > 0) {
    my_class = cls.n - 1;
    for (int c = 0; c < cls.n; ++c) {
      if (count <= cls.bm[c]) {
        my_class = c;
        break;
      }
    }
  }
  int64_t class_base = 0;
  for (int c = 0; c < cls.n; ++c) {
    const int nt = (my_class == c) ? (count + cls.bm[c] - 1) / cls.bm[c] : 0;
    int ctotal;
    const int base = block_exclusive_scan(nt, &ctotal);
    int32_t* list = tiles + class_base * 2;
    for (int j = 0; j < nt; ++j) {
      if (base + j < cls.bound[c]) {
        list[(base + j) * 2] = e;
        list[(base + j) * 2 + 1] = j * cls.bm[c];
      }
    }
    if (threadIdx.x == 0) tile_count[c] = ctotal < cls.bound[c] ? ctotal : (int)cls.bound[c];
    class_base += cls.bound[c];
  }
}

// Tile lists from per-expert counts already on the device (single expert
// GEMMs and the accumulator diagnostic).
__global__ __launch_bounds__(kScanThreads) void tiles_from_counts_kernel(const int32_t* counts, int experts,
                                                                          ClassArgs cls, int32_t* tiles,
                                                                          int32_t* tile_count) {
  const int e = threadIdx.x;
  emit_tiles(e < experts ? counts[e] : 0, e, cls, tiles, tile_count);
}

// Column scan of chunk_hist [chunks][experts]: entry (c, e) becomes the
// number of expert-e routes in chunks before c. The chunks of each expert are
// split into segments over all threads (thread tid: expert tid % experts,
// segment tid / experts); a segment is summed, the segment sums are scanned in
// LDS, and the segment is rewritten from its base. Loads go out kScanBatch at
// a time, so the walk costs chunks / (segments * kScanBatch) memory round trips
// instead of one per chunk.
constexpr int kScanBatch = 16;

__device__ __forceinline__ void route_scan_body(int experts, int64_t chunks, int32_t* chunk_hist, int32_t* counts,
                                                int32_t* offsets, const ClassArgs& cls, int32_t* tiles,
                                                int32_t* tile_count, const int32_t* chunk_invalid, int32_t* invalid) {
  __shared__ int seg_sum[kScanThreads];
  const int tid = threadIdx.x;
  {
    int v = 0;
    for (int64_t c = tid; c < chunks; c += kScanThreads) v += chunk_invalid[c];
    int total;
    block_exclusive_scan(v, &total);
    if (tid == 0) store_count(invalid, total);
  }
  const int segs = kScanThreads / experts;  // >= 1: experts <= kScanThreads
  const int e = tid % experts, sg = tid / experts;
  const bool active = sg < segs;
  const int64_t len = (chunks + segs - 1) / segs;
  const int64_t c0 = active ? sg * len : 0;
  const int64_t c1 = active ? (c0 + len < chunks ? c0 + len : chunks) : 0;
  int32_t* col = chunk_hist + c0 * experts + e;  // this segment's first entry
  const int n = c1 > c0 ? (int)(c1 - c0) : 0;  // trailing segments may be empty
  const int full = n - n % kScanBatch;

  int sum = 0;
  {
    const int32_t* q = col;
    for (int c = 0; c < full; c += kScanBatch, q += kScanBatch * experts) {
      int v[kScanBatch];
#pragma unroll
      for (int u = 0; u < kScanBatch; ++u) v[u] = q[u * experts];
#pragma unroll
      for (int u = 0; u < kScanBatch; ++u) sum += v[u];
    }
    for (int c = full; c < n; ++c, q += experts) sum += *q;
  }
  seg_sum[tid] = sum;
  __syncthreads();
  int running = 0, count = 0;
  if (active) {
    for (int q = 0; q < segs; ++q) {
      const int w = seg_sum[q * experts + e];
      if (q < sg) running += w;
      count += w;
    }
  }
  {
    int32_t* q = col;
    for (int c = 0; c < full; c += kScanBatch, q += kScanBatch * experts) {
      int v[kScanBatch];
#pragma unroll
      for (int u = 0; u < kScanBatch; ++u) v[u] = q[u * experts];
#pragma unroll
      for (int u = 0; u < kScanBatch; ++u) {
        q[u * experts] = running;
        running += v[u];
      }
    }
    for (int c = full; c < n; ++c, q += experts) {
      const int v = *q;
      *q = running;
      running += v;
    }
  }
  // threads 0 .. experts-1 (segment 0) carry their expert's total
  const bool owner = tid < experts;
  if (owner) counts[e] = count;
  int total;
  const int off = block_exclusive_scan(owner ? count : 0, &total);
  if (owner) offsets[e] = off;
  if (tid == 0) offsets[experts] = total;
  emit_tiles(owner ? count : 0, tid, cls, tiles, tile_count);
}

__global__ __launch_bounds__(kScanThreads) void route_scan_kernel(int experts, int64_t chunks, int32_t* chunk_hist,
                                                                   int32_t* counts, int32_t* offsets,
                                                                   ClassArgs cls, int32_t* tiles,
                                                                   int32_t* tile_count, const int32_t* chunk_invalid,
                                                                   int32_t* invalid) {
  route_scan_body(experts, chunks, chunk_hist, counts, offsets, cls, tiles, tile_count, chunk_invalid, invalid);
}

__global__ __launch_bounds__(kRouteChunk) void route_scatter_kernel(RouteArgs a, int64_t routes,
                                                                     const int32_t* chunk_hist,
                                                                     const int32_t* offsets, int32_t* sorted_routes,
                                                                     int32_t* row_token, int32_t* route_pos,
                                                                     int32_t* queues) {
  __shared__ __attribute__((aligned(16))) int32_t ex[kRouteChunk];
  const int tid = threadIdx.x;
  zero_queues(queues);
  const int64_t r = (int64_t)blockIdx.x * kRouteChunk + tid;
  int e = -1;
  if (r < routes) {
    bool valid;
    e = route_expert(a, r, &valid);
  }
  ex[tid] = e;
  __syncthreads();
  if (r >= routes) return;
  if (e < 0) {
    route_pos[r] = -1;
    return;
  }
  // stable rank within the chunk: earlier routes of the same expert, four
  // list entries per LDS read
  int rank = 0;
  const int4* ex4 = (const int4*)ex;
  int j = 0;
  for (; j + 4 <= tid; j += 4) {
    const int4 q = ex4[j / 4];
    rank += (q.x == e) + (q.y == e) + (q.z == e) + (q.w == e);
  }
  for (; j < tid; ++j) rank += ex[j] == e;
  const int pos = offsets[e] + chunk_hist[(int64_t)blockIdx.x * a.experts + e] + rank;
  sorted_routes[pos] = (int32_t)r;
  row_token[pos] = (int32_t)(r / a.kt);
  route_pos[r] = pos;
}

// Decode-sized routing (routes <= kScanThreads) in one workgroup, one route
// per thread: LDS histogram, the expert scan and tile lists, then the stable
// scatter, where a route's rank is the number of earlier routes of its expert
// (a scan of the LDS expert list, four entries per read). Produces exactly
// the outputs of the count / scan / scatter kernels.
struct RouteOut {
  int32_t* counts;
  int32_t* offsets;
  int32_t* tiles;
  int32_t* tile_count;
  int32_t* sorted_routes;
  int32_t* row_token;
  int32_t* route_pos;
  float* route_weight;
  int32_t* invalid;
  int32_t* queues;
};

__device__ __forceinline__ void route_small_body(const RouteArgs& a, int routes, const ClassArgs& cls,
                                                 const RouteOut& o) {
  int32_t* counts = o.counts;
  int32_t* offsets = o.offsets;
  int32_t* tiles = o.tiles;
  int32_t* tile_count = o.tile_count;
  int32_t* sorted_routes = o.sorted_routes;
  int32_t* row_token = o.row_token;
  int32_t* route_pos = o.route_pos;
  float* route_weight = o.route_weight;
  int32_t* invalid = o.invalid;
  __shared__ int32_t hist[kMaxExperts];
  __shared__ __attribute__((aligned(16))) int32_t ex[kScanThreads];
  __shared__ int32_t n_invalid;
  const int tid = threadIdx.x;
  hist[tid] = 0;  // kMaxExperts == kScanThreads
  if (tid == 0) n_invalid = 0;
  int e = -1;
  if (tid < routes) {
    bool valid;
    e = route_expert(a, tid, &valid);
    route_weight[tid] = route_weight_of(a, tid);
  }
  ex[tid] = e;  // -1: invalid or past the last route
  __syncthreads();
  if (tid < routes) {
    if (e >= 0)
      atomicAdd(&hist[e], 1);
    else
      atomicAdd(&n_invalid, 1);
  }
  __syncthreads();
  if (tid == 0) store_count(invalid, n_invalid);  // the count is written, not accumulated
  const bool owner = tid < a.experts;
  const int count = owner ? hist[tid] : 0;
  int total;
  const int off = block_exclusive_scan(count, &total);
  if (owner) {
    counts[tid] = count;
    offsets[tid] = off;
  }
  if (tid == 0) offsets[a.experts] = total;
  emit_tiles(count, tid, cls, tiles, tile_count);
  __syncthreads();  // every thread has read its hist entry
  if (owner) hist[tid] = off;
  __syncthreads();
  if (tid >= routes) return;
  if (e < 0) {
    route_pos[tid] = -1;
    return;
  }
  int rank = 0;
  const int4* ex4 = (const int4*)ex;
  int j = 0;
  for (; j + 4 <= tid; j += 4) {
    const int4 q = ex4[j / 4];
    rank += (q.x == e) + (q.y == e) + (q.z == e) + (q.w == e);
  }
  for (; j < tid; ++j) rank += ex[j] == e;
  const int pos = hist[e] + rank;
  sorted_routes[pos] = tid;
  row_token[pos] = tid / a.kt;
  route_pos[tid] = pos;
}

__global__ __launch_bounds__(kScanThreads) void route_small_kernel(RouteArgs a, int routes, ClassArgs cls,
                                                                   RouteOut o) {
  zero_queues(o.queues);
  route_small_body(a, routes, cls, o);
}

// Small-batch front end in one launch: workgroup 0 builds the routes as
// route_small_kernel; workgroup b >= 1 quantises token rows 4 (b - 1) ..
// 4 (b - 1) + 3, kRowThreads threads per row (quant_row_wg). The two jobs
// are independent (the token rows do not depend on the routing), so they
// share a launch instead of running back to back.
constexpr int kQuantRowsPerGroup = kScanThreads / kRowThreads;

// Workgroup b >= 1 of a shared launch: token rows 4 (b - 1) .. 4 (b - 1) + 3.
template <int CAP>
__device__ __forceinline__ void quant_row_group(const QuantRows& qr) {
  __shared__ float wmax[kScanThreads / kWave];
  const int g = threadIdx.x / kRowThreads;
  const int64_t row = (int64_t)(blockIdx.x - 1) * kQuantRowsPerGroup + g;
  quant_row_wg<CAP>(qr.x, qr.cols, qr.rounding, qr.q, qr.ldq, qr.scales, row, row < qr.rows,
                    (int)threadIdx.x % kRowThreads, wmax + g * (kRowThreads / kWave));
}

template <int CAP>
__global__ __launch_bounds__(kScanThreads) void route_quant_small_kernel(RouteArgs a, int routes, ClassArgs cls,
                                                                         RouteOut o, QuantRows qr) {
  if (blockIdx.x == 0) {
    zero_queues(o.queues);
    route_small_body(a, routes, cls, o);
    return;
  }
  quant_row_group<CAP>(qr);
}

// Larger routings: the token rows are quantised by extra workgroups of the
// count launch (one row per kRowThreads-thread workgroup), so the column scan,
// a single latency-bound workgroup, runs with the memory system to itself
// (beside the quantisation it took C4's route from ~40 to ~72 us).
static_assert(kRouteChunk == kRowThreads, "count workgroups and row workgroups share the launch's block size");
template <int CAP>
__global__ __launch_bounds__(kRouteChunk) void route_count_quant_kernel(RouteArgs a, int64_t routes, int64_t chunks,
                                                                         int32_t* chunk_hist, float* route_weight,
                                                                         int32_t* chunk_invalid, QuantRows qr) {
  if ((int64_t)blockIdx.x < chunks) {
    route_count_body(a, routes, chunk_hist, route_weight, chunk_invalid);
    return;
  }
  __shared__ float wmax[kRowThreads / kWave];
  const int64_t row = (int64_t)blockIdx.x - chunks;
  quant_row_wg<CAP>(qr.x, qr.cols, qr.rounding, qr.q, qr.ldq, qr.scales, row, true, (int)threadIdx.x, wmax);
}

// 16-byte units per thread when kRowThreads threads quantise one row of
// `quant` (1, 2, 4 or 8), or 0 when the rows do not qualify for a shared
// launch (the caller then runs quant_rows_launch).
int quant_cap(const QuantRows* quant) {
  if (!quant || quant->rows <= 0 || quant->cols % 8 || quant->ldq % 8 || quant->rows > (int64_t)INT32_MAX / 2)
    return 0;
  const int64_t pt = ceil_div(quant->cols / 8, kRowThreads);
  return pt <= 1 ? 1 : pt <= 2 ? 2 : pt <= 4 ? 4 : pt <= 8 ? 8 : 0;
}

// Calls launch(std::integral_constant<int, cap>) for cap in {1, 2, 4, 8}.
template <typename F>
void with_cap(int cap, F&& launch) {
  switch (cap) {
    case 1: launch(std::integral_constant<int, 1>{}); break;
    case 2: launch(std::integral_constant<int, 2>{}); break;
    case 4: launch(std::integral_constant<int, 4>{}); break;
    default: launch(std::integral_constant<int, 8>{}); break;
  }
}

ClassArgs class_args(const TileClasses& tc) {
  ClassArgs ca;
  ca.n = tc.n;
  for (int c = 0; c < kMaxClasses; ++c) {
    ca.bm[c] = tc.bm[c];
    ca.bound[c] = tc.bound[c];
  }
  return ca;
}

}  // namespace

int tiles_from_counts_launch(const int32_t* counts, int64_t experts, const TileClasses& tc, int32_t* tiles,
                             int32_t* tile_count, hipStream_t stream) {
  if (experts <= 0 || experts > kMaxExperts) return fail(FCMOE_EINVAL, "experts must be in [1, 1024]");
  hipLaunchKernelGGL(tiles_from_counts_kernel, dim3(1), dim3(kScanThreads), 0, stream, counts, (int)experts,
                     class_args(tc), tiles, tile_count);
  return check_launch("tiles_from_counts");
}

TileClasses make_tile_classes(const int* bms, int n, int64_t routes, int64_t experts) {
  TileClasses tc;
  tc.n = n;
  for (int c = 0; c < n; ++c) {
    tc.bm[c] = bms[c];
    // Experts in class c have more than bm[c-1] rows (class 0: at least one).
    const int64_t lower = c == 0 ? 1 : (int64_t)bms[c - 1] + 1;
    int64_t ex = routes / lower;
    if (ex > experts) ex = experts;
    int64_t bound = ex;
    if (c == n - 1) bound = ex + ceil_div(routes, bms[c]);  // multi-tile experts
    tc.bound[c] = bound > 0 ? bound : 1;
  }
  return tc;
}

void route_take(Arena& ar, RouteBuffers& rb, int64_t routes, int64_t experts, const TileClasses& tc) {
  const int64_t chunks = ceil_div(routes, kRouteChunk);
  rb.chunk_hist = ar.take<int32_t>(chunks * experts);
  rb.chunk_invalid = ar.take<int32_t>(chunks);
  rb.counts = ar.take<int32_t>(experts);
  rb.offsets = ar.take<int32_t>(experts + 1);
  rb.sorted_routes = ar.take<int32_t>(routes);
  rb.row_token = ar.take<int32_t>(routes);
  rb.route_pos = ar.take<int32_t>(routes);
  rb.route_weight = ar.take<float>(routes);
  int64_t tiles = 0;
  for (int c = 0; c < tc.n; ++c) tiles += tc.bound[c];
  rb.tiles = ar.take<int32_t>(2 * tiles);
  rb.tile_count = ar.take<int32_t>(kMaxClasses);
  rb.invalid = ar.take<int32_t>(1);
  rb.queues = ar.take<int32_t>(kRouteQueues);
}

int route_launch(const void* ids, int ids_is_i64, const float* topk_w, int64_t tokens, int64_t top_k,
                 int64_t experts, int64_t valid_experts, int64_t shared_id, float routed_scale, bool scale_routed,
                 const RouteBuffers& rb, const TileClasses& tc, int32_t* invalid_out, hipStream_t stream,
                 const QuantRows* quant, bool* quant_done) {
  if (quant_done) *quant_done = false;
  if (experts <= 0 || experts > kMaxExperts) return fail(FCMOE_EINVAL, "experts must be in [1, 1024]");
  const int64_t kt = top_k + (shared_id >= 0 ? 1 : 0);
  const int64_t routes = tokens * kt;
  if (routes <= 0) return FCMOE_OK;
  if (routes > INT32_MAX / 2) return fail(FCMOE_EINVAL, "too many routes");
  RouteArgs a;
  a.ids = ids;
  a.ids_is_i64 = ids_is_i64;
  a.topk_w = topk_w;
  a.tokens = tokens;
  a.top_k = (int)top_k;
  a.kt = (int)kt;
  a.experts = (int)experts;
  a.valid_experts = (int)valid_experts;
  a.shared_id = (int)shared_id;
  a.scale = routed_scale;
  a.scale_routed = scale_routed ? 1 : 0;
  const int64_t chunks = ceil_div(routes, kRouteChunk);
  int32_t* invalid = invalid_out ? invalid_out : rb.invalid;
  const ClassArgs ca = class_args(tc);
  if (routes <= kScanThreads) {
    const RouteOut o{rb.counts,    rb.offsets,   rb.tiles,        rb.tile_count, rb.sorted_routes,
                     rb.row_token, rb.route_pos, rb.route_weight, invalid,      rb.queues};
    if (const int cap = quant_done ? quant_cap(quant) : 0) {
      const dim3 grid((unsigned)(1 + ceil_div(quant->rows, kQuantRowsPerGroup))), block(kScanThreads);
      with_cap(cap, [&](auto c) {
        hipLaunchKernelGGL(route_quant_small_kernel<decltype(c)::value>, grid, block, 0, stream, a, (int)routes, ca,
                           o, *quant);
      });
      *quant_done = true;
      return check_launch("route_quant");
    }
    hipLaunchKernelGGL(route_small_kernel, dim3(1), dim3(kScanThreads), 0, stream, a, (int)routes, ca, o);
    return check_launch("route");
  }
  if (const int cap = quant_done ? quant_cap(quant) : 0) {
    with_cap(cap, [&](auto c) {
      hipLaunchKernelGGL(route_count_quant_kernel<decltype(c)::value>, dim3((unsigned)(chunks + quant->rows)),
                         dim3(kRouteChunk), experts * sizeof(int32_t), stream, a, routes, chunks, rb.chunk_hist,
                         rb.route_weight, rb.chunk_invalid, *quant);
    });
    *quant_done = true;
  } else {
    hipLaunchKernelGGL(route_count_kernel, dim3((unsigned)chunks), dim3(kRouteChunk), experts * sizeof(int32_t),
                       stream, a, routes, rb.chunk_hist, rb.route_weight, rb.chunk_invalid);
  }
  hipLaunchKernelGGL(route_scan_kernel, dim3(1), dim3(kScanThreads), 0, stream, (int)experts, chunks, rb.chunk_hist,
                     rb.counts, rb.offsets, ca, rb.tiles, rb.tile_count, rb.chunk_invalid, invalid);
  hipLaunchKernelGGL(route_scatter_kernel, dim3((unsigned)chunks), dim3(kRouteChunk), 0, stream, a, routes,
                     rb.chunk_hist, rb.offsets, rb.sorted_routes, rb.row_token, rb.route_pos, rb.queues);
  return check_launch("route");
}

}  // namespace fcmoe
