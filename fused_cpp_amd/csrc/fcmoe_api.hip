// fcmoe_api.hip -- the C ABI (include/fcmoe.h): argument validation,
// workspace layout and the launch sequence of each fused operator.
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

#include "fcmoe_device.h"
#include "fcmoe_internal.h"

namespace fcmoe {

namespace {
thread_local std::string g_error;

// Tile rows of the grouped GEMM classes (the tokens-per-expert selector): an
// expert with c routed rows runs in the smallest class of the forward's class
// set with BM >= c; larger experts (the shared expert at prefill) are split
// into tiles of the last class. Every tile size the kernels provide; the
// index of a size here is its stage-timing slot. i8gemm and the diagnostic
// grouped GEMM use all six.
constexpr int kClassBM[] = {16, 32, 64, 128, 192, 256};
constexpr int kI8ClassBM[] = {256};  // i8gemm above kSmallMRows rows
constexpr int kNumClasses = 6;
// Decode: when an expert averages at most this many routed rows, everything
// (the shared expert too, in several 16-row tiles) runs in the single BM=16
// class: one launch per GEMM stage, no empty class launches, and weight
// streaming is the only cost (a multi-tile expert re-reads its weights from
// L2 / Infinity Cache, not HBM, since its tiles run side by side).
constexpr int kDecodeRowsPerExpert = 8;

// Stage-timing slot of a class: the index of its BM in kClassBM, so a stage
// is named by its tile rows whatever class set the forward uses.
int class_slot(int bm) {
  for (int i = 0; i < kNumClasses; ++i)
    if (kClassBM[i] == bm) return i;
  return kNumClasses - 1;
}

// Prefill (W8A8 and BF16): experts of 17-128 rows take the LDS-staged
// 128-row tile rather than the register-ring 32/64-row tiles. Their weights
// are read once either way, and the staged tile streams them faster with one
// class launch fewer per stage. Measured on the DSv3 W8A8 layer: T=1024
// 2.41 -> 2.17 ms, T=2048 2.63 -> 2.36, C3 3.27 -> 3.19, C4 4.68 -> 4.66;
// BF16 at T=512 / 4096 unchanged. Keeping either the 32- or the 64-row class
// made C3 slower (3.32 / 3.37 ms).
constexpr int kPrefillClassBM[] = {16, 128, 192, 256};
constexpr int kNumPrefillClasses = 4;

// Few rows in all (a dense MLP or i8gemm at decode batch sizes, a small MoE
// batch): the 16-row class, whose one- or eight-wave workgroups spread the
// weight stream over every CU. A larger class would give one workgroup per
// channel block and row tile, e.g. 8 for the DSv3 shared MLP at 64 rows on
// the 128-row tile; the 16-row tiles of one expert re-read its weights, which
// the tiles running side by side find in L2 / Infinity Cache.
// FCMOE_SMALL_ROWS overrides the bound (read on every call).
int64_t small_rows() {
  const char* v = getenv("FCMOE_SMALL_ROWS");
  return v && v[0] ? atoll(v) : 64;
}

bool decode_rows(int64_t routes, int64_t experts) {
  return routes <= kDecodeRowsPerExpert * experts || routes <= small_rows();
}

TileClasses select_classes(int64_t routes, int64_t experts) {
  if (decode_rows(routes, experts)) return make_tile_classes(kClassBM, 1, routes, experts);
  return make_tile_classes(kPrefillClassBM, kNumPrefillClasses, routes, experts);
}

struct W8A8Layout {
  int64_t kt, routes, hp, ip;
  TileClasses tc;
  RouteBuffers rb;
  int8_t* xq;
  float* xs;
  uint16_t* y;
  int8_t* q2;
  float* s2row;
  float* rowpart;  // [routes, ceil(F/16)] per gate-tile max |y| from the W13 epilogue
  float* route_out;
};

struct Bf16Layout {
  int64_t kt, routes, hp, ip, gu_ld;
  TileClasses tc;
  RouteBuffers rb;
  uint16_t* xpad;
  uint16_t* y;
  float* gate_up;
  float* route_out;
  float* partial = nullptr;  // small-M GEMMs' partial sums (smallm_mlp)
  size_t partial_bytes = 0;
};

int64_t tile_offset(const TileClasses& tc, int c) {
  int64_t off = 0;
  for (int i = 0; i < c; ++i) off += tc.bound[i];
  return off;
}

int check_shapes(const fcmoe_moe_args* a) {
  if (!a) return fail(FCMOE_EINVAL, "args is NULL");
  if (a->tokens < 0 || a->hidden <= 0 || a->inter <= 0) return fail(FCMOE_EINVAL, "bad tokens/hidden/inter");
  if (a->top_k < 0 || (a->top_k == 0 && a->shared_expert_id < 0)) return fail(FCMOE_EINVAL, "top_k must be positive");
  if (a->experts <= 0 || a->experts > 1024) return fail(FCMOE_EINVAL, "experts must be in [1, 1024]");
  if (a->valid_experts <= 0 || a->valid_experts > a->experts) return fail(FCMOE_EINVAL, "bad valid_experts");
  if (a->shared_expert_id >= a->experts) return fail(FCMOE_EINVAL, "shared_expert_id out of range");
  if (a->tokens > (int64_t)1 << 24) return fail(FCMOE_EINVAL, "tokens must be <= 2^24");
  return FCMOE_OK;
}

int check_common(const fcmoe_moe_args* a) {
  int rc = check_shapes(a);
  if (rc) return rc;
  if (a->tokens > 0 && (!a->x || !a->out || !a->w13 || !a->w2)) return fail(FCMOE_EINVAL, "NULL tensor");
  if (a->tokens > 0 && a->top_k > 0 && (!a->topk_ids || !a->topk_weights)) return fail(FCMOE_EINVAL, "NULL topk");
  return FCMOE_OK;
}

W8A8Layout w8a8_layout(const fcmoe_moe_args* a, Arena& ar) {
  W8A8Layout L;
  L.kt = a->top_k + (a->shared_expert_id >= 0 ? 1 : 0);
  L.routes = a->tokens * L.kt;
  L.hp = round_up(a->hidden, 64);
  L.ip = round_up(a->inter, 64);
  L.tc = select_classes(L.routes, a->experts);
  route_take(ar, L.rb, L.routes, a->experts, L.tc);
  L.xq = ar.take<int8_t>(a->tokens * L.hp);
  L.xs = ar.take<float>(a->tokens);
  L.y = ar.take<uint16_t>(L.routes * L.ip);
  L.q2 = ar.take<int8_t>(L.routes * L.ip);
  L.s2row = ar.take<float>(L.routes);
  L.rowpart = ar.take<float>(L.routes * ceil_div(a->inter, 16));
  L.route_out = ar.take<float>(L.routes * a->hidden);
  return L;
}

// BF16 and W8A16 share this layout. K is padded to the GEMM's K chunk: 32
// bf16 elements (64 bytes) for bf16 weights, 64 elements for int8 weights.
// W8A16 tile classes: 16 / 32 rows on the direct-A kernel, 128 / 192 / 256
// rows on the LDS-staged kernel (no 64-row W8A16 tile). The 192-row tile
// takes experts of 129-192 rows off the 256-row one, which ran them at half
// its rows (DSv3 shape, T = 4096 uniform: 4.63 -> 4.17 ms).
// A BF16 forward over one packed expert with at most 256 routes (the shared
// MLP, or a one-expert MoE, at decode batch sizes) runs its two GEMMs on the
// small-M kernel (fcmoe_gemm_smallm.hip): every weight byte read once, K split
// over about one workgroup per CU. The one-expert MoE and the shared MLP take
// the same path, so they stay equal bit for bit.
bool smallm_mlp(const fcmoe_moe_args* a, int64_t routes, bool w8) {
  return !w8 && a->experts == 1 && routes >= 1 && routes <= kSmallMRows && a->activation != FCMOE_ACT_SWIGLUOAI;
}

constexpr int kClassBMW8[] = {16, 32, 128, 192, 256};
constexpr int kNumClassesW8 = 5;
Bf16Layout bf16_layout(const fcmoe_moe_args* a, Arena& ar, bool w8 = false) {
  Bf16Layout L;
  const int64_t kmul = w8 ? 64 : 32;
  L.kt = a->top_k + (a->shared_expert_id >= 0 ? 1 : 0);
  L.routes = a->tokens * L.kt;
  L.hp = round_up(a->hidden, kmul);
  L.ip = round_up(a->inter, kmul);
  L.gu_ld = 2 * round_up(a->inter, 16);
  // W8A16's 128/256-row tiles run on the LDS-staged kernel, whose buffer
  // offsets are 32-bit: A and one expert's packed weights must stay under
  // 2 GiB; beyond that the forward keeps to the 16/32-row tiles.
  const bool w8_lds = a->tokens * L.hp * 2 < kLdsMaxABytes && L.routes * L.ip * 2 < kLdsMaxABytes &&
                      fcmoe_packed_expert_bytes(1, 2 * a->inter, a->hidden, 2) < kLdsMaxABytes &&
                      fcmoe_packed_expert_bytes(1, a->hidden, a->inter, 1) < kLdsMaxABytes;
  if (w8)
    L.tc = make_tile_classes(kClassBMW8,
                             decode_rows(L.routes, a->experts) ? 1 : (w8_lds ? kNumClassesW8 : 2),
                             L.routes, a->experts);
  else
    L.tc = select_classes(L.routes, a->experts);
  route_take(ar, L.rb, L.routes, a->experts, L.tc);
  L.xpad = (a->hidden % kmul) ? ar.take<uint16_t>(a->tokens * L.hp) : nullptr;
  L.y = ar.take<uint16_t>(L.routes * L.ip);
  L.gate_up = a->activation == FCMOE_ACT_SWIGLUOAI ? ar.take<float>(L.routes * L.gu_ld) : nullptr;
  L.route_out = ar.take<float>(L.routes * a->hidden);
  if (smallm_mlp(a, L.routes, w8)) {
    const int64_t kc13 = ceil_div(a->hidden * 2, 64), kc2 = ceil_div(a->inter * 2, 64);
    const int64_t p13 = smallm_bf16_splits(L.routes, kc13, 2 * ceil_div(a->inter, 16)) * 2 * a->inter;
    const int64_t p2 = smallm_bf16_splits(L.routes, kc2, ceil_div(a->hidden, 16)) * a->hidden;
    L.partial_bytes = (size_t)((p13 > p2 ? p13 : p2) * L.routes) * sizeof(float);
    L.partial = ar.take<float>(L.partial_bytes / sizeof(float));
  }
  return L;
}

// ---- stage timing: event pairs recorded around each stage launch ----
struct TimerRec {
  int stage;
  hipEvent_t a, b;
};
struct StageTimer {
  std::mutex mu;
  bool on = false;
  std::vector<TimerRec> recs;
  std::vector<hipEvent_t> pool;
  StageTimer() {
    const char* v = getenv("FUSED_CPP_MOE_STAGE_TIMING");
    on = v && v[0] && v[0] != '0';
  }
  hipEvent_t get() {
    if (!pool.empty()) {
      hipEvent_t e = pool.back();
      pool.pop_back();
      return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
  }
};
StageTimer& timer() {
  static StageTimer* t = new StageTimer();  // lives until process exit
  return *t;
}

struct Stage {
  int id;
  hipStream_t stream;
  hipEvent_t a = nullptr;
  Stage(int stage, hipStream_t s) : id(stage), stream(s) {
    StageTimer& t = timer();
    if (!t.on) return;
    std::lock_guard<std::mutex> g(t.mu);
    a = t.get();
    if (a) hipEventRecord(a, stream);
  }
  ~Stage() {
    if (!a) return;
    StageTimer& t = timer();
    std::lock_guard<std::mutex> g(t.mu);
    hipEvent_t b = t.get();
    if (!b) return;
    hipEventRecord(b, stream);
    t.recs.push_back({id, a, b});
  }
};

// ---- tile-class concurrency: the class launches of one GEMM stage are
// independent (disjoint experts), so at prefill they run on side streams
// forked from the caller's stream with events and joined back: the HBM-bound
// small-tile classes overlap the MFMA-bound 256-row class. Streams and events
// are per host thread and device (created on first use, default priority,
// kept until process exit); a stage with one class launches inline.
struct SideStreams {
  bool ready = false;
  hipStream_t s[kNumClasses] = {};
  hipEvent_t fork = nullptr;
  hipEvent_t join[kNumClasses] = {};
};
constexpr int kMaxDevices = 64;
thread_local SideStreams t_side[kMaxDevices];

int side_streams(SideStreams** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(FCMOE_EDEVICE, "hipGetDevice failed");
  SideStreams& ss = t_side[dev];
  if (!ss.ready) {
    if (hipEventCreateWithFlags(&ss.fork, hipEventDisableTiming) != hipSuccess)
      return fail(FCMOE_EDEVICE, "hipEventCreate failed");
    for (int c = 0; c < kNumClasses; ++c) {
      if (hipStreamCreateWithFlags(&ss.s[c], hipStreamNonBlocking) != hipSuccess ||
          hipEventCreateWithFlags(&ss.join[c], hipEventDisableTiming) != hipSuccess)
        return fail(FCMOE_EDEVICE, "side stream creation failed");
    }
    ss.ready = true;
  }
  *out = &ss;
  return FCMOE_OK;
}

// Launch one GEMM stage: class c runs gemm(c, stream_c). With several
// classes, the largest class (last) stays on the caller's stream and is
// launched first; the others are forked.
bool timing_on();
int persistent_wgs();

// Waits between two side streams under HIP graph capture are refused. The
// launch plans here fork from the caller's stream and join back into it
// only: every side stream waits on an event recorded on the caller's stream,
// and the caller's stream waits on each side stream's join event. A dropped
// form that also made one side stream wait on another's event ended a
// capture with a host segmentation fault in hipStreamEndCapture (its other
// changes were launches of kinds the kept plans capture without trouble);
// fork_wait refuses that edge while the caller's stream is capturing, and
// w8a8_run refuses a call that would add one before it enqueues anything.
// FCMOE_SIDE_CHAIN_WAIT=1 adds such an edge to the W8A8 prefill fork (side
// stream 1 waits for side stream 0's join event; harmless outside capture)
// so that tests can reach the refusal.
bool side_chain_wait() {
  const char* v = getenv("FCMOE_SIDE_CHAIN_WAIT");
  return v && v[0] == '1';
}

bool stream_capturing(hipStream_t stream) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(stream, &st) == hipSuccess && st == hipStreamCaptureStatusActive;
}

// `waiter` waits for `ev`, last recorded on `recorded_on`; `caller` is the
// forward's own stream.
int fork_wait(hipStream_t waiter, hipEvent_t ev, hipStream_t recorded_on, hipStream_t caller) {
  if (waiter != caller && recorded_on != caller && stream_capturing(caller))
    return fail(FCMOE_EINVAL, "a wait between two side streams is refused under HIP graph capture");
  if (hipStreamWaitEvent(waiter, ev, 0) != hipSuccess) return fail(FCMOE_EDEVICE, "stream wait failed");
  return FCMOE_OK;
}


template <typename F>
int run_classes(const TileClasses& tc, hipStream_t stream, F&& gemm, bool serial = false) {
  // Stage timing brackets each launch with events on its stream, so it runs
  // the classes one after another: each event pair then times one kernel.
  // `serial` does the same for callers that must not create streams.
  if (tc.n <= 1 || serial || timing_on()) {
    for (int c = 0; c < tc.n; ++c) {
      const int rc = gemm(c, stream);
      if (rc) return rc;
    }
    return FCMOE_OK;
  }
  SideStreams* ss = nullptr;
  int rc = side_streams(&ss);
  if (rc) return rc;
  if (hipEventRecord(ss->fork, stream) != hipSuccess) return fail(FCMOE_EDEVICE, "hipEventRecord failed");
  if ((rc = gemm(tc.n - 1, stream))) return rc;
  for (int c = tc.n - 2; c >= 0; --c) {
    if ((rc = fork_wait(ss->s[c], ss->fork, stream, stream))) return rc;
    if ((rc = gemm(c, ss->s[c]))) return rc;
    if (hipEventRecord(ss->join[c], ss->s[c]) != hipSuccess) return fail(FCMOE_EDEVICE, "hipEventRecord failed");
  }
  for (int c = tc.n - 2; c >= 0; --c)
    if ((rc = fork_wait(stream, ss->join[c], ss->s[c], stream))) return rc;
  return FCMOE_OK;
}

// Workgroups of a persistent launch: the device's CU count, rounded down to
// a multiple of the XCD count (the LDS kernel's item order keeps each item on
// the XCD of the workgroup that runs it). Cached per device.
int persistent_wgs() {
  static int cache[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  if (!cache[dev]) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 8) cus = 256;
    cache[dev] = cus / 8 * 8;
  }
  return cache[dev];
}

bool timing_on() {
  StageTimer& t = timer();
  std::lock_guard<std::mutex> g(t.mu);
  return t.on;
}

// Rows run grid-stride over y (grid.y is capped at 65535).
__global__ void pad_rows_kernel(const uint16_t* x, int64_t rows, int64_t cols, int64_t ld, uint16_t* dst) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= ld) return;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) dst[r * ld + c] = c < cols ? x[r * cols + c] : (uint16_t)0;
}

// The one expert of an i8gemm above the small-M kernel's rows: its count,
// offsets and the tile list of its one class (tiles of bm rows), in one launch.
__global__ __launch_bounds__(256) void single_expert_tiles_kernel(int32_t* counts, int32_t* offsets, int32_t* tiles,
                                                                  int32_t* tile_count, int32_t m, int32_t bm) {
  const int32_t nt = (m + bm - 1) / bm;
  for (int32_t j = blockIdx.x * blockDim.x + threadIdx.x; j < nt; j += gridDim.x * blockDim.x) {
    tiles[2 * j] = 0;
    tiles[2 * j + 1] = j * bm;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    counts[0] = m;
    offsets[0] = 0;
    offsets[1] = m;
    tile_count[0] = nt;
  }
}

}  // namespace

void set_error(const std::string& msg) { g_error = msg; }

int fail(int code, const std::string& msg) {
  g_error = msg;
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(FCMOE_EDEVICE, std::string(what) + ": " + hipGetErrorString(e));
  return FCMOE_OK;
}

}  // namespace fcmoe

using namespace fcmoe;

extern "C" const char* fcmoe_last_error(void) { return g_error.c_str(); }

extern "C" int fcmoe_abi_version(void) { return 1; }

// ---------------------------------------------------------------- routing --

extern "C" size_t fcmoe_route_workspace_bytes(int64_t tokens, int64_t top_k, int64_t experts, int64_t shared_id) {
  Arena ar;
  RouteBuffers rb;
  const int64_t routes = tokens * (top_k + (shared_id >= 0 ? 1 : 0));
  TileClasses tc = make_tile_classes(kClassBM, kNumClasses, routes, experts);
  route_take(ar, rb, routes, experts, tc);
  return ar.used + 256;
}

extern "C" int fcmoe_route_build(const void* topk_ids, int ids_is_i64, int64_t tokens, int64_t top_k,
                                 int64_t experts, int64_t shared_id, int32_t* counts, int32_t* offsets,
                                 int32_t* sorted_routes, int32_t* invalid_count, void* workspace,
                                 size_t workspace_bytes, hipStream_t stream) {
  if (tokens < 0 || top_k < 0 || experts <= 0 || experts > 1024 || shared_id >= experts)
    return fail(FCMOE_EINVAL, "route_build: bad shape");
  const int64_t kt = top_k + (shared_id >= 0 ? 1 : 0);
  const int64_t routes = tokens * kt;
  Arena ar;
  ar.base = (char*)workspace;
  ar.cap = workspace_bytes;
  RouteBuffers rb;
  TileClasses tc = make_tile_classes(kClassBM, kNumClasses, routes, experts);
  route_take(ar, rb, routes, experts, tc);
  if (!ar.ok()) return fail(FCMOE_ESPACE, "route_build: workspace too small");
  if (routes == 0) return fail(FCMOE_EINVAL, "route_build: no routes");
  int rc = route_launch(topk_ids, ids_is_i64, nullptr, tokens, top_k, experts, experts, shared_id, 1.0f, false, rb,
                        tc, nullptr, stream);
  if (rc) return rc;
  // route_launch reads topk weights only for the combine; pass a dummy-safe
  // path by copying results out.
  if (hipMemcpyAsync(counts, rb.counts, experts * sizeof(int32_t), hipMemcpyDeviceToDevice, stream) != hipSuccess ||
      hipMemcpyAsync(offsets, rb.offsets, (experts + 1) * sizeof(int32_t), hipMemcpyDeviceToDevice, stream) !=
          hipSuccess ||
      hipMemcpyAsync(sorted_routes, rb.sorted_routes, routes * sizeof(int32_t), hipMemcpyDeviceToDevice, stream) !=
          hipSuccess ||
      (invalid_count &&
       hipMemcpyAsync(invalid_count, rb.invalid, sizeof(int32_t), hipMemcpyDeviceToDevice, stream) != hipSuccess))
    return fail(FCMOE_EDEVICE, "route_build: copy failed");
  return FCMOE_OK;
}

// ------------------------------------------------------------------ W8A8 --

extern "C" size_t fcmoe_w8a8_workspace_bytes(const fcmoe_moe_args* a) {
  if (check_shapes(a)) return 0;
  Arena ar;
  w8a8_layout(a, ar);
  return ar.used + 256;
}

namespace {

// ---- W8A8 prefill: two launch plans per GEMM stage, chosen on the device.
//
// Classic plan: one launch per tile class (16 / 128 / 192 / 256 rows), the
// classes side by side on forked streams. Mixed plan: two persistent
// launches that share every CU -- the 16-row class streams its experts'
// weights from HBM on a 4-wave workgroup per CU while a persistent
// 256-row-tile launch (2 x 4 waves, at most 216 VGPRs) runs every larger
// expert's MFMA work; row fragments past an expert's rows skip their MFMAs,
// so the 128/192-row experts cost their own rows. With many experts of at
// most 16 rows beside MFMA-bound ones (skewed routing, C3: 149 such experts)
// the HBM stream hides under the MFMA work (C3 3.12 -> 2.81 ms); with few of
// them the classic plan is faster (uniform routing at T = 1024: 2.15 vs 2.30
// ms, C4 4.30 vs 5.10 ms), and so it is when there is little MFMA work beside
// them (uniform T = 256: 2.19 vs 5.43 ms -- the 4-wave streaming launch is
// tuned to sit beside MFMA workgroups, not to stream alone). The route scan's
// tile counts pick the plan: mixed when the 16-row class has at least
// kPrefillMixedMinTiles tiles and the 256-row class at least
// kPrefillMixedMinBigTiles; every launch of the other plan exits at once (no
// host round trip).
constexpr int kPrefillMixedMinTiles = 32;
constexpr int kPrefillMixedMinBigTiles = 16;

// FCMOE_PREFILL_MIXED_MIN_TILES overrides the threshold (0: always the mixed
// plan; a large value: never); read on every call so that tests can run both
// plans on one input.
int mixed_min_tiles() {
  const char* v = getenv("FCMOE_PREFILL_MIXED_MIN_TILES");
  return v && v[0] ? atoi(v) : kPrefillMixedMinTiles;
}

// Partitioned classic plan on (default) or off (FCMOE_PREFILL_PART=0, so
// that tests can compare both); read on every call.
bool part_enabled() {
  const char* v = getenv("FCMOE_PREFILL_PART");
  return !(v && v[0] == '0');
}

// Decode batches of at most this many tokens (FCMOE_DECODE_TAIL_MAX_T; 0
// turns both off) run requant, W2 and the merge as one launch (the tail), and
// a one-token batch runs route, row quantisation and W13 as one (the head).
// At one token the tail saves two launches (C2 shape: 0.082 -> 0.077 ms) and
// the head one more (0.074 ms); at two the tokens' workgroups each stream the
// shared expert's weights, and the tail is slower (0.133 -> 0.136 ms).
constexpr int kDecodeTailMaxTokens = 1;
int decode_tail_max_tokens() {
  const char* v = getenv("FCMOE_DECODE_TAIL_MAX_T");
  return v && v[0] ? atoi(v) : kDecodeTailMaxTokens;
}

// One W8A8 GEMM stage (epilogue epi, stage-timing base id stage0) over the
// prefill class set {16, 128, 192, 256}, or over any other class set with the
// classic launches only.
int run_w8a8_stage(const TileClasses& tc, const RouteBuffers& rb, int epi, const GemmParams& base, int stage0,
                   int stage_mixed, bool serial, hipStream_t stream) {
  const bool prefill = tc.n == 4 && tc.bm[0] == 16 && tc.bm[3] == 256;
  GemmParams gate = base;
  if (prefill) {
    gate.plan_tiles = rb.tile_count;  // class 0: the 16-row tiles
    gate.plan_min = mixed_min_tiles();
    if (gate.plan_min > 0) {  // a forced mixed plan (0) skips the second condition
      gate.plan_tiles2 = rb.tile_count + 3;  // class 3: the 256-row tiles
      gate.plan_min2 = kPrefillMixedMinBigTiles;
    }
    // Mixed plan. The persistent MFMA launch takes classes 256, 192, 128 (in
    // that order) as one item space; the 16-row class streams beside it.
    GemmParams pm = gate;
    pm.plan_mixed = 1;
    pm.persist = persistent_wgs();
    pm.queue = rb.queues + (stage_mixed == FCMOE_STAGE_W13_MIXED_MFMA ? 0 : 8);
    pm.u_n = 3;
    int64_t big_bound = 0;
    for (int u = 0; u < 3; ++u) {
      const int c = 3 - u;
      pm.u_tiles[u] = rb.tiles + 2 * tile_offset(tc, c);
      pm.u_count[u] = rb.tile_count + c;
      big_bound += tc.bound[c];
    }
    // Partitioned classic plan: the persistent launch also carries the
    // 256-row class for the case that the classic plan is chosen (its own
    // queue counters: 16..23 for W13, 24..31 for W2).
    const int32_t* part = gate.plan_min > 0 && part_enabled() ? rb.tile_count : nullptr;
    pm.part_counts = part;
    pm.part_tiles = rb.tiles + 2 * tile_offset(tc, 3);
    pm.part_queue = rb.queues + (stage_mixed == FCMOE_STAGE_W13_MIXED_MFMA ? 16 : 24);
    GemmParams ps = gate;
    ps.plan_mixed = 1;
    ps.persist = persistent_wgs();
    ps.stream_role = 1;
    ps.tiles = rb.tiles;
    ps.tile_count = rb.tile_count;
    // Classic-plan launch of class c.
    auto classic = [&](int c, hipStream_t s) {
      GemmParams p = gate;
      p.plan_mixed = 0;
      p.tiles = rb.tiles + 2 * tile_offset(tc, c);
      p.tile_count = rb.tile_count + c;
      if (c == 3 && part) {  // exits when the persistent launch takes this class
        p.part_counts = part;
        p.part_exit = 1;
      }
      Stage st(stage0 + class_slot(tc.bm[c]), s);
      return gemm_launch(epi, tc.bm[c], p, tc.bound[c], s);
    };
    int rc;
    if (serial || timing_on()) {
      {
        Stage st(stage_mixed, stream);
        if ((rc = gemm_launch(epi, 256, pm, big_bound, stream))) return rc;
      }
      {
        Stage st(stage_mixed + 1, stream);
        if ((rc = gemm_launch(epi, 16, ps, tc.bound[0], stream))) return rc;
      }
      for (int c = 0; c < tc.n; ++c)
        if ((rc = classic(c, stream))) return rc;
      return FCMOE_OK;
    }
    // Every launch of both plans under one fork: the mixed plan's MFMA launch
    // on the caller's stream (first, so its workgroups hold every CU before
    // the streaming ones arrive), the rest on three side streams; the plan
    // not taken exits at once, beside the one that runs. The device has 4
    // hardware queues, so launches are paired on streams such that at most
    // one of a pair has much work under either plan: the 16-row streaming
    // launch, then the classic 16-row class (the mixed plan runs the first,
    // the classic plan the second); the classic 256-row class (it exits when
    // the persistent launch takes it), then the 128-row class; the 192-row
    // class alone. (With a stream per launch, C4's 128-row launch queued
    // behind the 192-row one on a shared hardware queue.)
    SideStreams* ss = nullptr;
    if ((rc = side_streams(&ss))) return rc;
    if (hipEventRecord(ss->fork, stream) != hipSuccess) return fail(FCMOE_EDEVICE, "hipEventRecord failed");
    if ((rc = gemm_launch(epi, 256, pm, big_bound, stream))) return rc;
    const bool with_classic = gate.plan_min > 0;  // forced mixed plan: no classic launches
    constexpr int kSides = 3;
    for (int k = 0; k < kSides; ++k) {
      hipStream_t s = ss->s[k];
      if ((rc = fork_wait(s, ss->fork, stream, stream))) return rc;
      if (k == 1 && side_chain_wait() && (rc = fork_wait(s, ss->join[0], ss->s[0], stream))) return rc;
      if (k == 0) {
        if ((rc = gemm_launch(epi, 16, ps, tc.bound[0], s))) return rc;
        if (with_classic && (rc = classic(0, s))) return rc;
      } else if (with_classic) {
        if ((rc = classic(k == 1 ? 3 : 2, s))) return rc;
        if (k == 1 && (rc = classic(1, s))) return rc;
      }
      if (hipEventRecord(ss->join[k], s) != hipSuccess) return fail(FCMOE_EDEVICE, "hipEventRecord failed");
    }
    for (int k = 0; k < kSides; ++k)
      if ((rc = fork_wait(stream, ss->join[k], ss->s[k], stream))) return rc;
    return FCMOE_OK;
  }
  // Outside the prefill class set: the classic launches only.
  return run_classes(tc, stream, [&](int c, hipStream_t s) {
    GemmParams p = base;
    p.tiles = rb.tiles + 2 * tile_offset(tc, c);
    p.tile_count = rb.tile_count + c;
    Stage st(stage0 + class_slot(tc.bm[c]), s);
    return gemm_launch(epi, tc.bm[c], p, tc.bound[c], s);
  }, serial);
}

// The W8A8 forward over a given workspace. serial_classes runs the class
// launches of a GEMM stage on `stream` one after another (no side streams).
int w8a8_run(const fcmoe_moe_args* a, char* ws_base, size_t ws_bytes, bool serial_classes, hipStream_t stream) {
  int rc = check_shapes(a);
  if (rc) return rc;
  if (a->activation != FCMOE_ACT_SILU_CLAMP10)
    return fail(FCMOE_EINVAL, "W8A8 supports only clamped SwiGLU with limit 10.0");
  if (a->hidden % 16 || a->inter % 16) return fail(FCMOE_EINVAL, "W8A8 requires H and F to be multiples of 16");
  if (a->skip_weighted) return fail(FCMOE_EINVAL, "W8A8 requires weighted TopK merge");
  if ((rc = check_common(a))) return rc;
  if (!a->w13_scale || !a->w2_scale) return fail(FCMOE_EINVAL, "W8A8 scales are NULL");
  if (a->tokens == 0) return FCMOE_OK;
  if (!serial_classes && !timing_on() && side_chain_wait() && stream_capturing(stream))
    return fail(FCMOE_EINVAL, "a wait between two side streams is refused under HIP graph capture");
  Arena ar;
  ar.base = ws_base;
  ar.cap = ws_bytes;
  if (!ar.base) return fail(FCMOE_ESPACE, "workspace is NULL");
  W8A8Layout L = w8a8_layout(a, ar);
  if (!ar.ok()) return fail(FCMOE_ESPACE, "W8A8 workspace too small");
  const int64_t H = a->hidden, I = a->inter;
  const int64_t parts = ceil_div(I, 16);
  // the fused tail's whole launch domain (decode_tail_launch refuses anything
  // else), so that a larger FCMOE_DECODE_TAIL_MAX_T falls back to the unfused
  // launches instead of failing
  const bool tail = a->tokens <= decode_tail_max_tokens() && a->tokens <= 65535 && L.kt <= kDecodeTailSlots &&
                    parts <= 2 * kWave && H > 0;
  auto decode_tail = [&]() {
    // requant + W2 + merge in one launch (timed as the W2 16-row stage)
    DecodeTailArgs d{};
    d.tokens = a->tokens;
    d.kt = (int)L.kt;
    d.top_k = (int)a->top_k;
    d.shared_id = (int)a->shared_expert_id;
    d.ids_is_i64 = a->ids_is_i64;
    d.ids = a->topk_ids;
    d.route_pos = L.rb.route_pos;
    d.route_weight = L.rb.route_weight;
    d.y = L.y;
    d.ldy = L.ip;
    d.rowpart = L.rowpart;
    d.parts = parts;
    d.inter = I;
    d.w = a->w2;
    d.w_expert_bytes = fcmoe_packed_expert_bytes(1, H, I, 1);
    d.k_chunks = L.ip / 64;
    d.scale_col = a->w2_scale;
    d.hidden = H;
    d.q2 = L.q2;
    d.ldq = L.ip;
    d.s2row = L.s2row;
    d.route_out = L.route_out;
    d.out = a->out;
    Stage st(FCMOE_STAGE_W2_CLASS0 + class_slot(16), stream);
    return decode_tail_launch(d, stream);
  };
  if (tail && a->tokens == 1 && L.hp <= kDecodeHeadMaxK && ceil_div(H / 8, 64) <= 16) {
    // one token: route + row quantisation + W13 in one launch (timed as the
    // W13 16-row stage), then the tail
    DecodeHeadArgs h{};
    h.kt = (int)L.kt;
    h.top_k = (int)a->top_k;
    h.shared_id = (int)a->shared_expert_id;
    h.ids_is_i64 = a->ids_is_i64;
    h.valid_experts = (int)a->valid_experts;
    h.scale_routed = a->shared_expert_id >= 0 ? 1 : 0;
    h.scale = a->routed_scaling;
    h.ids = a->topk_ids;
    h.topk_w = a->topk_weights;
    h.x = (const uint16_t*)a->x;
    h.hidden = H;
    h.w = a->w13;
    h.w_expert_bytes = fcmoe_packed_expert_bytes(1, 2 * I, H, 2);
    h.k_chunks = L.hp / 64;
    h.n_tiles = parts;
    h.inter = I;
    h.scale_col = a->w13_scale;
    h.y = L.y;
    h.ldy = L.ip;
    h.rowpart = L.rowpart;
    h.xs = L.xs;
    h.route_pos = L.rb.route_pos;
    h.route_weight = L.rb.route_weight;
    h.sorted_routes = L.rb.sorted_routes;
    h.row_token = L.rb.row_token;
    h.invalid = a->invalid_count ? a->invalid_count : L.rb.invalid;
    {
      Stage st(FCMOE_STAGE_W13_CLASS0 + class_slot(16), stream);
      if ((rc = decode_head_launch(h, stream))) return rc;
    }
    return decode_tail();
  }

  bool quant_done = false;
  {
    // At small batch the token rows are quantised in the route launch.
    Stage st(FCMOE_STAGE_ROUTE, stream);
    const QuantRows qr{a->x, a->tokens, H, 0, L.xq, L.hp, L.xs};
    rc = route_launch(a->topk_ids, a->ids_is_i64, a->topk_weights, a->tokens, a->top_k, a->experts,
                      a->valid_experts, a->shared_expert_id, a->routed_scaling, a->shared_expert_id >= 0, L.rb, L.tc,
                      a->invalid_count, stream, &qr, &quant_done);
    if (rc) return rc;
  }
  if (!quant_done) {
    Stage st(FCMOE_STAGE_QUANT, stream);
    rc = quant_rows_launch(a->x, 0, a->tokens, H, 0, L.xq, L.hp, L.xs, stream);
    if (rc) return rc;
  }

  GemmParams g13{};
  g13.a = L.xq;
  g13.lda = L.hp;
  g13.a_rows = a->tokens;
  g13.row_map = L.rb.row_token;
  g13.offsets = L.rb.offsets;
  g13.counts = L.rb.counts;
  g13.w = a->w13;
  g13.w_expert_bytes = fcmoe_packed_expert_bytes(1, 2 * I, H, 2);
  g13.n = 2 * I;
  g13.n_half = I;
  g13.n_tiles = ceil_div(I, 16);
  g13.k_chunks = L.hp / 64;
  g13.n_groups = 2;
  g13.out = L.y;
  g13.ldo = L.ip;
  g13.scale_row = L.xs;
  g13.scale_col = a->w13_scale;
  g13.rowpart = L.rowpart;
  rc = run_w8a8_stage(L.tc, L.rb, kEpiW13SwigluI8, g13, FCMOE_STAGE_W13_CLASS0, FCMOE_STAGE_W13_MIXED_MFMA,
                      serial_classes, stream);
  if (rc) return rc;
  if (tail) return decode_tail();
  {
    Stage st(FCMOE_STAGE_REQUANT, stream);
    rc = requant_launch(L.y, L.ip, L.routes, I, L.rowpart, ceil_div(I, 16), L.q2, L.ip, L.s2row, stream);
    if (rc) return rc;
  }

  GemmParams g2{};
  g2.a = L.q2;
  g2.a_rows = L.routes;
  g2.lda = L.ip;
  g2.row_map = nullptr;
  g2.offsets = L.rb.offsets;
  g2.counts = L.rb.counts;
  g2.w = a->w2;
  g2.w_expert_bytes = fcmoe_packed_expert_bytes(1, H, I, 1);
  g2.n = H;
  g2.n_half = H;
  g2.n_tiles = ceil_div(H, 16);
  g2.k_chunks = L.ip / 64;
  g2.n_groups = 1;
  g2.out = L.route_out;
  g2.ldo = H;
  g2.scale_row = L.s2row;
  g2.scale_col = a->w2_scale;
  g2.sorted_routes = L.rb.sorted_routes;
  rc = run_w8a8_stage(L.tc, L.rb, kEpiW2RouteI8, g2, FCMOE_STAGE_W2_CLASS0, FCMOE_STAGE_W2_MIXED_MFMA,
                      serial_classes, stream);
  if (rc) return rc;
  Stage st(FCMOE_STAGE_COMBINE, stream);
  return combine_launch(L.route_out, L.rb.route_weight, L.rb.route_pos, a->tokens, L.kt, H, 0, 0, a->out, stream);
}

// Scratch of fcmoe_w8a8_forward_noalloc: one copy per GPU, held until the
// process ends. Host code never passes `scratch` itself (on the host the name
// is a stand-in, not a device address): each device's address comes from
// hipGetSymbolAddress, looked up once per device with that device current.
__device__ __align__(256) char scratch[FCMOE_NOALLOC_SCRATCH_BYTES];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_ptr(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(FCMOE_EDEVICE, "hipGetDevice failed");
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(FCMOE_EDEVICE, std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return FCMOE_OK;
}

}  // namespace

extern "C" int fcmoe_w8a8_forward(const fcmoe_moe_args* a, hipStream_t stream) {
  if (!a) return fail(FCMOE_EINVAL, "args is NULL");
  return w8a8_run(a, (char*)a->workspace, a->workspace_bytes, false, stream);
}

extern "C" int fcmoe_w8a8_forward_noalloc(const fcmoe_moe_args* a, hipStream_t stream) {
  int rc = check_shapes(a);
  if (rc) return rc;
  const size_t need = fcmoe_w8a8_workspace_bytes(a);
  if (need > (size_t)FCMOE_NOALLOC_SCRATCH_BYTES)
    return fail(FCMOE_ESPACE, "w8a8_forward_noalloc: this call needs " + std::to_string(need) +
                                  " bytes of scratch, more than the fixed " +
                                  std::to_string((size_t)FCMOE_NOALLOC_SCRATCH_BYTES) + " bytes");
  void* ws = nullptr;
  if ((rc = scratch_ptr(&ws))) return rc;
  return w8a8_run(a, (char*)ws, FCMOE_NOALLOC_SCRATCH_BYTES, true, stream);
}

extern "C" int fcmoe_w8a8_stage_views(const fcmoe_moe_args* a, const int32_t** sorted_routes, const uint16_t** y,
                                      int64_t* ldy, const int8_t** q2, int64_t* ldq, const float** s2row,
                                      const float** route_out) {
  int rc = check_common(a);
  if (rc) return rc;
  Arena ar;
  ar.base = (char*)a->workspace;
  ar.cap = a->workspace_bytes;
  W8A8Layout L = w8a8_layout(a, ar);
  if (!ar.ok() || !ar.base) return fail(FCMOE_ESPACE, "workspace too small");
  if (sorted_routes) *sorted_routes = L.rb.sorted_routes;
  if (y) *y = L.y;
  if (ldy) *ldy = L.ip;
  if (q2) *q2 = L.q2;
  if (ldq) *ldq = L.ip;
  if (s2row) *s2row = L.s2row;
  if (route_out) *route_out = L.route_out;
  return FCMOE_OK;
}

// ------------------------------------------------------------------ BF16 --

namespace {

// BF16 weights (w8 = false) or W8A16: int8 per-channel weights with fp32
// scales against bf16 activations (w8 = true). Same routing, activation and
// combine; the GEMMs differ in operand type and epilogue.
int bf16_family_forward(const fcmoe_moe_args* a, hipStream_t stream, bool w8) {
  int rc = check_shapes(a);
  if (rc) return rc;
  if (a->activation < FCMOE_ACT_SILU || a->activation > FCMOE_ACT_SILU_CLAMP10)
    return fail(FCMOE_EINVAL, "unsupported activation");
  if (w8) {
    if (a->activation == FCMOE_ACT_SWIGLUOAI) return fail(FCMOE_EINVAL, "W8A16 supports silu, gelu and silu_clamp10");
    if (a->w13_bias || a->w2_bias) return fail(FCMOE_EINVAL, "W8A16 fused MoE does not support biases");
    if (!a->w13_scale || !a->w2_scale) return fail(FCMOE_EINVAL, "W8A16 needs w13_scale and w2_scale");
  }
  const int64_t kt = a->top_k + (a->shared_expert_id >= 0 ? 1 : 0);
  if (a->skip_weighted && kt != 1) return fail(FCMOE_EINVAL, "skip_weighted is only valid when top_k == 1");
  if ((rc = check_common(a))) return rc;
  if (a->tokens == 0) return FCMOE_OK;
  Arena ar;
  ar.base = (char*)a->workspace;
  ar.cap = a->workspace_bytes;
  if (!ar.base) return fail(FCMOE_ESPACE, "workspace is NULL");
  Bf16Layout L = bf16_layout(a, ar, w8);
  if (!ar.ok()) return fail(FCMOE_ESPACE, "BF16 workspace too small");
  const int64_t kmul = w8 ? 64 : 32;
  const int64_t H = a->hidden, I = a->inter;

  // The dense shared MLP on the small-M kernel (one expert, no routed slot):
  // every token's one route is row t with weight 1, so no route build runs
  // (the route views of fcmoe_bf16_stage_views are then not written).
  const bool dense = smallm_mlp(a, L.routes, w8) && a->top_k == 0 && a->shared_expert_id == 0;
  if (!dense) {
    Stage st(FCMOE_STAGE_ROUTE, stream);
    rc = route_launch(a->topk_ids, a->ids_is_i64, a->topk_weights, a->tokens, a->top_k, a->experts,
                      a->valid_experts, a->shared_expert_id, a->routed_scaling,
                      a->shared_expert_id >= 0 && a->top_k > 0, L.rb, L.tc, a->invalid_count, stream);
    if (rc) return rc;
  }
  const uint16_t* xa = a->x;
  if (L.xpad) {
    hipLaunchKernelGGL(pad_rows_kernel, dim3((unsigned)ceil_div(L.hp, 256), (unsigned)std::min<int64_t>(a->tokens, 65535)),
                       dim3(256), 0,
                       stream, a->x, a->tokens, H, L.hp, L.xpad);
    if ((rc = check_launch("pad_rows"))) return rc;
    xa = L.xpad;
  }
  // y columns [F, ip) feed W2's zero-padded K and must be finite zeros.
  if (I % kmul) {
    rc = fill_u32_launch((uint32_t*)L.y, L.routes * L.ip / 2, 0u, stream);
    if (rc) return rc;
  }
  const bool fused = a->activation != FCMOE_ACT_SWIGLUOAI;
  if (smallm_mlp(a, L.routes, w8)) {
    SmallMBf16 q{};
    q.a = xa;
    q.lda_bytes = L.hp * 2;
    q.a_rows = a->tokens;
    q.row_map = dense ? nullptr : L.rb.row_token;
    q.m = L.routes;
    q.k_chunks = ceil_div(H * 2, 64);
    q.w = a->w13;
    q.n_groups = 2;
    q.n_half = I;
    q.bias = a->w13_bias;
    q.out = L.y;
    q.ldo = L.ip;
    q.activation = a->activation;
    q.partial = L.partial;
    q.partial_bytes = L.partial_bytes;
    q.m_dev = dense ? nullptr : L.rb.counts;  // expert 0's routed rows
    {
      Stage st(FCMOE_STAGE_W13_CLASS0 + class_slot(16), stream);
      if ((rc = smallm_bf16_launch(q, stream))) return rc;
    }
    q.a = L.y;
    q.lda_bytes = L.ip * 2;
    q.a_rows = L.routes;
    q.row_map = nullptr;
    q.k_chunks = ceil_div(I * 2, 64);
    q.w = a->w2;
    q.n_groups = 1;
    q.n_half = H;
    q.bias = a->w2_bias;
    q.out = L.route_out;
    q.ldo = H;
    q.out_row = L.rb.sorted_routes;
    if (kt == 1) {  // the W2 reduce also merges the token's one route
      q.merge_out = a->out;
      q.route_pos = dense ? nullptr : L.rb.route_pos;
      q.route_weight = dense ? nullptr : L.rb.route_weight;
      q.tokens = a->tokens;
      q.skip_weighted = a->skip_weighted;
      q.invalid_count = dense ? a->invalid_count : nullptr;
    }
    {
      Stage st(FCMOE_STAGE_W2_CLASS0 + class_slot(16), stream);
      if ((rc = smallm_bf16_launch(q, stream))) return rc;
    }
    if (kt == 1) return FCMOE_OK;
  } else {
  GemmParams g13{};
  g13.a = xa;
  g13.lda = L.hp;
  g13.a_rows = a->tokens;
  g13.row_map = L.rb.row_token;
  g13.offsets = L.rb.offsets;
  g13.counts = L.rb.counts;
  g13.w = a->w13;
  g13.w_expert_bytes = fcmoe_packed_expert_bytes(w8 ? 1 : 2, 2 * I, H, 2);
  g13.n = 2 * I;
  g13.n_half = I;
  g13.n_tiles = ceil_div(I, 16);
  g13.k_chunks = w8 ? ceil_div(H, 64) : ceil_div(H * 2, 64);
  g13.n_groups = 2;
  g13.out = fused ? (void*)L.y : (void*)L.gate_up;
  g13.ldo = fused ? L.ip : L.gu_ld;
  g13.bias = a->w13_bias;
  g13.scale_col = w8 ? a->w13_scale : nullptr;
  g13.activation = a->activation;
  const int epi13 = w8 ? kEpiW13ActW8 : (fused ? kEpiW13ActBf16 : kEpiRawF32Bias);
  rc = run_classes(L.tc, stream, [&](int c, hipStream_t s) {
    GemmParams p = g13;
    p.tiles = L.rb.tiles + 2 * tile_offset(L.tc, c);
    p.tile_count = L.rb.tile_count + c;
    Stage st(FCMOE_STAGE_W13_CLASS0 + class_slot(L.tc.bm[c]), s);
    return gemm_launch(epi13, L.tc.bm[c], p, L.tc.bound[c], s);
  });
  if (rc) return rc;
  if (!fused) {
    Stage st(FCMOE_STAGE_ACT, stream);
    rc = act_bf16_launch(L.gate_up, L.gu_ld, L.routes, I, round_up(I, 16), a->activation, L.y, L.ip, stream);
    if (rc) return rc;
  }
  GemmParams g2{};
  g2.a = L.y;
  g2.lda = L.ip;
  g2.a_rows = L.routes;
  g2.offsets = L.rb.offsets;
  g2.counts = L.rb.counts;
  g2.w = a->w2;
  g2.w_expert_bytes = fcmoe_packed_expert_bytes(w8 ? 1 : 2, H, I, 1);
  g2.n = H;
  g2.n_half = H;
  g2.n_tiles = ceil_div(H, 16);
  g2.k_chunks = w8 ? ceil_div(I, 64) : ceil_div(I * 2, 64);
  g2.n_groups = 1;
  g2.out = L.route_out;
  g2.ldo = H;
  g2.bias = a->w2_bias;
  g2.scale_col = w8 ? a->w2_scale : nullptr;
  g2.sorted_routes = L.rb.sorted_routes;
  rc = run_classes(L.tc, stream, [&](int c, hipStream_t s) {
    GemmParams p = g2;
    p.tiles = L.rb.tiles + 2 * tile_offset(L.tc, c);
    p.tile_count = L.rb.tile_count + c;
    Stage st(FCMOE_STAGE_W2_CLASS0 + class_slot(L.tc.bm[c]), s);
    return gemm_launch(w8 ? kEpiW2RouteW8 : kEpiW2RouteBf16, L.tc.bm[c], p, L.tc.bound[c], s);
  });
  if (rc) return rc;
  }
  const int tree = (kt == 2 || kt == 4 || kt == 6 || kt == 8) ? 1 : 0;
  Stage st(FCMOE_STAGE_COMBINE, stream);
  return combine_launch(L.route_out, L.rb.route_weight, L.rb.route_pos, a->tokens, kt, H, tree, a->skip_weighted,
                        a->out, stream);
}

}  // namespace

extern "C" size_t fcmoe_bf16_workspace_bytes(const fcmoe_moe_args* a) {
  if (check_shapes(a)) return 0;
  Arena ar;
  bf16_layout(a, ar);
  return ar.used + 256;
}

extern "C" int fcmoe_bf16_forward(const fcmoe_moe_args* a, hipStream_t stream) {
  return bf16_family_forward(a, stream, false);
}

extern "C" size_t fcmoe_w8a16_workspace_bytes(const fcmoe_moe_args* a) {
  if (check_shapes(a)) return 0;
  Arena ar;
  bf16_layout(a, ar, true);
  return ar.used + 256;
}

extern "C" int fcmoe_w8a16_forward(const fcmoe_moe_args* a, hipStream_t stream) {
  return bf16_family_forward(a, stream, true);
}

extern "C" int fcmoe_bf16_stage_views(const fcmoe_moe_args* a, int w8a16, const int32_t** route_pos,
                                      const float** route_weight, const float** route_out) {
  int rc = check_common(a);
  if (rc) return rc;
  Arena ar;
  ar.base = (char*)a->workspace;
  ar.cap = a->workspace_bytes;
  Bf16Layout L = bf16_layout(a, ar, w8a16 != 0);
  if (!ar.ok() || !ar.base) return fail(FCMOE_ESPACE, "workspace too small");
  if (route_pos) *route_pos = L.rb.route_pos;
  if (route_weight) *route_weight = L.rb.route_weight;
  if (route_out) *route_out = L.route_out;
  return FCMOE_OK;
}

// ---------------------------------------------------------------- i8gemm --

namespace {
struct I8Layout {
  int64_t m;
  int64_t kp;
  TileClasses tc;
  int8_t* xq;
  float* xs;
  int32_t* counts;
  int32_t* offsets;
  int32_t* tiles;
  int32_t* tile_count;
  int32_t* partial;  // small-M K splits' partial sums (empty with one split)
  size_t partial_bytes;
};
// partial_bytes: room for the small-M GEMMs' partial sums (the largest of the
// GEMMs that run on this layout)
I8Layout i8_layout(int64_t m, int64_t k, size_t partial_bytes, Arena& ar) {
  I8Layout L;
  L.m = m;
  L.kp = round_up(k, 64);
  // above the small-M kernel's rows the one expert takes 256-row tiles (the
  // 192-row tile has no register room for split K)
  L.tc = make_tile_classes(kI8ClassBM, 1, m, 1);
  L.xq = ar.take<int8_t>(m * L.kp);
  L.xs = ar.take<float>(m);
  L.counts = ar.take<int32_t>(1);
  L.offsets = ar.take<int32_t>(2);
  int64_t t = 0;
  for (int c = 0; c < L.tc.n; ++c) t += L.tc.bound[c];
  L.tiles = ar.take<int32_t>(2 * t);
  L.tile_count = ar.take<int32_t>(kMaxClasses);
  L.partial = ar.take<int32_t>(partial_bytes / sizeof(int32_t));
  L.partial_bytes = partial_bytes;
  return L;
}
}  // namespace

namespace {
// K splits of an i8gemm above the small-M kernel's rows, on the LDS-staged
// 256-row tiles: when its items (row tiles x 384-channel blocks) fill less
// than half of the CUs, K is cut into ranges of an even
// number of chunks, at least 16, so that about one item runs per CU; the
// splits' int32 sums go to the workspace and a reduce launch applies the
// epilogue. Returns the splits (1: none) and the chunks per split.
int64_t i8gemm_lds_splits(int64_t m, int64_t k, int64_t n, int64_t* cps_out) {
  const int64_t kc = ceil_div(k, 64), nt = ceil_div(n, 16);
  if (cps_out) *cps_out = kc;
  if (m <= kSmallMRows) return 1;
  // only the LDS-staged tiles take K ranges (A and the weights under 2 GiB)
  if (m * kc * 64 >= kLdsMaxABytes || fcmoe_packed_expert_bytes(1, n, k, 1) >= kLdsMaxABytes) return 1;
  const int64_t items = ceil_div(m, 256) * ceil_div(nt, 24);
  int64_t s = persistent_wgs() / items;  // (2 or 4 times as many: slower at 300-4096 rows)
  if (s > kc / 16) s = kc / 16;
  if (s < 2) return 1;
  int64_t cps = ceil_div(kc, s);
  cps += cps & 1;
  if (cps_out) *cps_out = cps;
  return ceil_div(kc, cps);
}

// Partial-sum bytes of one i8gemm: the small-M kernel's, or the LDS tiles'
// K splits.
size_t i8gemm_partial_bytes(int64_t m, int64_t k, int64_t n) {
  if (m <= kSmallMRows) return smallm_workspace_bytes(m, k, n);
  const int64_t s = i8gemm_lds_splits(m, k, n, nullptr);
  return s > 1 ? (size_t)(s * m * n) * sizeof(int32_t) : 0;
}
}  // namespace

extern "C" size_t fcmoe_i8gemm_workspace_bytes(int64_t m, int64_t k, int64_t n) {
  Arena ar;
  i8_layout(m, k, i8gemm_partial_bytes(m, k, n), ar);
  return ar.used + 256;
}

namespace {
// Both GEMMs of a pair on the small-M kernel run as one launch, so their
// partial sums need room side by side; otherwise (and with the fused launch
// turned off) the two GEMMs run one after the other and share it. The
// workspace covers either.
bool pair_smallm(int64_t m, int64_t k, int64_t n1, int64_t n2) {
  return smallm_splits(m, k, n1) > 0 && smallm_splits(m, k, n2) > 0;
}
size_t pair_partial_bytes(int64_t m, int64_t k, int64_t n1, int64_t n2) {
  const size_t p1 = i8gemm_partial_bytes(m, k, n1), p2 = i8gemm_partial_bytes(m, k, n2);
  const size_t sep = p1 > p2 ? p1 : p2;  // the two GEMMs one after the other (FCMOE_I8GEMM_PAIR_FUSED=0 too)
  if (!pair_smallm(m, k, n1, n2)) return sep;
  const size_t fused = smallm_pair_workspace_bytes(m, k, n1, n2);
  return fused > sep ? fused : sep;
}
}  // namespace

extern "C" size_t fcmoe_i8gemm_pair_workspace_bytes(int64_t m, int64_t k, int64_t n1, int64_t n2) {
  Arena ar;
  i8_layout(m, k, pair_partial_bytes(m, k, n1, n2), ar);
  return ar.used + 256;
}

namespace {

// FCMOE_I8GEMM_PAIR_FUSED=0: the pair's small-M GEMMs as two launches
bool pair_fused() {
  const char* v = getenv("FCMOE_I8GEMM_PAIR_FUSED");
  return !(v && v[0] == '0');
}

// One int8 GEMM of the quantised rows in L against a packed [n, k] weight.
int i8gemm_run(const I8Layout& L, int64_t k, const void* w_packed, const float* w_scale, int64_t n, const float* bias,
               void* out, int out_is_bf16, hipStream_t stream) {
  if (smallm_splits(L.m, k, n) > 0) {
    Stage st(FCMOE_STAGE_W13_CLASS0 + class_slot(16), stream);
    return smallm_i8gemm_launch(L.xq, L.kp, L.m, k, w_packed, L.xs, w_scale, n, bias, out, out_is_bf16, L.partial,
                                L.partial_bytes, stream);
  }
  GemmParams g{};
  g.a = L.xq;
  g.lda = L.kp;
  g.a_rows = L.m;
  g.offsets = L.offsets;
  g.counts = L.counts;
  g.w = w_packed;
  g.w_expert_bytes = fcmoe_packed_expert_bytes(1, n, k, 1);
  g.n = n;
  g.n_half = n;
  g.n_tiles = ceil_div(n, 16);
  g.k_chunks = L.kp / 64;
  g.n_groups = 1;
  g.out = out;
  g.ldo = n;
  g.scale_row = L.xs;
  g.scale_col = w_scale;
  g.bias = bias;
  g.out_bf16 = out_is_bf16;
  g.cus = persistent_wgs();
  int64_t cps = 0;
  const int64_t splits = i8gemm_lds_splits(L.m, k, n, &cps);
  if (splits > 1) {
    if (!L.partial || L.partial_bytes < (size_t)(splits * L.m * n) * sizeof(int32_t))
      return fail(FCMOE_ESPACE, "i8gemm: split-K partial-sum workspace too small");
    g.k_total = g.k_chunks;
    g.k_chunks = cps;
    g.split_out = L.partial;
    g.split_rows = L.m;
  }
  // One expert of m rows: only its class (rows in (bm[c-1], bm[c]], the last
  // class above) gets tiles, so the other classes' launches are not enqueued
  // (5 empty launches cost the 4096-row pair ~0.04 ms).
  int only = L.tc.n - 1;
  for (int c = 0; c < L.tc.n; ++c)
    if (L.m <= L.tc.bm[c]) {
      only = c;
      break;
    }
  for (int c = 0; c < L.tc.n; ++c) {
    if (c != only) continue;
    GemmParams p = g;
    p.tiles = L.tiles + 2 * tile_offset(L.tc, c);
    p.tile_count = L.tile_count + c;
    Stage st(FCMOE_STAGE_W13_CLASS0 + class_slot(L.tc.bm[c]), stream);
    // its tiles exactly: one below the last class, ceil(m / bm) in it
    const int64_t tiles = c == L.tc.n - 1 ? ceil_div(L.m, L.tc.bm[c]) : 1;
    const int rc = gemm_launch(kEpiI8Gemm, L.tc.bm[c], p, tiles, stream);
    if (rc) return rc;
    if (splits > 1)
      return i8gemm_reduce_launch(L.partial, splits, L.m, n, L.xs, w_scale, bias, out, out_is_bf16, stream);
  }
  return FCMOE_OK;
}

// Row quantisation (ties to even) and the single-expert tile list.
int i8gemm_prologue(const void* x, int x_is_f32, int64_t m, int64_t k, size_t partial_bytes, void* workspace,
                    size_t workspace_bytes, I8Layout* L, hipStream_t stream) {
  Arena ar;
  ar.base = (char*)workspace;
  ar.cap = workspace_bytes;
  *L = i8_layout(m, k, partial_bytes, ar);
  if (!ar.base || !ar.ok()) return fail(FCMOE_ESPACE, "i8gemm: workspace too small");
  int rc;
  {
    Stage st(FCMOE_STAGE_QUANT, stream);
    if ((rc = quant_rows_launch(x, x_is_f32, m, k, 1, L->xq, L->kp, L->xs, stream))) return rc;
  }
  if (smallm_splits(m, k, 1) > 0) return FCMOE_OK;  // the small-M GEMM needs no tile list
  if (L->tc.n != 1 || L->tc.bound[0] < ceil_div(m, L->tc.bm[0])) return fail(FCMOE_EINVAL, "i8gemm: tile classes");
  const int64_t nt = ceil_div(m, L->tc.bm[0]);
  hipLaunchKernelGGL(single_expert_tiles_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(nt, 256), 1024)), dim3(256),
                     0, stream, L->counts, L->offsets, L->tiles, L->tile_count, (int32_t)m, (int32_t)L->tc.bm[0]);
  return check_launch("i8gemm tiles");
}

}  // namespace

extern "C" int fcmoe_i8gemm(const void* x, int x_is_f32, int64_t m, int64_t k, const void* w_packed,
                            const float* w_scale, int64_t n, const float* bias, void* out, int out_is_bf16,
                            void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (m < 0 || k <= 0 || n <= 0 || !w_packed || !w_scale) return fail(FCMOE_EINVAL, "i8gemm: bad args");
  if (m == 0) return FCMOE_OK;
  if (m > INT32_MAX / 2) return fail(FCMOE_EINVAL, "i8gemm: too many rows");
  I8Layout L;
  int rc = i8gemm_prologue(x, x_is_f32, m, k, i8gemm_partial_bytes(m, k, n), workspace, workspace_bytes, &L, stream);
  if (rc) return rc;
  return i8gemm_run(L, k, w_packed, w_scale, n, bias, out, out_is_bf16, stream);
}

extern "C" int fcmoe_i8gemm_pair(const uint16_t* x, int64_t m, int64_t k, const void* w1_packed, const float* w1_scale,
                                 int64_t n1, const void* w2_packed, const float* w2_scale, int64_t n2, uint16_t* out1,
                                 uint16_t* out2, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (m < 0 || k <= 0 || n1 <= 0 || n2 <= 0 || !w1_packed || !w1_scale || !w2_packed || !w2_scale)
    return fail(FCMOE_EINVAL, "i8gemm_pair: bad args");
  if (m == 0) return FCMOE_OK;
  if (m > INT32_MAX / 2) return fail(FCMOE_EINVAL, "i8gemm_pair: too many rows");
  if (!x || !out1 || !out2) return fail(FCMOE_EINVAL, "i8gemm_pair: NULL tensor");
  I8Layout L;
  int rc = i8gemm_prologue(x, 0, m, k, pair_partial_bytes(m, k, n1, n2), workspace, workspace_bytes, &L, stream);
  if (rc) return rc;
  if (pair_smallm(m, k, n1, n2) && pair_fused()) {
    Stage st(FCMOE_STAGE_W13_CLASS0 + class_slot(16), stream);
    return smallm_i8gemm_pair_launch(L.xq, L.kp, m, k, L.xs, w1_packed, w1_scale, n1, out1, w2_packed, w2_scale, n2,
                                     out2, L.partial, L.partial_bytes, stream);
  }
  if ((rc = i8gemm_run(L, k, w1_packed, w1_scale, n1, nullptr, out1, 1, stream))) return rc;
  return i8gemm_run(L, k, w2_packed, w2_scale, n2, nullptr, out2, 1, stream);
}

// ------------------------------------------------------------ diagnostics --

extern "C" size_t fcmoe_grouped_gemm_workspace_bytes(int64_t experts, int64_t total_rows) {
  TileClasses tc = make_tile_classes(kClassBM, kNumClasses, total_rows, experts);
  int64_t t = 0;
  for (int c = 0; c < tc.n; ++c) t += tc.bound[c];
  return (size_t)(2 * t + kMaxClasses) * sizeof(int32_t) + 512;
}

extern "C" int fcmoe_grouped_gemm_i8_acc(const int8_t* a, int64_t lda, const int32_t* row_map, const int32_t* counts,
                                         const int32_t* offsets, int64_t experts, int64_t total_rows,
                                         const void* w_packed, int64_t n, int64_t k, int32_t* acc, void* workspace,
                                         size_t workspace_bytes, hipStream_t stream) {
  if (!a || !counts || !offsets || !w_packed || !acc || lda % 64 || lda < k || experts <= 0 || experts > 1024)
    return fail(FCMOE_EINVAL, "grouped_gemm_i8_acc: bad args");
  if (total_rows <= 0) return FCMOE_OK;
  if (workspace_bytes < fcmoe_grouped_gemm_workspace_bytes(experts, total_rows) || !workspace)
    return fail(FCMOE_ESPACE, "grouped_gemm_i8_acc: workspace too small");
  TileClasses tc = make_tile_classes(kClassBM, kNumClasses, total_rows, experts);
  Arena ar;
  ar.base = (char*)workspace;
  ar.cap = workspace_bytes;
  int64_t t = 0;
  for (int c = 0; c < tc.n; ++c) t += tc.bound[c];
  int32_t* tiles = ar.take<int32_t>(2 * t);
  int32_t* tile_count = ar.take<int32_t>(kMaxClasses);
  int rc = tiles_from_counts_launch(counts, experts, tc, tiles, tile_count, stream);
  if (rc) return rc;
  GemmParams g{};
  g.a = a;
  g.lda = lda;
  g.a_rows = row_map ? 0 : total_rows;  // gathered rows: the caller keeps A under 2 GiB
  g.row_map = row_map;
  g.offsets = offsets;
  g.counts = counts;
  g.w = w_packed;
  g.w_expert_bytes = fcmoe_packed_expert_bytes(1, n, k, 1);
  g.n = n;
  g.n_half = n;
  g.n_tiles = ceil_div(n, 16);
  g.k_chunks = ceil_div(k, 64);
  g.n_groups = 1;
  g.out = acc;
  g.ldo = n;
  for (int c = 0; c < tc.n; ++c) {
    GemmParams p = g;
    p.tiles = tiles + 2 * tile_offset(tc, c);
    p.tile_count = tile_count + c;
    rc = gemm_launch(kEpiRawI32, tc.bm[c], p, tc.bound[c], stream);
    if (rc) return rc;
  }
  return FCMOE_OK;
}

// ----------------------------------------------------------- stage timing --

extern "C" int fcmoe_stage_timing_enable(int enable) {
  StageTimer& t = timer();
  std::lock_guard<std::mutex> g(t.mu);
  t.on = enable != 0;
  return FCMOE_OK;
}

extern "C" int fcmoe_w8a8_prefill_plan(const int32_t* class_tiles, int* part_wgs_out) {
  if (!class_tiles) return fail(FCMOE_EINVAL, "class_tiles is NULL");
  const int min_tiles = mixed_min_tiles();
  const bool mixed = class_tiles[0] >= min_tiles && (min_tiles <= 0 || class_tiles[3] >= kPrefillMixedMinBigTiles);
  const int w = !mixed && min_tiles > 0 && part_enabled() ? part_wgs(class_tiles) : 0;
  if (part_wgs_out) *part_wgs_out = w;
  return mixed ? 1 : (w > 0 ? 2 : 0);
}

extern "C" int fcmoe_stage_timing_read(double* total_ms, int64_t* launches) {
  StageTimer& t = timer();
  std::lock_guard<std::mutex> g(t.mu);
  for (int i = 0; i < FCMOE_STAGE_COUNT; ++i) {
    if (total_ms) total_ms[i] = 0.0;
    if (launches) launches[i] = 0;
  }
  int rc = FCMOE_OK;
  for (const TimerRec& r : t.recs) {
    float ms = 0.0f;
    if (hipEventSynchronize(r.b) != hipSuccess || hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess) {
      rc = fail(FCMOE_EDEVICE, "stage timing: event query failed");
    } else if (r.stage >= 0 && r.stage < FCMOE_STAGE_COUNT) {
      if (total_ms) total_ms[r.stage] += ms;
      if (launches) launches[r.stage] += 1;
    }
    t.pool.push_back(r.a);
    t.pool.push_back(r.b);
  }
  t.recs.clear();
  return rc;
}
