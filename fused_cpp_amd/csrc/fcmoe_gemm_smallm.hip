// fcmoe_gemm_smallm.hip -- i8gemm at few rows (M <= 256), weight streaming.
//
// At decode batch sizes an i8gemm is a weight stream: DeepSeek's attention
// output projection at 64 rows reads 117 MB of int8 weights for 15 GOP. The
// row-tiled grouped GEMM gives such a product one workgroup per channel block
// (28 workgroups for a [7168, 16384] weight on the 64-row tile), or re-reads
// the weights for every 16-row tile. Here:
//   * a workgroup is 8 waves, one 16-channel weight tile each, over a range
//     of K chunks; every wave holds all M rows (FM = ceil(M / 16) row
//     fragments of v_mfma_i32_16x16x64_i8), so each weight byte is read once;
//   * the rows' 64-byte K chunk (FM KB) is staged in LDS by buffer_load ...
//     lds and read by all 8 waves: A costs FM KB of L2 reads per 8 KB of
//     weights;
//   * each wave streams its tile's 1 KB chunks with nontemporal buffer loads
//     into a register ring; A stages and weight chunks are issued in pairs, kSmDepth
//     - 1 pairs ahead;
//   * K is split over the grid's y dimension so that the launch has about one
//     workgroup per CU; the splits' exact int32 partial sums go to a workspace
//     and a second launch adds them (in split order; int32 sums are exact in
//     any order) and applies the i8gemm epilogue. With one split the GEMM
//     launch applies the epilogue itself.
// The epilogue is write_scaled_output's (csrc/i8gemm.cpp:148-164):
// (float)acc * s_x * s_w left to right, + bias, then bf16 (RNE) or fp32.
//
// The same kernel runs the BF16 dense MLP at few rows (one packed expert, at
// most 256 routes: the shared MLP at decode batch sizes) on
// v_mfma_f32_16x16x32_bf16: A rows gathered through the route order's token
// map, fp32 partial sums always written, and a reduce launch that adds the
// splits in split order and applies the W13 activation (gate + bias,
// up + bias, act_bf16_mode, bf16) or the W2 route store (+ bias, fp32 route
// rows for the combine).
#include <cstdlib>
#include <utility>

#include "fcmoe_gemm_common.h"

namespace fcmoe {

namespace {

constexpr int kSmWaves = 8;  // waves per workgroup, one 16-channel tile each
constexpr int kSmDepth = 8;  // ring depth: A stages (LDS) and weight chunks (registers)
constexpr int kSmBufWord3 = 0x00020000;
typedef __attribute__((address_space(3))) void* sm_lds_ptr;

template <int N>
__device__ __forceinline__ void sm_wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

struct SmallMArgs {
  const void* a;               // rows [*, lda]: int8 (i8gemm) or bf16
  int64_t lda;                 // bytes per row (a multiple of 64)
  const int32_t* row_map;      // row r of the product reads A row row_map[r] (null: r)
  int m;
  int64_t kc;                  // 64-byte K chunks
  int64_t cps;                 // chunks per split (grid.y splits)
  const void* w;               // packed [n_groups][n_tiles][kc][64 lanes][16 B]
  int64_t n_groups, n_tiles;   // weight tiles per group (total n_groups x n_tiles)
  int64_t n_half;              // logical channels per group
  int64_t n;                   // logical channels (n_groups x n_half): partial-sum row width
  const float* scale_row;      // [m] (i8gemm)
  const float* scale_col;      // [n] (i8gemm)
  const float* bias;           // [n] or null
  void* out;
  int out_bf16;
  int64_t ldo;
  void* partial;               // [splits][m][n] int32 (int8) / fp32 (bf16); null: direct i8gemm epilogue
  const int32_t* out_row;      // route store: output row of product row r (the flat route)
  int activation;              // W13 activation store: FCMOE_ACT_*
  const int32_t* m_dev;        // rows actually routed (device; null: m): the MoE route
                               // build drops invalid ids, so fewer than m rows may exist
};

__device__ __forceinline__ void sm_store(const SmallMArgs& p, int row, int64_t ch, int32_t acc) {
  // write_scaled_output, csrc/i8gemm.cpp:148-164 (left to right)
  float v = (float)acc * p.scale_row[row] * p.scale_col[ch];
  if (p.bias) v = v + p.bias[ch];
  if (p.out_bf16)
    ((uint16_t*)p.out)[(int64_t)row * p.ldo + ch] = f32_to_bf16(v);
  else
    ((float*)p.out)[(int64_t)row * p.ldo + ch] = v;
}

// Workgroup (bx, by) of one small-M GEMM: weight tiles 8 bx .. 8 bx + 7, K
// split by.
template <bool I8, int FM>
__device__ __forceinline__ void smallm_body(const SmallMArgs& p, int bx, int by) {
#if __HIP_DEVICE_COMPILE__
  constexpr int D = kSmDepth;
  constexpr int ABYTES = FM * 1024;  // 16 FM rows x 64 bytes
  constexpr int LA = (FM + kSmWaves - 1) / kSmWaves;  // A loads per wave and chunk
  static_assert(FM <= kSmWaves || FM % kSmWaves == 0, "the waves' A loads cover every row fragment once");
  constexpr int OPS = LA + 1;  // vector-memory ops per (A stage, weight chunk) pair
  typedef typename Acc<I8>::type AccT;
  __shared__ __attribute__((aligned(1024))) uint8_t sa[D * ABYTES];
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int64_t tile = (int64_t)bx * kSmWaves + wave;  // packed tile (group-major)
  const bool tv = tile < p.n_groups * p.n_tiles;
  const int64_t c0 = (int64_t)by * p.cps;
  const int64_t c1 = c0 + p.cps < p.kc ? c0 + p.cps : p.kc;
  // 32-bit chunk counters keep the loop's compares scalar (a 64-bit compare
  // took a VGPR with a load in flight and drained the ring every 8 chunks)
  const int nch = (int)(c1 - c0);  // >= 1 (the host sizes the splits)

  // A stage loads of this wave: fragments g = (wave + 8 u) % FM, u < LA, rows
  // 16 g + lane / 4 (with FM < 8, waves beyond FM repeat a load: same bytes to
  // the same place, so every wave issues LA A loads per chunk and the wait
  // counts are uniform). 16-byte unit u of row r sits at slot u ^ ((r >> 2) &
  // 3): the 16 rows of a fragment read fall on distinct banks.
  const int aunit = (lane % 4) ^ ((lane >> 4) & 3);
  const int rows_valid = p.m_dev ? *p.m_dev : p.m;
  const __amdgpu_buffer_rsrc_t rsrc_a =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.a), (short)0, 0x7ffffff0, kSmBufWord3);
  int g[LA];
  uint32_t voff_a[LA];
#pragma unroll
  for (int u = 0; u < LA; ++u) {
    g[u] = (wave + kSmWaves * u) % FM;
    const int ar = g[u] * 16 + lane / 4;
    const int arow_local = ar < rows_valid ? ar : (rows_valid > 0 ? rows_valid - 1 : 0);
    // rows past the routed ones re-read the last routed row (or x row 0);
    // their sums are never stored
    const int64_t arow = p.row_map && rows_valid > 0 ? (int64_t)p.row_map[arow_local] : (int64_t)arow_local;
    voff_a[u] = (uint32_t)(arow * p.lda + aunit * 16);
  }
  // The tile's weights through a buffer resource: the chunk offset goes in
  // the scalar operand and the lane offset is fixed, so no address VGPR is
  // computed per load (a 64-bit address written into a ring register with an
  // older load pending made the compiler drain the ring).
  const __amdgpu_buffer_rsrc_t rsrc_b = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const uint8_t*)p.w + (tv ? tile : 0) * p.kc * 1024), (short)0, (int)(p.kc * 1024), kSmBufWord3);
  const int voff_b = lane * 16;
  const int frag = (lane % 16) * 64 + (((lane / 16) ^ ((lane % 16) >> 2)) * 16);

  v4i bq[D];
  AccT acc[FM];
#pragma unroll
  for (int i = 0; i < FM; ++i) acc[i] = AccT{0, 0, 0, 0};

  // pair t: A stage and weight chunk of the split's chunk t (past the end:
  // the last chunk again, never consumed)
  auto issue = [&](int t, auto slot_c) {
    constexpr int slot = decltype(slot_c)::value;
    const int64_t c = c0 + (t < nch ? t : nch - 1);
#pragma unroll
    for (int u = 0; u < LA; ++u)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_a, (sm_lds_ptr)(sa + slot * ABYTES + g[u] * 1024), 16,
                                               voff_a[u], (int)(c * 64), 0, 0);
    // keep each pair in issue order (A, then the weights): the wait counts
    // below, and the compiler's own for the weight registers, assume it
    __builtin_amdgcn_sched_barrier(0);
    bq[slot] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rsrc_b, voff_b, (int)(c * 1024), 2));
    __builtin_amdgcn_sched_barrier(0);
  };
  [&]<int... S>(std::integer_sequence<int, S...>) {
    (issue(S, std::integral_constant<int, S>{}), ...);
  }(std::make_integer_sequence<int, D - 1>{});

  auto body = [&](int t, auto slot_c) {
    constexpr int slot = decltype(slot_c)::value;
    // this wave's pair t has landed (pairs t+1 .. t+D-2 may not); after the
    // barrier every wave's A stage t has, and no wave reads stage t-1 any more
    sm_wait_vmcnt<OPS * (D - 2)>();
    __builtin_amdgcn_s_barrier();
    issue(t + D - 1, std::integral_constant<int, (slot + D - 1) % D>{});
    v4i af[FM];
#pragma unroll
    for (int i = 0; i < FM; ++i) af[i] = *(const v4i*)(sa + slot * ABYTES + i * 1024 + frag);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      if constexpr (I8)
        acc[i] = mfma(af[i], bq[slot], acc[i]);
      else
        acc[i] = mfma(__builtin_bit_cast(v8bf, af[i]), __builtin_bit_cast(v8bf, bq[slot]), acc[i]);
    }
  };
  // whole rings of D chunks, then the rest: no conditional step inside the
  // loop, so the compiler's wait counts at the loop header match the steady
  // state (a conditional step made it wait for all but the newest pair)
  int t0 = 0;
  for (; t0 + D <= nch; t0 += D) {
    [&]<int... S>(std::integer_sequence<int, S...>) {
      (body(t0 + S, std::integral_constant<int, S>{}), ...);
    }(std::make_integer_sequence<int, D>{});
  }
  [&]<int... S>(std::integer_sequence<int, S...>) {
    ((t0 + S < nch ? body(t0 + S, std::integral_constant<int, S>{}) : void()), ...);
  }(std::make_integer_sequence<int, D>{});
  sm_wait_vmcnt<0>();

  if (!tv) return;
  const int64_t grp = tile / p.n_tiles;
  const int64_t cin = (tile - grp * p.n_tiles) * 16 + lane % 16;
  if (cin >= p.n_half) return;
  const int64_t ch = grp * p.n_half + cin;  // logical channel
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = i * 16 + (lane / 16) * 4 + q;
      if (row >= p.m) continue;
      const int64_t e = ((int64_t)by * p.m + row) * p.n + ch;
      if constexpr (I8) {
        if (p.partial)
          ((int32_t*)p.partial)[e] = acc[i][q];
        else
          sm_store(p, row, ch, acc[i][q]);
      } else {
        ((float*)p.partial)[e] = acc[i][q];
      }
    }
#endif
}

template <bool I8, int FM>
__global__ __launch_bounds__(kSmWaves * kWave) void smallm_kernel(SmallMArgs p) {
  smallm_body<I8, FM>(p, (int)blockIdx.x, (int)blockIdx.y);
}

// Two int8 GEMMs of the same rows in one launch (the i8gemm pair): workgroups
// x < x1 run the first (splits s1), the rest the second (splits s2); grid.y
// covers the larger split count and workgroups past their GEMM's splits exit.
template <int FM>
__global__ __launch_bounds__(kSmWaves * kWave) void smallm_pair_kernel(SmallMArgs p1, SmallMArgs p2, int x1, int s1,
                                                                        int s2) {
  const int bx = (int)blockIdx.x, by = (int)blockIdx.y;
  if (bx < x1) {
    if (by < s1) smallm_body<true, FM>(p1, bx, by);
  } else if (by < s2) {
    smallm_body<true, FM>(p2, bx - x1, by);
  }
}

// Adds the splits' partial sums (split order) and applies the epilogue; one
// thread per output element, grid-stride.
__global__ __launch_bounds__(256) void smallm_reduce_kernel(SmallMArgs p, int splits) {
  const int64_t total = (int64_t)p.m * p.n;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    int32_t acc = 0;
    for (int s = 0; s < splits; ++s) acc += ((const int32_t*)p.partial)[(int64_t)s * total + e];
    sm_store(p, (int)(e / p.n), e % p.n, acc);
  }
}

// BF16 W13: y[r][f] = bf16(act(gate + bias, up + bias)) over the gate
// channels f < n_half (up channel n_half + f), the splits' fp32 sums added in
// split order; the arithmetic after the sums is the W13 activation
// epilogue's (fcmoe_gemm_common.h).
__global__ __launch_bounds__(256) void smallm_act_kernel(SmallMArgs p, int splits) {
  const int64_t total = (int64_t)p.m * p.n_half, plane = (int64_t)p.m * p.n;
  const float* part = (const float*)p.partial;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / p.n_half, f = e % p.n_half;
    const int64_t eg = r * p.n + f, eu = eg + p.n_half;
    float gate = part[eg], up = part[eu];
    for (int s = 1; s < splits; ++s) {
      gate = gate + part[s * plane + eg];
      up = up + part[s * plane + eu];
    }
    if (p.bias) {
      gate = gate + p.bias[f];
      up = up + p.bias[p.n_half + f];
    }
    ((uint16_t*)p.out)[r * p.ldo + f] = f32_to_bf16(act_bf16_mode(gate, up, p.activation));
  }
}

// BF16 W2: route_out[out_row[r]][h] = sum (+ bias[h]), the splits' fp32 sums
// added in split order.
__global__ __launch_bounds__(256) void smallm_route_kernel(SmallMArgs p, int splits) {
  const int64_t total = (int64_t)p.m * p.n;
  const float* part = (const float*)p.partial;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / p.n, h = e % p.n;
    if (p.m_dev && r >= *p.m_dev) continue;  // a dropped route: no row to store
    float v = part[e];
    for (int s = 1; s < splits; ++s) v = v + part[s * total + e];
    if (p.bias) v = v + p.bias[h];
    ((float*)p.out)[(int64_t)p.out_row[r] * p.ldo + h] = v;
  }
}

// BF16 W2 with one route per token: token t's route row (product row
// route_pos[t], -1: dropped; row t with weight 1 when route_pos is null) = the
// splits' fp32 sums in split order (+ bias[h]), stored to route_out[t] (the
// flat route) and merged in place of the combine launch, with its arithmetic
// for one slot: acc = fma(row, weight, 0), or the row itself with
// skip_weighted, 0 for a dropped route; out = bf16(acc).
__global__ __launch_bounds__(256) void smallm_route_merge_kernel(SmallMArgs p, int splits, const int32_t* route_pos,
                                                                 const float* route_weight, int skip_weighted,
                                                                 uint16_t* out, int64_t tokens,
                                                                 int32_t* invalid_count) {
  const int64_t total = tokens * p.n, plane = (int64_t)p.m * p.n;
  const float* part = (const float*)p.partial;
  if (invalid_count && blockIdx.x == 0 && threadIdx.x == 0) store_count(invalid_count, 0);
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = e / p.n, h = e % p.n;
    const int pos = route_pos ? route_pos[t] : (int)t;
    float acc = 0.0f;
    if (pos >= 0) {
      const int64_t i = (int64_t)pos * p.n + h;
      float v = part[i];
      for (int s = 1; s < splits; ++s) v = v + part[s * plane + i];
      if (p.bias) v = v + p.bias[h];
      ((float*)p.out)[t * p.ldo + h] = v;
      acc = skip_weighted ? v : __builtin_fmaf(v, route_weight ? route_weight[t] : 1.0f, 0.0f);
    }
    out[e] = f32_to_bf16(acc);
  }
}

}  // namespace

namespace {

// K splits for a product of m rows over kc chunks and `tiles` weight tiles
// (0 outside the domain): workgroups (tile groups x splits) up to the target
// (FCMOE_SMALLM_WGS, default 256: about one per CU), at least 8 chunks a split.
int64_t splits_for(int64_t m, int64_t kc, int64_t tiles) {
  if (m <= 0 || m > kSmallMRows || kc <= 0 || tiles <= 0) return 0;
  const int64_t groups = ceil_div(tiles, kSmWaves);
  static const int64_t target = [] {
    const char* v = getenv("FCMOE_SMALLM_WGS");
    return v && v[0] ? (int64_t)atoll(v) : (int64_t)256;
  }();
  int64_t s = target / groups;
  const int64_t smax = kc / 8 > 1 ? kc / 8 : 1;
  if (s > smax) s = smax;
  if (s < 1) s = 1;
  const int64_t cps = ceil_div(kc, s);
  return ceil_div(kc, cps);
}

int launch_gemm(const SmallMArgs& p0, int64_t splits, bool i8, hipStream_t stream) {
  SmallMArgs p = p0;
  p.cps = ceil_div(p.kc, splits);
  const dim3 grid((unsigned)ceil_div(p.n_groups * p.n_tiles, kSmWaves), (unsigned)splits), block(kSmWaves * kWave);
  const int fm = (int)ceil_div(p.m, 16);
  if (i8) {
    if (fm == 1)
      hipLaunchKernelGGL((smallm_kernel<true, 1>), grid, block, 0, stream, p);
    else if (fm == 2)
      hipLaunchKernelGGL((smallm_kernel<true, 2>), grid, block, 0, stream, p);
    else if (fm <= 4)
      hipLaunchKernelGGL((smallm_kernel<true, 4>), grid, block, 0, stream, p);
    else if (fm <= 8)
      hipLaunchKernelGGL((smallm_kernel<true, 8>), grid, block, 0, stream, p);
    else
      hipLaunchKernelGGL((smallm_kernel<true, 16>), grid, block, 0, stream, p);
  } else {
    if (fm == 1)
      hipLaunchKernelGGL((smallm_kernel<false, 1>), grid, block, 0, stream, p);
    else if (fm == 2)
      hipLaunchKernelGGL((smallm_kernel<false, 2>), grid, block, 0, stream, p);
    else if (fm <= 4)
      hipLaunchKernelGGL((smallm_kernel<false, 4>), grid, block, 0, stream, p);
    else if (fm <= 8)
      hipLaunchKernelGGL((smallm_kernel<false, 8>), grid, block, 0, stream, p);
    else
      hipLaunchKernelGGL((smallm_kernel<false, 16>), grid, block, 0, stream, p);
  }
  return check_launch("smallm_gemm");
}

unsigned reduce_blocks(int64_t total) { return (unsigned)(ceil_div(total, 256) < 4096 ? ceil_div(total, 256) : 4096); }

}  // namespace

int64_t smallm_splits(int64_t m, int64_t k, int64_t n) {
  if (k <= 0 || n <= 0) return 0;
  return splits_for(m, ceil_div(k, 64), ceil_div(n, 16));
}

size_t smallm_workspace_bytes(int64_t m, int64_t k, int64_t n) {
  const int64_t s = smallm_splits(m, k, n);
  return s > 1 ? (size_t)(s * m * n) * sizeof(int32_t) : 0;
}

// The pair's one launch: the split count that brings both GEMMs' workgroups
// together to about one per CU (DeepSeek V4's [24576 + 8192, 1536] at 64 rows:
// 192 + 64 workgroups, one split, no reduce: 0.0275 -> 0.018 ms against each
// GEMM split on its own, 1 and 3 ways).
int64_t smallm_pair_splits(int64_t m, int64_t k, int64_t n1, int64_t n2) {
  if (smallm_splits(m, k, n1) <= 0 || smallm_splits(m, k, n2) <= 0) return 0;
  return splits_for(m, ceil_div(k, 64), round_up(ceil_div(n1, 16), kSmWaves) + round_up(ceil_div(n2, 16), kSmWaves));
}

size_t smallm_pair_workspace_bytes(int64_t m, int64_t k, int64_t n1, int64_t n2) {
  const int64_t s = smallm_pair_splits(m, k, n1, n2);
  return s > 1 ? (size_t)(s * m * (n1 + n2)) * sizeof(int32_t) : 0;
}

int smallm_i8gemm_launch(const int8_t* a, int64_t lda, int64_t m, int64_t k, const void* w_packed,
                         const float* scale_row, const float* scale_col, int64_t n, const float* bias, void* out,
                         int out_bf16, int32_t* partial, size_t partial_bytes, hipStream_t stream) {
  const int64_t splits = smallm_splits(m, k, n);
  if (splits <= 0) return fail(FCMOE_EINVAL, "small-M i8gemm: shape outside its domain");
  if (lda % 64 || lda < round_up(k, 64) || (int64_t)m * lda >= 0x7ffffff0)
    return fail(FCMOE_EINVAL, "small-M i8gemm: bad row stride");
  if (splits > 1 && (!partial || partial_bytes < smallm_workspace_bytes(m, k, n)))
    return fail(FCMOE_ESPACE, "small-M i8gemm: partial-sum workspace too small");
  SmallMArgs p{};
  p.a = a;
  p.lda = lda;
  p.m = (int)m;
  p.kc = ceil_div(k, 64);
  p.w = w_packed;
  p.n_groups = 1;
  p.n_tiles = ceil_div(n, 16);
  p.n_half = n;
  p.n = n;
  p.scale_row = scale_row;
  p.scale_col = scale_col;
  p.bias = bias;
  p.out = out;
  p.out_bf16 = out_bf16;
  p.ldo = n;
  p.partial = splits > 1 ? partial : nullptr;
  int rc = launch_gemm(p, splits, true, stream);
  if (rc || splits == 1) return rc;
  hipLaunchKernelGGL(smallm_reduce_kernel, dim3(reduce_blocks(m * n)), dim3(256), 0, stream, p, (int)splits);
  return check_launch("smallm_reduce");
}

int smallm_i8gemm_pair_launch(const int8_t* a, int64_t lda, int64_t m, int64_t k, const float* scale_row,
                              const void* w1, const float* sc1, int64_t n1, uint16_t* out1, const void* w2,
                              const float* sc2, int64_t n2, uint16_t* out2, int32_t* partial, size_t partial_bytes,
                              hipStream_t stream) {
  const int64_t s1 = smallm_pair_splits(m, k, n1, n2), s2 = s1;
  if (s1 <= 0) return fail(FCMOE_EINVAL, "small-M i8gemm pair: shape outside its domain");
  if (lda % 64 || lda < round_up(k, 64) || (int64_t)m * lda >= 0x7ffffff0)
    return fail(FCMOE_EINVAL, "small-M i8gemm pair: bad row stride");
  if (partial_bytes < smallm_pair_workspace_bytes(m, k, n1, n2) || (!partial && partial_bytes))
    return fail(FCMOE_ESPACE, "small-M i8gemm pair: partial-sum workspace too small");
  SmallMArgs p[2]{};
  const void* ws[2] = {w1, w2};
  const float* scs[2] = {sc1, sc2};
  const int64_t ns[2] = {n1, n2}, ss[2] = {s1, s2};
  uint16_t* outs[2] = {out1, out2};
  int32_t* part = partial;
  for (int g = 0; g < 2; ++g) {
    SmallMArgs& q = p[g];
    q.a = a;
    q.lda = lda;
    q.m = (int)m;
    q.kc = ceil_div(k, 64);
    q.cps = ceil_div(q.kc, ss[g]);
    q.w = ws[g];
    q.n_groups = 1;
    q.n_tiles = ceil_div(ns[g], 16);
    q.n_half = ns[g];
    q.n = ns[g];
    q.scale_row = scale_row;
    q.scale_col = scs[g];
    q.out = outs[g];
    q.out_bf16 = 1;
    q.ldo = ns[g];
    q.partial = ss[g] > 1 ? part : nullptr;
    if (ss[g] > 1) part += ss[g] * m * ns[g];
  }
  const int x1 = (int)ceil_div(p[0].n_tiles, kSmWaves), x2 = (int)ceil_div(p[1].n_tiles, kSmWaves);
  const dim3 grid((unsigned)(x1 + x2), (unsigned)(s1 > s2 ? s1 : s2)), block(kSmWaves * kWave);
  const int fm = (int)ceil_div(m, 16);
  if (fm == 1)
    hipLaunchKernelGGL(smallm_pair_kernel<1>, grid, block, 0, stream, p[0], p[1], x1, (int)s1, (int)s2);
  else if (fm == 2)
    hipLaunchKernelGGL(smallm_pair_kernel<2>, grid, block, 0, stream, p[0], p[1], x1, (int)s1, (int)s2);
  else if (fm <= 4)
    hipLaunchKernelGGL(smallm_pair_kernel<4>, grid, block, 0, stream, p[0], p[1], x1, (int)s1, (int)s2);
  else if (fm <= 8)
    hipLaunchKernelGGL(smallm_pair_kernel<8>, grid, block, 0, stream, p[0], p[1], x1, (int)s1, (int)s2);
  else
    hipLaunchKernelGGL(smallm_pair_kernel<16>, grid, block, 0, stream, p[0], p[1], x1, (int)s1, (int)s2);
  int rc = check_launch("smallm_pair_gemm");
  for (int g = 0; g < 2 && !rc; ++g) {
    if (ss[g] <= 1) continue;
    hipLaunchKernelGGL(smallm_reduce_kernel, dim3(reduce_blocks(m * ns[g])), dim3(256), 0, stream, p[g], (int)ss[g]);
    rc = check_launch("smallm_reduce");
  }
  return rc;
}

int i8gemm_reduce_launch(const int32_t* partial, int64_t splits, int64_t m, int64_t n, const float* scale_row,
                         const float* scale_col, const float* bias, void* out, int out_bf16, hipStream_t stream) {
  if (splits < 1 || m <= 0 || n <= 0 || m * n > INT32_MAX) return fail(FCMOE_EINVAL, "i8gemm reduce: bad shape");
  SmallMArgs p{};
  p.m = (int)m;
  p.n = n;
  p.n_half = n;
  p.scale_row = scale_row;
  p.scale_col = scale_col;
  p.bias = bias;
  p.out = out;
  p.out_bf16 = out_bf16;
  p.ldo = n;
  p.partial = const_cast<int32_t*>(partial);
  hipLaunchKernelGGL(smallm_reduce_kernel, dim3(reduce_blocks(m * n)), dim3(256), 0, stream, p, (int)splits);
  return check_launch("i8gemm_reduce");
}

int64_t smallm_bf16_splits(int64_t m, int64_t k_chunks, int64_t tiles) { return splits_for(m, k_chunks, tiles); }

int smallm_bf16_launch(const SmallMBf16& q, hipStream_t stream) {
  const int64_t tiles = q.n_groups * ceil_div(q.n_half, 16);
  const int64_t splits = splits_for(q.m, q.k_chunks, tiles);
  if (splits <= 0) return fail(FCMOE_EINVAL, "small-M BF16 GEMM: shape outside its domain");
  if (q.lda_bytes % 64 || q.lda_bytes < q.k_chunks * 64 || q.a_rows * q.lda_bytes >= 0x7ffffff0)
    return fail(FCMOE_EINVAL, "small-M BF16 GEMM: bad row stride");
  const int64_t n = q.n_groups * q.n_half;
  if (!q.partial || q.partial_bytes < (size_t)(splits * q.m * n) * sizeof(float))
    return fail(FCMOE_ESPACE, "small-M BF16 GEMM: partial-sum workspace too small");
  SmallMArgs p{};
  p.a = q.a;
  p.lda = q.lda_bytes;
  p.row_map = q.row_map;
  p.m = (int)q.m;
  p.kc = q.k_chunks;
  p.w = q.w;
  p.n_groups = q.n_groups;
  p.n_tiles = ceil_div(q.n_half, 16);
  p.n_half = q.n_half;
  p.n = n;
  p.bias = q.bias;
  p.out = q.out;
  p.ldo = q.ldo;
  p.partial = q.partial;
  p.out_row = q.out_row;
  p.activation = q.activation;
  p.m_dev = q.m_dev;
  int rc = launch_gemm(p, splits, false, stream);
  if (rc) return rc;
  if (q.merge_out) {
    hipLaunchKernelGGL(smallm_route_merge_kernel, dim3(reduce_blocks(q.tokens * n)), dim3(256), 0, stream, p,
                       (int)splits, q.route_pos, q.route_weight, q.skip_weighted, q.merge_out, q.tokens,
                       q.invalid_count);
  } else if (q.out_row) {
    hipLaunchKernelGGL(smallm_route_kernel, dim3(reduce_blocks(q.m * n)), dim3(256), 0, stream, p, (int)splits);
  } else {
    hipLaunchKernelGGL(smallm_act_kernel, dim3(reduce_blocks(q.m * q.n_half)), dim3(256), 0, stream, p,
                       (int)splits);
  }
  return check_launch("smallm_bf16_reduce");
}

}  // namespace fcmoe
