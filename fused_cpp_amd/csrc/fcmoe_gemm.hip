// fcmoe_gemm.hip -- grouped (per-expert) GEMM on CDNA4 MFMA with fused
// epilogues. One template serves int8 (v_mfma_i32_16x16x64_i8, exact int32
// accumulation) and bf16 (v_mfma_f32_16x16x32_bf16, fp32 accumulation).
//
// Work decomposition
//   grid.x = tiles * n_blocks. A tile is (expert, first row) from the route
//   kernel's per-class list; its BM rows are the expert's routed rows in
//   sorted (ascending flat route) order. A workgroup is 4 wavefronts arranged
//   WM x WN; a wave owns FM 16-row fragments x 4 16-channel tiles.
//
// Data movement
//   B (weights, HBM-streamed, read once per M tile): packed offline in the
//   exact MFMA operand order (1 KiB per 16-channel x 64-byte tile chunk), so
//   each lane issues one 16-byte global load per tile per chunk, straight into
//   registers, software-pipelined one K step ahead. No LDS round trip.
//   A (routed activation rows, gathered through row_map): staged through
//   double-buffered LDS (row stride 64*FK+16 bytes keeps the 16 rows of a
//   ds_read_b128 on distinct banks), one barrier per K step.
//
// Operand order: lane l supplies row/column (l % 16) and bytes
// [16*(l/16), 16*(l/16)+16) of the current 64-byte K chunk for both A and B;
// since A and B use the same lane->K mapping, the products pair the same k
// whatever the hardware's internal K order. D lane l, register i holds row
// 4*(l/16)+i, column l%16.
#include <cstdlib>
#include <utility>

#include "fcmoe_gemm_common.h"

namespace fcmoe {

namespace {


template <bool I8, int EPI, int WM, int WN, int FM, int FN, int NB, bool ADIRECT>
__device__ __forceinline__ void grouped_gemm_body(const GemmParams& p, int n_blocks) {
  constexpr int kThreads = WM * WN * kWave;
  constexpr int BM = WM * FM * 16;
  constexpr int ROWB = 64 + 16;                    // LDS row stride (bytes): 16 rows hit distinct banks
  constexpr int UNITS = BM * 4;                    // 16-byte A units per 64-byte K chunk
  constexpr int UPT = (UNITS + kThreads - 1) / kThreads;
  constexpr bool PAIR = epi_pair(EPI);
  // W8A16: bf16 A, int8 B. A K chunk is 64 elements = 128 bytes (two 16-byte
  // fragments per lane); each chunk runs two bf16 MFMAs per tile pair.
  constexpr bool W8 = epi_w8(EPI);
  constexpr int AW = W8 ? 2 : 1;
  static_assert(!ADIRECT || WM == 1, "direct A fragments assume one wave row");
  static_assert(!W8 || (ADIRECT && !I8), "W8A16 runs on the direct-A path with fp32 accumulators");
  typedef typename Acc<I8>::type AccT;

  __shared__ __attribute__((aligned(16))) uint8_t sA[ADIRECT ? 1 : 3][ADIRECT ? 16 : BM * ROWB];

  // Tiles run last-first: the route kernel lists experts in id order and the
  // appended shared expert (the largest) is last, so it starts first.
  if (!plan_open(p)) return;
  const int count = *p.tile_count;
  const int total_items = count * n_blocks;
  // Persistent launches (p.persist > 0, direct-A tiles only) run a fixed
  // grid whose workgroups stride over the items; otherwise each workgroup
  // runs item blockIdx.x once.
  const int item_step = (ADIRECT && p.persist > 0) ? (int)gridDim.x : total_items;
  for (int item = (int)blockIdx.x; item < total_items; item += item_step) {
  const int tile = count - 1 - item / n_blocks;
  const int nb = item % n_blocks;
  const int expert = p.tiles[2 * tile];
  const int m0 = p.tiles[2 * tile + 1];
  const int rows_left = p.counts[expert] - m0;
  const int rows = rows_left < BM ? rows_left : BM;
  const int pos0 = p.offsets[expert] + m0;

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = tid / kWave;
  const int wm = wave / WN;
  const int wn = wave % WN;

  // ---- this wave's four channel tiles (global tile index within expert)
  int64_t gtile[FN];
  bool tvalid[FN];
  const int64_t total_tiles = (int64_t)p.n_groups * p.n_tiles;
  if (PAIR) {
    // first FN/2 slots: gate tiles; last FN/2: the matching up tiles
    constexpr int HP = FN / 2;
    const int64_t pair0 = ((int64_t)nb * WN + wn) * HP;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int64_t pr = pair0 + (j % HP);
      tvalid[j] = pr < p.n_tiles;
      gtile[j] = (j < HP ? 0 : p.n_tiles) + pr;
    }
  } else {
    const int64_t t0 = ((int64_t)nb * WN + wn) * FN;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      gtile[j] = t0 + j;
      tvalid[j] = gtile[j] < total_tiles;
    }
  }
  const uint8_t* wbase = (const uint8_t*)p.w + (int64_t)expert * p.w_expert_bytes;
  const v4i* bptr[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j)
    bptr[j] = (const v4i*)(wbase + (tvalid[j] ? gtile[j] : 0) * p.k_chunks * 1024) + lane;

  const int64_t lda_bytes = p.lda * (I8 ? 1 : 2);  // bf16 rows for the bf16 and W8A16 paths
  const int64_t kc = p.k_chunks;

  // ---- A sources. Direct: lane l reads row l%16 of each fragment, bytes
  // 16*(l/16) of the chunk. LDS: thread units of 16 bytes per chunk. Rows
  // past the tile's end read the tile's last row instead (every load is then
  // unconditional); their accumulator rows are discarded by the epilogue.
  const uint8_t* afrag[ADIRECT ? FM : 1];
  const uint8_t* asrc[ADIRECT ? 1 : UPT];
  int adst[ADIRECT ? 1 : UPT];
  auto row_ptr = [&](int r) {
    const int pos = pos0 + (r < rows ? r : rows - 1);
    const int64_t arow = p.row_map ? (int64_t)p.row_map[pos] : (int64_t)pos;
    return (const uint8_t*)p.a + arow * lda_bytes;
  };
  if constexpr (ADIRECT) {
#pragma unroll
    for (int i = 0; i < FM; ++i) afrag[i] = row_ptr(i * 16 + lane % 16) + (lane / 16) * 16 * AW;
  } else {
    static_assert(UNITS % kThreads == 0, "LDS A tiles must split evenly over the workgroup");
    // compile-time unit indices keep these arrays in registers
    [&]<int... U>(std::integer_sequence<int, U...>) {
      ((adst[U] = ((tid + U * kThreads) / 4) * ROWB + ((tid + U * kThreads) % 4) * 16,
        asrc[U] = row_ptr((tid + U * kThreads) / 4) + ((tid + U * kThreads) % 4) * 16),
       ...);
    }(std::make_integer_sequence<int, UPT>{});
  }

  // Prefetch ring: slot s holds the weight (and direct A) fragments of one
  // 64-byte K chunk; chunk c+NB-1 is issued before chunk c is consumed, so
  // NB-1 chunks of loads stay in flight per wave. Slots are compile-time
  // indices (the loop body is unrolled), letting the compiler wait only for
  // the slot being consumed.
  //
  // LDS path (three A buffers, chunk c in buffer c % 3): A(c) is loaded to
  // registers in iteration c-3 (two register sets, by chunk parity), stored
  // to its buffer at the start of iteration c-2 and made visible by the
  // barrier that ends iteration c-2. Iteration c reads buffer c % 3 with the
  // fragment reads running two fragments ahead of the MFMAs, and ends by
  // reading the first two fragments of chunk c+1, so the next iteration's
  // MFMAs start right after its barrier.
  constexpr int U = (ADIRECT || NB % 2 == 0) ? NB : 2 * NB;  // unroll: slot and set are constants
  static_assert(ADIRECT || FM >= 3, "the fragment ring runs two fragments ahead");
  v4i bq[NB][FN];
  v4i aq[ADIRECT ? NB : 1][ADIRECT ? FM : 1][AW];
  v4i areg[ADIRECT ? 1 : 2][ADIRECT ? 1 : UPT];
  v4i af[ADIRECT ? 1 : FM];  // LDS fragments of the current chunk

  // Loads are branch-free (a conditional load splits the block and the
  // compiler then drains every outstanding load before the next MFMA). Chunks
  // past the end re-read the last chunk (an L2 hit) and are never consumed.
  auto issue = [&](int64_t c, auto slot_c) {
    constexpr int slot = decltype(slot_c)::value;
    const int64_t cc = c < kc ? c : kc - 1;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      if constexpr (ADIRECT) {
        // Small tiles read each weight byte once: nontemporal loads stream it
        // past the caches (measured ~12% more read bandwidth on MI355X).
        bq[slot][j] = __builtin_nontemporal_load(bptr[j] + cc * kWave);
      } else {
        bq[slot][j] = bptr[j][cc * kWave];
      }
    }
    if constexpr (ADIRECT) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int h = 0; h < AW; ++h) aq[slot][i][h] = *(const v4i*)(afrag[i] + cc * 64 * AW + h * 16);
    }
  };
  auto load_a_regs = [&](int64_t c, auto set_c) {
    if constexpr (!ADIRECT) {
      constexpr int set = decltype(set_c)::value;
      const int64_t cc = c < kc ? c : kc - 1;
      [&]<int... Q>(std::integer_sequence<int, Q...>) {
        ((areg[set][Q] = *(const v4i*)(asrc[Q] + cc * 64)), ...);
      }(std::make_integer_sequence<int, UPT>{});
    }
  };
  auto store_a_lds = [&](int buf, auto set_c) {
    if constexpr (!ADIRECT) {
      constexpr int set = decltype(set_c)::value;
      [&]<int... Q>(std::integer_sequence<int, Q...>) {
        ((*(v4i*)(&sA[buf][adst[Q]]) = areg[set][Q]), ...);
      }(std::make_integer_sequence<int, UPT>{});
    }
  };
  const int frag_off = (wm * FM * 16 + (lane % 16)) * ROWB + (lane / 16) * 16;
  auto read_frag = [&](int buf, int i) -> v4i { return *(const v4i*)(&sA[buf][frag_off + i * 16 * ROWB]); };

  AccT acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = AccT{0, 0, 0, 0};

  auto mfma_row = [&](v4i av, int i, auto slot_c) {
    constexpr int slot = decltype(slot_c)::value;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      if constexpr (I8) {
        acc[i][j] = mfma(av, bq[slot][j], acc[i][j]);
      } else {
        acc[i][j] = mfma(__builtin_bit_cast(v8bf, av), __builtin_bit_cast(v8bf, bq[slot][j]), acc[i][j]);
      }
    }
  };

  // prologue
  [&]<int... S>(std::integer_sequence<int, S...>) {
    (issue(S, std::integral_constant<int, S>{}), ...);
  }(std::make_integer_sequence<int, NB - 1>{});
  if constexpr (!ADIRECT) {
    load_a_regs(0, std::integral_constant<int, 0>{});
    load_a_regs(1, std::integral_constant<int, 1>{});
    store_a_lds(0, std::integral_constant<int, 0>{});
    store_a_lds(1, std::integral_constant<int, 1>{});
    load_a_regs(2, std::integral_constant<int, 0>{});
    lds_barrier();
    af[0] = read_frag(0, 0);
    if constexpr (FM > 1) af[1] = read_frag(0, 1);
  }

  int buf = 0;  // c % 3
  auto body = [&](int64_t c, auto b_c) {
    constexpr int b = decltype(b_c)::value;
    if constexpr (ADIRECT) {
      issue(c + NB - 1, std::integral_constant<int, (b + NB - 1) % NB>{});
      // keep the prefetch ahead of this chunk's MFMAs (the scheduler would
      // otherwise sink the loads below them and drain the ring)
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (W8) {
        // int8 weights -> bf16 once per tile, reused by every row fragment
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          v4i lo, hi;
          i8x16_to_bf16(bq[b % NB][j], lo, hi);
#pragma unroll
          for (int i = 0; i < FM; ++i) {
            acc[i][j] = mfma(__builtin_bit_cast(v8bf, aq[b % NB][i][0]), __builtin_bit_cast(v8bf, lo), acc[i][j]);
            acc[i][j] = mfma(__builtin_bit_cast(v8bf, aq[b % NB][i][1]), __builtin_bit_cast(v8bf, hi), acc[i][j]);
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < FM; ++i) mfma_row(aq[b % NB][i][0], i, std::integral_constant<int, b % NB>{});
      }
      __builtin_amdgcn_sched_barrier(0);
    } else {
      const int buf2 = buf == 0 ? 2 : buf - 1;  // (c + 2) % 3
      const int buf1 = buf == 2 ? 0 : buf + 1;  // (c + 1) % 3
      store_a_lds(buf2, std::integral_constant<int, b % 2>{});
      load_a_regs(c + 3, std::integral_constant<int, (b + 1) % 2>{});
      issue(c + NB - 1, std::integral_constant<int, (b + NB - 1) % NB>{});
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        // fragment i+2 of this chunk, or the first two of the next chunk
        if (i + 2 < FM)
          af[(i + 2) % FM] = read_frag(buf, i + 2);
        else
          af[(i + 2) % FM] = read_frag(buf1, i + 2 - FM);
        mfma_row(af[i], i, std::integral_constant<int, b % NB>{});
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
        __builtin_amdgcn_sched_group_barrier(0x008, FN, 0); // then FN MFMAs
      }
      __builtin_amdgcn_sched_barrier(0);
      lds_barrier();
      buf = buf1;
    }
  };
  int64_t c0 = 0;
  for (; c0 + U <= kc; c0 += U) {
    [&]<int... S>(std::integer_sequence<int, S...>) {
      (body(c0 + S, std::integral_constant<int, S>{}), ...);
    }(std::make_integer_sequence<int, U>{});
  }
  // tail (< U chunks): slots continue from 0
  [&]<int... S>(std::integer_sequence<int, S...>) {
    ((c0 + S < kc ? body(c0 + S, std::integral_constant<int, S>{}) : void()), ...);
  }(std::make_integer_sequence<int, U - 1>{});

  gemm_epilogue<I8, EPI, FM, FN>(p, acc, gtile, tvalid, wm * FM * 16, rows, pos0, expert, lane);
  }
}

template <bool I8, int EPI, int WM, int WN, int FM, int FN, int NB, bool ADIRECT>
__global__ __launch_bounds__(WM * WN * kWave) void grouped_gemm_kernel(GemmParams p, int n_blocks) {
  grouped_gemm_body<I8, EPI, WM, WN, FM, FN, NB, ADIRECT>(p, n_blocks);
}

// Persistent streaming form (16-row tiles beside the persistent LDS-kernel
// launch): at most 80 VGPRs (6 waves per SIMD), so one of its waves fits on
// each SIMD next to two waves of that kernel.
template <bool I8, int EPI, int WM, int WN, int FM, int FN, int NB, bool ADIRECT>
__global__ __launch_bounds__(WM * WN * kWave) __attribute__((amdgpu_waves_per_eu(6))) void
grouped_gemm_stream_kernel(GemmParams p, int n_blocks) {
  grouped_gemm_body<I8, EPI, WM, WN, FM, FN, NB, ADIRECT>(p, n_blocks);
}

template <bool I8, int EPI, int WM, int WN, int FM, int FN, int NB, bool ADIRECT, bool STREAM = false>
int launch_cfg(const GemmParams& p, int64_t max_tiles, hipStream_t stream) {
  constexpr bool PAIR = epi_pair(EPI);
  const int64_t per_block = PAIR ? FN / 2 * WN : FN * WN;
  const int64_t units = PAIR ? p.n_tiles : (int64_t)p.n_groups * p.n_tiles;
  const int64_t n_blocks = ceil_div(units, per_block);
  int64_t grid = max_tiles * n_blocks;
  if (grid <= 0) return FCMOE_OK;
  if (ADIRECT && p.persist > 0 && grid > p.persist) grid = p.persist;
  if (grid > INT32_MAX) return fail(FCMOE_EINVAL, "grouped gemm grid too large");
  if constexpr (STREAM) {
    hipLaunchKernelGGL((grouped_gemm_stream_kernel<I8, EPI, WM, WN, FM, FN, NB, ADIRECT>), dim3((unsigned)grid),
                       dim3(WM * WN * kWave), 0, stream, p, (int)n_blocks);
  } else {
    hipLaunchKernelGGL((grouped_gemm_kernel<I8, EPI, WM, WN, FM, FN, NB, ADIRECT>), dim3((unsigned)grid),
                       dim3(WM * WN * kWave), 0, stream, p, (int)n_blocks);
  }
  return check_launch("grouped_gemm");
}

// Tile bound (the host's upper limit on a launch's tiles) up to which the
// 16-row class runs one-wave workgroups.
constexpr int64_t kDecodeFewTiles = 80;

template <bool I8, int EPI>
int launch_bm(int bm, const GemmParams& p, int64_t max_tiles, hipStream_t stream) {
  switch (bm) {
    case 16:
      // decode: 8 waves per workgroup with an 8-deep ring. W13 pairs one gate
      // and one up tile per wave; W2 (short K) streams one tile per wave.
      // Measured on the DSv3 C2 layer against 4 waves (W13 2+2 tiles with a
      // 4-deep ring, W2 2 tiles): W2 0.527 -> 0.506 ms, W13 0.964 -> 0.961 ms.
      // Small decode batches (a few dozen tiles at most): one wave per
      // workgroup. A CU streams at most ~40 GB/s, so the bytes must spread
      // evenly over all 256 CUs; 8-wave workgroups leave CUs idle at T=1
      // (144 workgroups) or doubled up at T=2 (272 workgroups, W13
      // 0.108 -> 0.083 ms with one-wave workgroups; T=8 0.243 -> 0.233 ms).
      // At C2 (T=64) the 8-wave form is faster (0.929 vs 0.944 ms).
      // W2 (K = 2048: 32 chunks per tile) keeps 11 chunks in flight per wave
      // instead of 7: C2 W2 0.504 -> 0.487 ms, T=8 0.117 -> 0.113 ms, T=1
      // 25.2 -> 24.4 us. W13 gains nothing from it (T=2 0.080 -> 0.086 ms
      // with one-wave workgroups) and keeps the 8-deep ring.
      // The mixed plan's streaming launches (at most 80 VGPRs): the deepest
      // rings that fit, 2 for W13 (2 tiles a wave), 5 for W2 (C3 W2 alone
      // 0.492 -> 0.466 ms against 4, layer 2.78 -> 2.75 ms).
      if (p.stream_role) {
        if constexpr (epi_pair(EPI))
          return launch_cfg<I8, EPI, 1, 4, 1, 2, 2, true, true>(p, max_tiles, stream);
        else
          return launch_cfg<I8, EPI, 1, 4, 1, 1, 5, true, true>(p, max_tiles, stream);
      }
      if (max_tiles <= kDecodeFewTiles) {
        if constexpr (epi_pair(EPI))
          return launch_cfg<I8, EPI, 1, 1, 1, 2, 8, true>(p, max_tiles, stream);
        else
          return launch_cfg<I8, EPI, 1, 1, 1, 1, 12, true>(p, max_tiles, stream);
      }
      if constexpr (epi_pair(EPI))
        return launch_cfg<I8, EPI, 1, 8, 1, 2, 8, true>(p, max_tiles, stream);
      else
        return launch_cfg<I8, EPI, 1, 8, 1, 1, 12, true>(p, max_tiles, stream);
    case 32:
      return launch_cfg<I8, EPI, 1, 4, 2, 4, 4, true>(p, max_tiles, stream);
    case 64:
      return launch_cfg<I8, EPI, 1, 4, 4, 4, 4, false>(p, max_tiles, stream);
    case 128:
      return launch_cfg<I8, EPI, 2, 2, 4, 4, 4, false>(p, max_tiles, stream);
    case 192:
      return launch_cfg<I8, EPI, 2, 2, 6, 4, 2, false>(p, max_tiles, stream);
    case 256:
      return launch_cfg<I8, EPI, 2, 2, 8, 4, 2, false>(p, max_tiles, stream);
    default:
      return fail(FCMOE_EINVAL, "unsupported tile rows");
  }
}

// W8A16 on the direct-A kernel: tiles of 16 or 32 rows (decode and the
// small prefill classes; 128 and 256 rows run on the LDS-staged kernel).
template <int EPI>
int launch_bm_w8(int bm, const GemmParams& p, int64_t max_tiles, hipStream_t stream) {
  switch (bm) {
    case 16:
      // W13 runs 8 waves of one gate+up pair with a 6-deep ring (C1 shape:
      // 0.754 -> 0.747 ms against 4 waves of 2+2 tiles; ring depth 4 / 6 / 8:
      // 0.707 / 0.699 / 0.714 ms on a later box). W2 keeps 4 waves of 2
      // tiles: the int8 -> bf16 widening makes the one-tile-per-wave form
      // slower (0.404 vs 0.445 ms); a 12-deep ring against 8: 0.385 vs 0.396.
      if constexpr (epi_pair(EPI))
        return launch_cfg<false, EPI, 1, 8, 1, 2, 6, true>(p, max_tiles, stream);
      else
        return launch_cfg<false, EPI, 1, 4, 1, 2, 12, true>(p, max_tiles, stream);
    case 32:
      return launch_cfg<false, EPI, 1, 4, 2, 4, 4, true>(p, max_tiles, stream);
    default:
      return fail(FCMOE_EINVAL, "W8A16 tiles are 16 or 32 rows");
  }
}

}  // namespace

int gemm_launch(int epi, int bm, const GemmParams& p, int64_t max_tiles, hipStream_t stream) {
  static const bool use_lds = [] {
    const char* v = getenv("FCMOE_GEMM_LDS");
    return !(v && v[0] == '0');
  }();
  // The LDS-staged kernel addresses A and one expert's weights through
  // buffer resources with 32-bit offsets: 2 GiB or more of either runs on
  // the register-ring kernel (64-bit addresses). W8A16 has no register-ring tile above 32 rows; its forward
  // keeps to the 16/32-row classes for such an A.
  const bool a_int8 = epi == kEpiRawI32 || epi == kEpiW13SwigluI8 || epi == kEpiW2RouteI8 || epi == kEpiI8Gemm;
  const bool a_fits = (p.a_rows <= 0 || p.a_rows * p.lda * (a_int8 ? 1 : 2) < kLdsMaxABytes) &&
                      p.w_expert_bytes < kLdsMaxABytes;  // one expert's weights: one buffer resource too
  if (bm >= 128 && epi_w8(epi) && !a_fits)
    return fail(FCMOE_EINVAL, "W8A16 LDS tiles need A and each expert's weights under 2 GiB");
  if (bm >= 128 && a_fits && (use_lds || epi_w8(epi))) return gemm_lds_launch(epi, bm, p, max_tiles, stream);
  if (epi == kEpiW13ActW8) return launch_bm_w8<kEpiW13ActW8>(bm, p, max_tiles, stream);
  if (epi == kEpiW2RouteW8) return launch_bm_w8<kEpiW2RouteW8>(bm, p, max_tiles, stream);
  switch (epi) {
    case kEpiRawI32:
      return launch_bm<true, kEpiRawI32>(bm, p, max_tiles, stream);
    case kEpiW13SwigluI8:
      return launch_bm<true, kEpiW13SwigluI8>(bm, p, max_tiles, stream);
    case kEpiW2RouteI8:
      return launch_bm<true, kEpiW2RouteI8>(bm, p, max_tiles, stream);
    case kEpiI8Gemm:
      return launch_bm<true, kEpiI8Gemm>(bm, p, max_tiles, stream);
    case kEpiW13ActBf16:
      return launch_bm<false, kEpiW13ActBf16>(bm, p, max_tiles, stream);
    case kEpiRawF32Bias:
      return launch_bm<false, kEpiRawF32Bias>(bm, p, max_tiles, stream);
    case kEpiW2RouteBf16:
      return launch_bm<false, kEpiW2RouteBf16>(bm, p, max_tiles, stream);
    default:
      return fail(FCMOE_EINVAL, "unknown epilogue");
  }
}

}  // namespace fcmoe
