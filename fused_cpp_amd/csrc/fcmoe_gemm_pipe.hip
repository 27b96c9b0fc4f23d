// fcmoe_gemm_pipe.hip -- the persistent 256 x 256 int8 grouped GEMM of the
// W8A8 prefill plans, one wave per SIMD.
//
// The LDS-staged kernel (fcmoe_gemm_lds.hip) runs 2 waves per SIMD of
// 128 x 64 wave tiles with accumulators in VGPRs, and starts every K chunk
// with a barrier and a burst of fragment reads that all 8 waves wait out
// before their first MFMA: its K loop ran at ~45% of the MFMA pipe.
// Here each SIMD runs one wave of a 128 x 128 tile (2 x 2 waves, the same
// 256-row x 256-channel workgroup tile and item space):
//   * the 256 int32 accumulators per lane live in AGPRs (this file is built
//     without the VGPR-form flag the other GEMMs use), the fragments in
//     VGPRs;
//   * per 64-byte K chunk a wave reads 8 A and 8 B fragments (64 KB per
//     workgroup against 96 KB for 8 waves of 128 x 64) for 64 MFMAs;
//   * fragments are double-buffered in registers: while the MFMAs of chunk c
//     run, the wave reads chunk c+1's fragments, so no chunk starts on an
//     LDS round trip, and the chunk's stage loads (buffer_load ... lds, one
//     per row of MFMAs) are spread through it;
//   * a 4-stage LDS ring keeps 3 chunks of loads in flight behind the one
//     being read (~3 chunk times of latency cover for weights coming from
//     HBM).
// One wave's 256 AGPRs + at most 160 VGPRs leave room on every SIMD for the
// 16-row streaming launch's wave (80 VGPRs) that the mixed plan runs beside
// it. The arithmetic (exact int32 sums, the staged epilogues) is the
// LDS-staged kernel's, so results are bit-identical.
#include "fcmoe_gemm_lds_common.h"

namespace fcmoe {

namespace {

constexpr int kPipeWM = 2;    // wave rows
constexpr int kPipeWN = 2;    // wave columns
constexpr int kPipeFM = 8;    // 16-row fragments per wave
constexpr int kPipeFN = 6;    // 16-channel tiles per wave
constexpr int kPipeStages = 4;
constexpr int kPipeWaves = kPipeWM * kPipeWN;
constexpr int kPipeThreads = kPipeWaves * kWave;
constexpr int kPipeBM = kPipeWM * kPipeFM * 16;   // 256 rows
constexpr int kPipeNT = kPipeWN * kPipeFN;        // 16 channel tiles
constexpr int kPipeABytes = kPipeBM * 64;         // A rows of one chunk: 16 KB
constexpr int kPipeBBytes = kPipeNT * 1024;       // weight tiles of one chunk: 16 KB
constexpr int kPipeStageBytes = kPipeABytes + kPipeBBytes;
// Per-wave LDS areas of the epilogue: the staged rows (staged_epilogue's
// slices, from 0) and the fragment accumulators on their way out of the
// AGPRs (from kAccStageBase).
constexpr int kAccStageBase = 32 * 1024;
constexpr int kPipeLA = kPipeABytes / 1024 / kPipeWaves;  // A loads per wave and chunk (4)
constexpr int kPipeLB = kPipeNT / kPipeWaves;             // B loads per wave and chunk (4)
constexpr int kPipeLoads = kPipeLA + kPipeLB;             // 8: one per row of MFMAs
static_assert(kPipeLoads <= kPipeFM, "at most one stage load per row of MFMAs");

struct PipeFrags {
  v4i a[kPipeFM];
  v4i b[kPipeFN];
};

template <int EPI>
__global__ __launch_bounds__(kPipeThreads) void grouped_gemm_pipe_kernel(GemmParams p, int n_blocks, int partial,
                                                                        int gm, int grid_items) {
#if __HIP_DEVICE_COMPILE__
  constexpr int FM = kPipeFM, FN = kPipeFN, WNW = kPipeWN;
  constexpr bool PAIR = epi_pair(EPI);
  constexpr int HP = FN / 2;
  static_assert(EPI == kEpiW13SwigluI8 || EPI == kEpiW2RouteI8, "W8A8 stage epilogues only");

  // One LDS object (a second one costs the K loop a vmcnt(0) per chunk): the
  // stage ring, then the epilogue metadata and the work-queue slot.
  constexpr int META = kPipeStages * kPipeStageBytes;
  constexpr int BM = kPipeBM, NT = kPipeNT;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[META + 8 * BM + 64 * NT + 16];
  static_assert(META + 8 * BM + 64 * NT + 16 <= 160 * 1024, "LDS budget");
  static_assert(kPipeWaves * staged_slice_bytes<FN>(EPI) <= kAccStageBase, "staging slices fit below the acc areas");
  static_assert(kAccStageBase + kPipeWaves * FN * 1024 <= META, "acc areas fit the stages");
  float* const meta_rs = (float*)(smem + META);
  int* const meta_orow = (int*)(smem + META + 4 * BM);
  float* const meta_cs = (float*)(smem + META + 8 * BM);
  int* const next_k = (int*)(smem + META + 8 * BM + 64 * NT);

  bool part = false;
  if (!plan_open(p)) {
    if (!p.part_counts || (int)blockIdx.x >= part_wgs(p.part_counts)) return;
    part = true;
  }
  if (part && gm == kLdsDealTiles) gm = kLdsGroupTiles;  // the partitioned plan keeps XCD windows
  const int32_t* const tiles0 = part ? p.part_tiles : p.tiles;
  int32_t* const queue = part ? p.part_queue : p.queue;
  const int u_n = part ? 0 : p.u_n;
  int ucount[3] = {0, 0, 0};
  int count = 0;
  for (int u = 0; u < u_n; ++u) {
    ucount[u] = *p.u_count[u];
    count += ucount[u];
  }
  if (u_n == 0) count = part ? p.part_counts[3] : *p.tile_count;

  const int xcd = (int)blockIdx.x % kXcds;
  int xcd_items;
  {
    const int nbf = partial ? n_blocks - 1 : n_blocks;
    const int F = count * nbf, P = partial ? count : 0;
    xcd_items = F / kXcds + (xcd < F % kXcds ? 1 : 0) + P / kXcds + (xcd < P % kXcds ? 1 : 0);
    if (gm == kLdsDealTiles) xcd_items = deal_tiles(count, xcd) * (nbf + (partial ? 1 : 0));
    if (gm <= 0) xcd_items = grid_items;
  }
  auto fetch_k = [&](int k_static) -> int {
    if (!queue) return k_static;
    __syncthreads();
    if (threadIdx.x == 0) *next_k = __hip_atomic_fetch_add(queue + xcd, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    return *next_k;
  };

  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int wm = wave / WNW;
  const int wn = wave % WNW;
  const int64_t kc = p.k_chunks;
  const int64_t total_tiles = (int64_t)p.n_groups * p.n_tiles;
  const int64_t lda_bytes = p.lda;
  const uint32_t voff_lane = (uint32_t)lane * 16;
  // fragment offsets within a stage: A row wm*128 + 16 i + lane%16, 16-byte
  // unit lane/16 at slot unit ^ ((row >> 2) & 3); B tile wn*8 + j, lane's 16 bytes
  const int a_frag = (wm * FM * 16 + lane % 16) * 64 + (((lane / 16) ^ ((lane % 16) >> 2)) * 16);
  const int b_frag = kPipeABytes + wn * FN * 1024 + lane * 16;

  int k = fetch_k((int)blockIdx.x / kXcds);
  for (int it = 0, slot = 0; k < xcd_items; ++it) {
    slot = gm <= 0 ? (int)blockIdx.x + it * (int)gridDim.x : k * kXcds + xcd;
    int tile_idx, nb;
    const bool have = lds_work_item(slot, count, n_blocks, partial != 0, gm, tile_idx, nb);
    k = fetch_k(k + (int)gridDim.x / kXcds);
    if (gm <= 0) k = slot + (int)gridDim.x < grid_items ? 0 : xcd_items;
    if (!have) continue;
    if (it > 0) __syncthreads();  // the previous item's epilogue is done with the stages

    const int32_t* tpair = tiles0 + 2 * (count - 1 - tile_idx);
    if (u_n > 0) {
      int t = tile_idx, u = 0;
      while (u + 1 < u_n && t >= ucount[u]) t -= ucount[u++];
      tpair = p.u_tiles[u] + 2 * (ucount[u] - 1 - t);
    }
    const int expert = tpair[0];
    const int m0 = tpair[1];
    const int rows_left = p.counts[expert] - m0;
    const int rows = rows_left < BM ? rows_left : BM;
    const int pos0 = p.offsets[expert] + m0;

    auto tile_of = [&](int wn_, int j, bool* valid) -> int64_t {
      if constexpr (PAIR) {
        const int64_t pr = ((int64_t)nb * WNW + wn_) * HP + (j % HP);
        *valid = pr < p.n_tiles;
        return (j < HP ? 0 : p.n_tiles) + pr;
      } else {
        const int64_t t = ((int64_t)nb * WNW + wn_) * FN + j;
        *valid = t < total_tiles;
        return t;
      }
    };

    // Stage loads of this wave: A loads g = wave + 4u (16 rows x 64 bytes
    // each), B loads t = wave + 4u (one 1 KB tile chunk each).
    const __amdgpu_buffer_rsrc_t rsrc_a =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.a), (short)0, 0x7ffffff0, kBufWord3);
    const __amdgpu_buffer_rsrc_t rsrc_b = __builtin_amdgcn_make_buffer_rsrc(
        (void*)((const uint8_t*)p.w + (int64_t)expert * p.w_expert_bytes), (short)0,
        (int)(p.w_expert_bytes < 0x7ffffff0 ? p.w_expert_bytes : 0x7ffffff0), kBufWord3);
    uint32_t voff_a[kPipeLA];
    int soff_b[kPipeLB];
#pragma unroll
    for (int u = 0; u < kPipeLA; ++u) {
      const int g = wave + kPipeWaves * u;
      const int r = g * 16 + lane / 4;
      const int unit = (lane % 4) ^ ((lane >> 4) & 3);  // == unit ^ ((r >> 2) & 3)
      const int pos = pos0 + (r < rows ? r : rows - 1);  // rows past the tile re-read the last row
      const int64_t arow = p.row_map ? (int64_t)p.row_map[pos] : (int64_t)pos;
      voff_a[u] = (uint32_t)(arow * lda_bytes + unit * 16);
    }
#pragma unroll
    for (int u = 0; u < kPipeLB; ++u) {
      const int t = wave + kPipeWaves * u;
      bool valid;
      const int64_t gt = tile_of(t / FN, t % FN, &valid);
      soff_b[u] = __builtin_amdgcn_readfirstlane((int)((valid ? gt : 0) * kc * 1024));
    }
    // load u (0..7) of chunk c into stage s: A loads first, then B
    auto issue_one = [&](int u, int64_t c, int s) {
      const int64_t cc = c < kc ? c : kc - 1;  // past the end: re-load the last chunk (never read)
      if (u < kPipeLA) {
        const int g = wave + kPipeWaves * u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_a, (lds_ptr_t)(smem + s * kPipeStageBytes + g * 1024), 16,
                                                 voff_a[u], (int)(cc * 64), 0, 0);
      } else {
        const int t = wave + kPipeWaves * (u - kPipeLA);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rsrc_b, (lds_ptr_t)(smem + s * kPipeStageBytes + kPipeABytes + t * 1024), 16, voff_lane,
            soff_b[u - kPipeLA] + (int)(cc * 1024), 0, 0);
      }
    };

    bool wave_live = wm * FM * 16 < rows;
    {
      bool any = false;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        bool v;
        (void)tile_of(wn, j, &v);
        any = any || v;
      }
      wave_live = wave_live && any;
    }
    // row fragments of this wave that hold rows of the expert (0: the wave skips its MFMAs)
    const int live_frags = __builtin_amdgcn_readfirstlane(wave_live ? (rows - wm * FM * 16 + 15) / 16 : 0);

    v4i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    // epilogue metadata, phase 1 (as the LDS-staged kernel)
    constexpr bool ROUTE = epi_route(EPI);
    const int mt = threadIdx.x;
    int m_row = 0, m_orow = 0;
    float m_rs = 0.0f;
    float m_cs = 0.0f;
    {
      const int pos = pos0 + (mt < rows ? mt : rows - 1);
      if constexpr (EPI == kEpiW13SwigluI8) m_row = p.row_map ? p.row_map[pos] : pos;
      if constexpr (EPI == kEpiW2RouteI8) m_rs = p.scale_row[pos];
      m_orow = ROUTE ? p.sorted_routes[pos] : pos;
    }
    static_assert(NT * 16 <= kPipeThreads && BM == kPipeThreads, "one metadata value per thread");
    if (mt < NT * 16) {
      bool valid;
      const int64_t gt = tile_of(mt / 16 / FN, (mt / 16) % FN, &valid);
      const int64_t g = gt / p.n_tiles;
      const int64_t cin = (gt - g * p.n_tiles) * 16 + mt % 16;
      if (valid && cin < p.n_half) m_cs = p.scale_col[(int64_t)expert * p.n + g * p.n_half + cin];
    }

    // prologue: chunks 0..3 in flight
#pragma unroll
    for (int s = 0; s < kPipeStages; ++s)
#pragma unroll
      for (int u = 0; u < kPipeLoads; ++u) issue_one(u, s, s);
    // epilogue metadata, phase 2
    if constexpr (EPI == kEpiW13SwigluI8) m_rs = p.scale_row[m_row];
    meta_rs[mt] = m_rs;
    meta_orow[mt] = m_orow;
    if (mt < NT * 16) meta_cs[mt] = m_cs;
    __builtin_amdgcn_s_waitcnt(0xC07F);  // retire the set-up's scalar and LDS ops (lgkmcnt(0))

    PipeFrags f0, f1;
    auto read_frags = [&](PipeFrags& f, int s) {
      const uint8_t* st = smem + s * kPipeStageBytes;
#pragma unroll
      for (int i = 0; i < FM; ++i) f.a[i] = *(const v4i*)(st + a_frag + i * 1024);
#pragma unroll
      for (int j = 0; j < FN; ++j) f.b[j] = *(const v4i*)(st + b_frag + j * 1024);
    };
    // One chunk: the MFMAs of chunk c (fragments `cur`), with chunk c+1's
    // fragment reads (into `nxt`) and chunk c+4's stage loads spread over its
    // rows. On entry this wave's chunk c+1 and c+2 loads may be in flight.
    auto step = [&](int64_t c, const PipeFrags& cur, PipeFrags& nxt) {
      // this wave's reads of chunk c (into cur) have completed and its chunk
      // c+1 loads have landed; after the barrier so have every wave's, and no
      // wave reads chunk c's stage any more
      __builtin_amdgcn_s_waitcnt(0xC07F);
      wait_vmcnt<2 * kPipeLoads>();
      __builtin_amdgcn_s_barrier();
      const int s_next = (int)((c + 1) % kPipeStages);
      const int s_free = (int)(c % kPipeStages);
      const uint8_t* st = smem + s_next * kPipeStageBytes;
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        nxt.a[i] = *(const v4i*)(st + a_frag + i * 1024);
        if (i < FN) nxt.b[i] = *(const v4i*)(st + b_frag + i * 1024);
        if (i < kPipeLoads) issue_one(i, c + kPipeStages, s_free);
        if (i < live_frags) {
#pragma unroll
          for (int j = 0; j < FN; ++j) acc[i][j] = mfma(cur.a[i], cur.b[j], acc[i][j]);
        }
        if (i < FN)
          __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // the fragment reads
        else
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        if (i < kPipeLoads) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // the stage load
        __builtin_amdgcn_sched_group_barrier(0x008, FN, 0);  // row i's MFMAs
      }
      __builtin_amdgcn_sched_barrier(0);
    };

    wait_vmcnt<(kPipeStages - 1) * kPipeLoads>();  // chunk 0 has landed
    __builtin_amdgcn_s_barrier();
    read_frags(f0, 0);
    // chunk pairs, then an odd last chunk (a conditional second step inside
    // the loop makes the compiler shuffle the accumulators between AGPRs)
    int64_t c = 0;
    for (; c + 1 < kc; c += 2) {
      step(c, f0, f1);
      step(c + 1, f1, f0);
    }
    if (c < kc) step(c, f0, f1);
    wait_vmcnt<0>();  // the trailing (unused) stage loads
    __builtin_amdgcn_s_waitcnt(0xC07F);
    // The epilogue reads the accumulators with an asm ds_write, which the
    // compiler's hazard tracking does not see: wait states after the last
    // MFMA's writes (more than the 18 a 16-pass MFMA needs).
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
    // the accumulators stay in AGPRs until the epilogue moves them out a
    // fragment at a time
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) asm volatile("" : "+a"(acc[i][j]));

    int64_t gtile[FN];
    bool tvalid[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) gtile[j] = tile_of(wn, j, &tvalid[j]);
    const EpiMeta meta{(lds_cfloat_ptr)meta_rs, (lds_cint_ptr)meta_orow, (lds_cfloat_ptr)meta_cs, wn * FN};
    __builtin_amdgcn_s_barrier();  // every wave is past its last fragment reads: the stages are free
    staged_epilogue<EPI, FM, FN, true>(p, acc, gtile, tvalid, wm * FM * 16, rows, pos0, expert, lane, meta,
                                 (lds_u8_ptr)(smem + wave * staged_slice_bytes<FN>(EPI)),
                                 (lds_u8_ptr)(smem + kAccStageBase + wave * FN * 1024));
  }
#endif
}

template <int EPI>
int launch_pipe(const GemmParams& p, int64_t max_tiles, hipStream_t stream) {
  const int64_t n_blocks = lds_blocks<EPI>(kPipeWN, kPipeFN, p);
  if (max_tiles * n_blocks <= 0) return FCMOE_OK;
  constexpr bool PAIR = epi_pair(EPI);
  const int64_t units = PAIR ? p.n_tiles : (int64_t)p.n_groups * p.n_tiles;
  const int partial = n_blocks * (PAIR ? kPipeWN * (kPipeFN / 2) : kPipeWN * kPipeFN) > units ? 1 : 0;
  const int64_t items = max_tiles * n_blocks + (partial ? kXcds : 0);
  if (items > INT32_MAX) return fail(FCMOE_EINVAL, "grouped gemm grid too large");
  if (p.persist <= 0) return fail(FCMOE_EINVAL, "the pipelined GEMM is persistent only");
  if (p.w_expert_bytes >= 0x7ffffff0) return fail(FCMOE_EINVAL, "expert weights exceed 2 GiB");
  if (p.lda % 64) return fail(FCMOE_EINVAL, "pipelined GEMM: A rows must be 64-byte aligned");
  const int64_t grid = items > p.persist ? p.persist : items;
  const int gm = p.u_n > 0 ? kLdsDealTiles : kLdsGroupTiles;
  hipLaunchKernelGGL(grouped_gemm_pipe_kernel<EPI>, dim3((unsigned)grid), dim3(kPipeThreads), 0, stream, p,
                     (int)n_blocks, partial, gm, (int)items);
  return check_launch("grouped_gemm_pipe");
}

}  // namespace

int gemm_pipe_launch(int epi, const GemmParams& p, int64_t max_tiles, hipStream_t stream) {
  switch (epi) {
    case kEpiW13SwigluI8:
      return launch_pipe<kEpiW13SwigluI8>(p, max_tiles, stream);
    case kEpiW2RouteI8:
      return launch_pipe<kEpiW2RouteI8>(p, max_tiles, stream);
    default:
      return fail(FCMOE_EINVAL, "pipelined GEMM: W8A8 W13 / W2 epilogues only");
  }
}

}  // namespace fcmoe
